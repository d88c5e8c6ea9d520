"""CPU oracle for the W4A16 dense-FFN decode path - TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import this
module, and only as the checker (or, for the baseline, as the thing timed on the host). The
product path never imports it.

* ``liboracle.so`` (w4a16_oracle.c): the format arithmetic and a double-accumulated
  dequant-then-matmul FFN with the reference's BF16 rounding points.
* numpy helpers restating the reference test's independent dequantizer
  (reference tests/test_quantization_kernel.py:60-78) and the CPU baseline.
* ``oracle/_ref``: the reference's own CPU sources compiled here (when built), used to pin the
  restatement.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")
GROUP = 128

_vp = ctypes.c_void_p
_ll = ctypes.c_longlong


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built (make -C oracle)")
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "orc_last_error": (ctypes.c_char_p, []),
        "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_layout_check": (ctypes.c_int, [_ll, _ll, _ll]),
        "orc_packed_code": (ctypes.c_int, [_vp, _ll, _ll, _ll]),
        "orc_quantize_int4": (ctypes.c_int, [_ll, _ll, _vp, _vp, _vp]),
        "orc_dequantize_int4": (ctypes.c_int, [_ll, _ll, _vp, _vp, _vp]),
        "orc_gemm_f64": (ctypes.c_int, [_ll, _ll, _ll, _vp, _vp, _vp, _vp]),
        "orc_gemm_bf16": (ctypes.c_int, [_ll, _ll, _ll, _vp, _vp, _vp, _vp]),
        "orc_silu_mul_packed": (ctypes.c_int, [_ll, _ll, _vp, _vp]),
        "orc_ffn_bf16": (ctypes.c_int, [_ll, _ll, _ll, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
        "orc_ffn_partial_f32": (ctypes.c_int, [_ll, _ll, _ll, _vp, _vp, _vp, _vp, _vp, _vp]),
        "orc_rmsnorm_bf16": (ctypes.c_int, [_ll, _ll, _vp, _vp, ctypes.c_int, ctypes.c_double, _vp]),
        "orc_rmsnorm_f32order_bf16": (ctypes.c_int, [_ll, _ll, _vp, _vp, ctypes.c_int, ctypes.c_float,
                                                     _vp, _vp]),
        "orc_residual_norm_bf16": (ctypes.c_int, [_ll, _ll, _vp, _vp, _vp, ctypes.c_int,
                                                  ctypes.c_double, _vp]),
        "orc_residual_add_bf16": (ctypes.c_int, [_ll, _vp, _vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class OracleError(RuntimeError):
    pass


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a):
    return a.ctypes.data if a is not None else None


def _ok(status, what):
    if status != 0:
        raise OracleError(f"{what}: {lib.orc_last_error().decode()} (status {status})")


# ---- BF16 (numpy, vectorised; same rule as orc_f32_to_bf16) ------------------------------------

def bf16_bits(values):
    """FP32 -> BF16 bits, round-to-nearest-even (reference csrc/linear_weight.cpp:34-44)."""
    u = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- format (C oracle) ---------------------------------------------------------------------------

def layout_check(n, k, group=GROUP):
    return lib.orc_layout_check(n, k, group)


def quantize(weights):
    w = _c(weights, np.float32)
    n, k = w.shape
    packed = np.zeros((n, k // 2), np.uint8)
    scales = np.zeros((n, k // GROUP), np.uint16)
    _ok(lib.orc_quantize_int4(n, k, _p(w), _p(packed), _p(scales)), "quantize")
    return packed, scales


def dequantize(packed, scales, n, k):
    out = np.zeros((n, k), np.float32)
    p, s = _c(packed, np.uint8), _c(scales, np.uint16)
    _ok(lib.orc_dequantize_int4(n, k, _p(p), _p(s), _p(out)), "dequantize")
    return out


def packed_code(packed, row, k, k_extent):
    return lib.orc_packed_code(_p(_c(packed, np.uint8)), row, k, k_extent)


def gemm_f64(x_bits, packed, scales, n, k):
    x = _c(x_bits, np.uint16).reshape(-1, k)
    out = np.zeros((x.shape[0], n), np.float64)
    _ok(lib.orc_gemm_f64(x.shape[0], n, k, _p(x), _p(_c(packed, np.uint8)),
                         _p(_c(scales, np.uint16)), _p(out)), "gemm_f64")
    return out


def gemm_bf16(x_bits, packed, scales, n, k):
    x = _c(x_bits, np.uint16).reshape(-1, k)
    out = np.zeros((x.shape[0], n), np.uint16)
    _ok(lib.orc_gemm_bf16(x.shape[0], n, k, _p(x), _p(_c(packed, np.uint8)),
                          _p(_c(scales, np.uint16)), _p(out)), "gemm_bf16")
    return out


def silu_mul_packed(packed_bits, tokens, inter):
    p = _c(packed_bits, np.uint16)
    out = np.zeros((tokens, inter), np.uint16)
    _ok(lib.orc_silu_mul_packed(tokens, inter, _p(p), _p(out)), "silu_mul_packed")
    return out


def ffn_bf16(x_bits, gu_packed, gu_scales, dn_packed, dn_scales, hidden, inter):
    """Returns (out [M,H], mid [M,2I], act [M,I]) as BF16 bits."""
    x = _c(x_bits, np.uint16).reshape(-1, hidden)
    m = x.shape[0]
    out = np.zeros((m, hidden), np.uint16)
    mid = np.zeros((m, 2 * inter), np.uint16)
    act = np.zeros((m, inter), np.uint16)
    _ok(lib.orc_ffn_bf16(m, hidden, inter, _p(x), _p(_c(gu_packed, np.uint8)),
                         _p(_c(gu_scales, np.uint16)), _p(_c(dn_packed, np.uint8)),
                         _p(_c(dn_scales, np.uint16)), _p(out), _p(mid), _p(act)), "ffn_bf16")
    return out, mid, act


def ffn_partial_f32(x_bits, gu_packed, gu_scales, dn_packed, dn_scales, hidden, inter):
    x = _c(x_bits, np.uint16).reshape(-1, hidden)
    m = x.shape[0]
    out = np.zeros((m, hidden), np.float32)
    _ok(lib.orc_ffn_partial_f32(m, hidden, inter, _p(x), _p(_c(gu_packed, np.uint8)),
                                _p(_c(gu_scales, np.uint16)), _p(_c(dn_packed, np.uint8)),
                                _p(_c(dn_scales, np.uint16)), _p(out)), "ffn_partial_f32")
    return out


def rmsnorm_bf16(x_bits, w_bits, norm_style, eps):
    """BF16 bits [rows, cols]: x * rsqrt(mean(x^2) + eps) * (bias + w), bias 1 for norm_style 0
    (Gemma) and 0 for 1 (plain)."""
    x = _c(x_bits, np.uint16)
    rows, cols = (1, x.shape[0]) if x.ndim == 1 else x.shape
    out = np.zeros((rows, cols), np.uint16)
    _ok(lib.orc_rmsnorm_bf16(rows, cols, _p(x), _p(_c(w_bits, np.uint16)), norm_style, eps,
                             _p(out)), "rmsnorm_bf16")
    return out


def rmsnorm_f32order_bf16(x_bits, w_bits, norm_style, eps):
    """The reference's in-tree FP32 order (residual_norm_kernel): returns (out bits [rows, cols],
    per-row FP32 scales)."""
    x = _c(x_bits, np.uint16)
    rows, cols = (1, x.shape[0]) if x.ndim == 1 else x.shape
    out = np.zeros((rows, cols), np.uint16)
    rms = np.zeros(rows, np.float32)
    _ok(lib.orc_rmsnorm_f32order_bf16(rows, cols, _p(x), _p(_c(w_bits, np.uint16)), norm_style,
                                      eps, _p(out), _p(rms)), "rmsnorm_f32order_bf16")
    return out, rms


def residual_norm_bf16(residual_bits, sub_bits, w_bits, norm_style, eps):
    """Returns (updated residual, normed) as BF16 bits [rows, cols]; the input is not modified."""
    r = np.array(_c(residual_bits, np.uint16), copy=True)
    r = r.reshape(1, -1) if r.ndim == 1 else r
    rows, cols = r.shape
    out = np.zeros((rows, cols), np.uint16)
    _ok(lib.orc_residual_norm_bf16(rows, cols, _p(r), _p(_c(sub_bits, np.uint16)),
                                   _p(_c(w_bits, np.uint16)), norm_style, eps, _p(out)),
        "residual_norm_bf16")
    return r, out


def residual_add_bf16(dst_bits, src_bits):
    d = np.array(_c(dst_bits, np.uint16), copy=True)
    _ok(lib.orc_residual_add_bf16(d.size, _p(d), _p(_c(src_bits, np.uint16))), "residual_add_bf16")
    return d


def lib_rmsnorm_raw(cols, eps, norm_style, rows=1):
    """The refusal path only: call with placeholder buffers."""
    x = np.zeros(max(cols, 1) * max(rows, 1), np.uint16)
    out = np.zeros_like(x)
    _ok(lib.orc_rmsnorm_bf16(rows, cols, _p(x), _p(x), norm_style, eps, _p(out)), "rmsnorm_bf16")


# ---- numpy restatement of the reference test's dequantizer and the CPU baseline ------------------

def dequantize_numpy(packed, scales, n, k):
    """w = code * f32(scale), vectorised (reference tests/test_quantization_kernel.py:60-70)."""
    p = np.asarray(packed, dtype=np.uint8).reshape(n, k // 2)
    lo = (p & 0x0F).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    codes = np.empty((n, k), dtype=np.float32)
    codes[:, 0::2] = np.where(lo >= 8, lo - 16, lo)
    codes[:, 1::2] = np.where(hi >= 8, hi - 16, hi)
    s = bf16_to_f32(np.asarray(scales, dtype=np.uint16).reshape(n, k // GROUP))
    codes *= np.repeat(s, GROUP, axis=1)
    return codes


def ffn_cpu_baseline(x_bits, gu_packed, gu_scales, dn_packed, dn_scales, hidden, inter):
    """The CPU path timed as the baseline: dequantize per call, FP32 matmul (BLAS), BF16 at
    the reference's rounding points (reference csrc/kernels/layers.cu:126-145)."""
    x = bf16_to_f32(x_bits).reshape(-1, hidden)
    wgu = dequantize_numpy(gu_packed, gu_scales, 2 * inter, hidden)
    mid = bf16_to_f32(bf16_bits(x @ wgu.T))
    g, u = mid[:, :inter].astype(np.float64), mid[:, inter:].astype(np.float64)
    act = bf16_to_f32(bf16_bits((g / (1.0 + np.exp(-g)) * u).astype(np.float32)))
    wdn = dequantize_numpy(dn_packed, dn_scales, hidden, inter)
    return bf16_bits(act @ wdn.T)


def ffn_cpu_matmul_only(x_bits, wgu, wdn, hidden, inter):
    """CPU baseline variant (ii): the same FFN on weights dequantized once beforehand (FP32 [2I, H]
    and [H, I]), so only the two matmuls and the SiLU run per call."""
    x = bf16_to_f32(x_bits).reshape(-1, hidden)
    mid = bf16_to_f32(bf16_bits(x @ wgu.T))
    g, u = mid[:, :inter].astype(np.float64), mid[:, inter:].astype(np.float64)
    act = bf16_to_f32(bf16_bits((g / (1.0 + np.exp(-g)) * u).astype(np.float32)))
    return bf16_bits(act @ wdn.T)


# ---- synthetic inputs ----------------------------------------------------------------------------

def synth_weight(n, k, seed, std=0.02):
    """BF16 ~N(0, std) weights widened to FP32, from numpy's PCG64 (seeded)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return bf16_to_f32(bf16_bits(rng.normal(0.0, std, size=(n, k)).astype(np.float32)))


def synth_activation(m, k, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    return bf16_bits(rng.normal(0.0, 1.0, size=(m, k)).astype(np.float32))


def ref_binary(name):
    path = os.path.join(REF_DIR, name)
    return path if os.path.exists(path) else None
