"""Host-side binding of libw4a16.so, the MI355X W4A16 dense-FFN decode library.

This module mirrors the reference's operator interface for the path:

* ``gemm_int4_bf16(a, packed, scales, out, M, N, K, group, stream)`` - reference
  csrc/include/layers.h:376-377 (C++, throws) -> here a status-returning C entry point; the Python
  wrapper raises ``W4A16Error`` where the reference throws ``std::invalid_argument``.
* ``kernel_silu_mul_packed(out, packed, tokens, intermediate)`` - reference
  csrc/kernels/silu.cu:78-95.
* ``mlp_int4`` - the INT4 branch of ``mlp_from_normed`` (reference csrc/kernels/layers.cu:126-145).
* ``test_gemm_int4`` - the reference bridge symbol (tests/kernels/kernel_bridge.cu:83-95).

Device tensors are torch CUDA tensors (on ROCm, HIP memory); torch is used only for device memory
and streams. There is no CPU fallback: if the library is missing the import fails.
"""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libw4a16.so")

GROUP = 128
TILE_ROWS = 8

W4A16_OK = 0
W4A16_ERR_HIP = -1
W4A16_ERR_ALLOC = -2
W4A16_ERR_WEIGHTS = -3
W4A16_ERR_CONFIG = -4
W4A16_ERR_STATE = -5


class W4A16Error(RuntimeError):
    """A nonzero status from the library, with its thread-local reason."""

    def __init__(self, status, message):
        super().__init__(f"{message} (status {status})")
        self.status = status


_vp = ctypes.c_void_p
_ll = ctypes.c_longlong
_i = ctypes.c_int

# name -> (restype, argtypes)
_SIGNATURES = {
    "w4a16_last_error": (ctypes.c_char_p, []),
    "w4a16_layout_init": (_i, [_ll, _ll, _ll, ctypes.POINTER(_ll), ctypes.POINTER(_ll)]),
    "w4a16_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
    "w4a16_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "w4a16_quantize_int4": (_i, [_ll, _ll, _vp, _vp, _vp]),
    "w4a16_dequantize_int4": (_i, [_ll, _ll, _vp, _vp, _vp]),
    "w4a16_tile_pack_host": (_i, [_ll, _ll, _i, _vp, _vp, _vp, _vp]),
    "w4a16_tile_unpack_host": (_i, [_ll, _ll, _i, _vp, _vp, _vp, _vp]),
    "w4a16_tile_pack_device": (_i, [_ll, _ll, _i, _vp, _vp, _vp, _vp, _vp]),
    "w4a16_dequant_tiled_device": (_i, [_ll, _ll, _i, _vp, _vp, _vp, _vp]),
    "w4a16_quantize_device": (_i, [_ll, _ll, _vp, _vp, _vp, _vp, _vp]),
    "gemm_int4_bf16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "silu_mul_packed_bf16": (_i, [_vp, _vp, _i, _i, _vp]),
    "gate_up_silu_int4_bf16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mlp_int4_bf16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mlp_int4_bf16_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "w4a16_rmsnorm_bf16": (_i, [_vp, _vp, _vp, _i, _i, _i, ctypes.c_float, _vp]),
    "w4a16_abi_version": (_i, []),
    "w4a16_split_wait_status": (_i, [_vp]),
    "w4a16_time_next_launch": (_i, [_i, _vp, _vp]),
    "w4a16_debug_slot_wait": (_i, [_vp, _i, _vp, _vp]),
    "mlp_int4_norm_bf16": (_i, [_vp, _vp, _i, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i,
                                _i, _vp]),
    "mlp_int4_norm_partial_f32": (_i, [_vp, _vp, _i, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _vp,
                                       _i, _i, _i, _vp]),
    "mlp_int4_residual_norm_bf16": (_i, [_vp, _vp, _vp, _i, ctypes.c_float, _vp, _vp, _vp, _vp,
                                         _vp, _vp, _i, _i, _i, _vp]),
    "engine_ffn_forward_residual_norm": (_i, [_vp, _i, _vp, _vp, _vp, _i, ctypes.c_float, _vp, _i,
                                              _vp]),
    "mlp_int4_partial_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "w4a16_manifest_check": (_i, [ctypes.c_char_p, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "w4a16_artifact_verify": (_i, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _ll,
                                   ctypes.c_char_p, ctypes.c_char_p]),
    "w4a16_sha256_hex": (_i, [_vp, ctypes.c_size_t, ctypes.c_char_p]),
    "w4a16_engine_create": (_vp, [_vp]),
    "w4a16_engine_destroy": (None, [_vp]),
    "engine_load_quantized_ffn": (_i, [_vp, ctypes.c_char_p]),
    "w4a16_load_quantized_ffn": (_i, [_vp, ctypes.c_char_p]),
    "engine_last_error": (ctypes.c_char_p, []),
    "engine_quantized_ffn_layers": (_i, [_vp]),
    "engine_ffn_operands": (_i, [_vp, _i, _vp]),
    "engine_ffn_routes_int4": (_i, [_vp, _i, _i, _i]),
    "engine_ffn_forward": (_i, [_vp, _i, _vp, _vp, _i, _vp]),
    "engine_ffn_forward_partial_f32": (_i, [_vp, _i, _vp, _vp, _i, _vp]),
    "engine_ffn_forward_norm": (_i, [_vp, _i, _vp, _vp, _i, ctypes.c_float, _vp, _i, _vp]),
    "engine_ffn_forward_norm_partial_f32": (_i, [_vp, _i, _vp, _vp, _i, ctypes.c_float, _vp, _i,
                                                 _vp]),
    "test_gemm_int4": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "test_silu_mul_packed": (_i, [_vp, _vp, _i, _i]),
}


def header_symbols():
    """Function names declared in include/w4a16.h (the exported C ABI)."""
    import re

    path = os.path.join(_HERE, "..", "include", "w4a16.h")
    with open(path) as handle:
        text = handle.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b([a-z_0-9]+)\s*\(", text)) - {"defined"})


def load_library(path=LIB_PATH):
    # torch ships its own libamdhip64.so.7; loading it first makes this library bind to the same
    # HIP runtime instead of /opt/rocm's, so torch tensors and these kernels share one runtime.
    try:
        import torch  # noqa: F401
    except ImportError:  # pragma: no cover - torch-free callers use the system runtime
        pass
    if not os.path.exists(path):
        raise ImportError(f"libw4a16.so is not built ({path}); run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


lib = load_library()


def last_error():
    return lib.w4a16_last_error().decode(errors="replace")


def _check(status, what):
    if status != W4A16_OK:
        raise W4A16Error(status, f"{what}: {last_error()}")


def _ptr(t):
    """Address of a torch tensor or numpy array (None -> NULL)."""
    if t is None:
        return None
    if isinstance(t, np.ndarray):
        return t.ctypes.data
    return t.data_ptr()


def _dev(t, nbytes, elem, what, device=None):
    """Check a device operand before its address reaches a kernel: a contiguous CUDA tensor with
    `elem`-byte elements (BF16 bits as int16/bfloat16, FP32, u8) holding at least `nbytes`, on
    `device` when given. The kernels trust their extents, so a short or strided buffer would be
    read or written out of bounds on the GPU; this raises W4A16Error instead."""
    if not hasattr(t, "data_ptr") or not hasattr(t, "is_cuda"):
        raise W4A16Error(W4A16_ERR_CONFIG, f"{what}: expected a CUDA tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise W4A16Error(W4A16_ERR_CONFIG, f"{what}: tensor is on {t.device}, not a GPU")
    if device is not None and t.device != device:
        raise W4A16Error(W4A16_ERR_CONFIG, f"{what}: tensor is on {t.device}, the call on {device}")
    if not t.is_contiguous():
        raise W4A16Error(W4A16_ERR_CONFIG, f"{what}: tensor is not contiguous")
    if t.element_size() != elem:
        raise W4A16Error(W4A16_ERR_CONFIG,
                         f"{what}: {t.dtype} has {t.element_size()}-byte elements, expected {elem}")
    have = t.numel() * elem
    if have < nbytes:
        raise W4A16Error(W4A16_ERR_CONFIG, f"{what}: {have} bytes, the call needs {nbytes}")
    return t.data_ptr()


def split_wait_status(stream=None):
    """Raise W4A16Error if a split-K combine wait gave up on the current device since the last
    check (synchronises the stream; reads and clears the device's count)."""
    _check(lib.w4a16_split_wait_status(_stream(stream)), "split_wait_status")


def _check_ffn(h, inter, gu, dn, what):
    """The gate/up pair is [2I, H] and the down weight [H, I]."""
    if not (gu.pair and gu.k == h and gu.n == 2 * inter and dn.n == h and dn.k == inter):
        raise W4A16Error(W4A16_ERR_CONFIG,
                         f"{what}: operands [{gu.n}, {gu.k}] (pair={gu.pair}) and [{dn.n}, {dn.k}] "
                         f"do not form an FFN of hidden {h}")


def _weight(w, what, device):
    """Device operands of a TiledWeight, checked against its extents."""
    return (_dev(w.packed, w.n * w.k // 2, 1, f"{what} packed", device),
            _dev(w.scales, w.n * (w.k // GROUP) * 2, 2, f"{what} scales", device))


def _stream(stream):
    if stream is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


# ----------------------------------------------------------------------------------------------
# Format (host)
# ----------------------------------------------------------------------------------------------


def layout_init(n, k, group=GROUP):
    pb, sc = _ll(0), _ll(0)
    _check(lib.w4a16_layout_init(n, k, group, ctypes.byref(pb), ctypes.byref(sc)), "layout_init")
    return pb.value, sc.value


def quantize_int4(weights):
    """FP32 [N, K] -> (packed u8 [N, K/2], scales u16 [N, K/128]), the converter's arithmetic."""
    w = np.ascontiguousarray(weights, dtype=np.float32)
    n, k = w.shape
    pb, sc = layout_init(n, k)
    packed = np.empty((n, k // 2), dtype=np.uint8)
    scales = np.empty((n, k // GROUP), dtype=np.uint16)
    _check(lib.w4a16_quantize_int4(n, k, _ptr(w), _ptr(packed), _ptr(scales)), "quantize_int4")
    return packed, scales


def dequantize_int4(packed, scales, n, k):
    out = np.empty((n, k), dtype=np.float32)
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    _check(lib.w4a16_dequantize_int4(n, k, _ptr(p), _ptr(s), _ptr(out)), "dequantize_int4")
    return out


def tile_pack_host(packed, scales, n, k, pair=False):
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    pt = np.empty(n * k // 2, dtype=np.uint8)
    st = np.empty(n * (k // GROUP), dtype=np.uint16)
    _check(lib.w4a16_tile_pack_host(n, k, int(pair), _ptr(p), _ptr(s), _ptr(pt), _ptr(st)),
           "tile_pack_host")
    return pt, st


def tile_unpack_host(packed_tiled, scales_tiled, n, k, pair=False):
    pt = np.ascontiguousarray(packed_tiled, dtype=np.uint8)
    st = np.ascontiguousarray(scales_tiled, dtype=np.uint16)
    p = np.empty((n, k // 2), dtype=np.uint8)
    s = np.empty((n, k // GROUP), dtype=np.uint16)
    _check(lib.w4a16_tile_unpack_host(n, k, int(pair), _ptr(pt), _ptr(st), _ptr(p), _ptr(s)),
           "tile_unpack_host")
    return p, s


# ----------------------------------------------------------------------------------------------
# Device operands
# ----------------------------------------------------------------------------------------------


class TiledWeight:
    """An INT4 weight resident on the device in tile order (packed u8 + BF16 scale bits)."""

    def __init__(self, packed, scales, n, k, pair):
        self.packed, self.scales, self.n, self.k, self.pair = packed, scales, n, k, pair

    @property
    def nbytes(self):
        return self.packed.numel() + self.scales.numel() * 2

    @classmethod
    def from_artifact(cls, packed, scales, n, k, pair=False, device="cuda", stream=None):
        """Upload artifact-layout (row-major) packed/scales and re-lay them on the device."""
        import torch

        p = torch.as_tensor(np.ascontiguousarray(packed, dtype=np.uint8)).reshape(-1).to(device)
        s = torch.as_tensor(np.ascontiguousarray(scales, dtype=np.uint16).view(np.int16))
        s = s.reshape(-1).to(device)
        return cls.from_device_artifact(p, s, n, k, pair, stream)

    @classmethod
    def from_device_artifact(cls, p, s, n, k, pair=False, stream=None):
        import torch

        layout_init(n, k)
        pp = _dev(p, n * k // 2, 1, "tile_pack_device packed")
        sp = _dev(s, n * (k // GROUP) * 2, 2, "tile_pack_device scales", p.device)
        pt = torch.empty(n * k // 2, dtype=torch.uint8, device=p.device)
        st = torch.empty(n * (k // GROUP), dtype=s.dtype, device=p.device)
        _check(lib.w4a16_tile_pack_device(n, k, int(pair), pp, sp, pt.data_ptr(), st.data_ptr(),
                                          _stream(stream)),
               "tile_pack_device")
        return cls(pt, st, n, k, pair)

    def dequantize(self, stream=None):
        import torch

        out = torch.empty((self.n, self.k), dtype=torch.float32, device=self.packed.device)
        wp, ws = _weight(self, "dequant_tiled_device", self.packed.device)
        _check(lib.w4a16_dequant_tiled_device(self.n, self.k, int(self.pair), wp, ws,
                                              out.data_ptr(), _stream(stream)),
               "dequant_tiled_device")
        return out


def quantize_device(weights, stream=None):
    """FP32 [N, K] CUDA tensor -> artifact-layout (packed, scales) CUDA tensors."""
    import torch

    n, k = weights.shape
    layout_init(n, k)
    weights = weights.contiguous()
    _dev(weights, n * k * 4, 4, "quantize_device weights")
    packed = torch.empty(n * k // 2, dtype=torch.uint8, device=weights.device)
    scales = torch.empty(n * (k // GROUP), dtype=torch.int16, device=weights.device)
    status = torch.zeros(1, dtype=torch.int32, device=weights.device)
    _check(lib.w4a16_quantize_device(n, k, weights.data_ptr(), packed.data_ptr(),
                                     scales.data_ptr(), status.data_ptr(), _stream(stream)),
           "quantize_device")
    if int(status.item()) != 0:
        raise W4A16Error(W4A16_ERR_CONFIG, "quantize_device: a nonfinite input or a scale the "
                                           "format cannot hold")
    return packed, scales


# ----------------------------------------------------------------------------------------------
# Compute
# ----------------------------------------------------------------------------------------------


def gemm_int4_bf16(a, w, out=None, stream=None):
    """out[M, N] = a[M, K] @ W^T; a/out are int16-viewed BF16 (or torch.bfloat16) tensors."""
    import torch

    m = a.shape[0]
    if a.dim() != 2 or a.shape[1] != w.k:
        raise W4A16Error(W4A16_ERR_CONFIG, f"gemm_int4_bf16: a is {tuple(a.shape)}, the weight "
                                           f"takes K={w.k}")
    if out is None:
        out = torch.empty((m, w.n), dtype=a.dtype, device=a.device)
    ap = _dev(a, m * w.k * 2, 2, "gemm_int4_bf16 a")
    wp, ws = _weight(w, "gemm_int4_bf16", a.device)
    op = _dev(out, m * w.n * 2, 2, "gemm_int4_bf16 out", a.device)
    _check(lib.gemm_int4_bf16(ap, wp, ws, op, m, w.n, w.k, GROUP, _stream(stream)),
           "gemm_int4_bf16")
    return out


def kernel_silu_mul_packed(out, packed, tokens, intermediate, stream=None):
    need = max(tokens, 0) * max(intermediate, 0) * 2
    op = _dev(out, need, 2, "silu_mul_packed out")
    pp = _dev(packed, 2 * need, 2, "silu_mul_packed packed", out.device)
    _check(lib.silu_mul_packed_bf16(op, pp, tokens, intermediate, _stream(stream)),
           "silu_mul_packed")
    return out


def gate_up_silu(x, gu, act=None, stream=None):
    import torch

    m, h = x.shape
    inter = gu.n // 2
    if h != gu.k:
        raise W4A16Error(W4A16_ERR_CONFIG, f"gate_up_silu: x has {h} columns, the pair takes {gu.k}")
    if act is None:
        act = torch.empty((m, inter), dtype=x.dtype, device=x.device)
    xp = _dev(x, m * h * 2, 2, "gate_up_silu x")
    wp, ws = _weight(gu, "gate_up_silu", x.device)
    ap = _dev(act, m * inter * 2, 2, "gate_up_silu act", x.device)
    _check(lib.gate_up_silu_int4_bf16(xp, wp, ws, ap, m, h, inter, _stream(stream)),
           "gate_up_silu")
    return act


def mlp_int4(x, gu, dn, out=None, act_ws=None, partial_f32=False, stream=None):
    """The INT4 dense MLP on already-normalised activations x [M, H] (BF16 bits)."""
    import torch

    m, h = x.shape
    inter = gu.n // 2
    _check_ffn(h, inter, gu, dn, "mlp_int4")
    if act_ws is None:
        act_ws = torch.empty((m, inter), dtype=x.dtype, device=x.device)
    if out is None:
        out = torch.empty((m, h), dtype=torch.float32 if partial_f32 else x.dtype,
                          device=x.device)
    osz = 4 if partial_f32 else 2
    xp = _dev(x, m * h * 2, 2, "mlp_int4 x")
    gp, gs = _weight(gu, "mlp_int4 gate/up", x.device)
    dp, ds = _weight(dn, "mlp_int4 down", x.device)
    op = _dev(out, m * h * osz, osz, "mlp_int4 out", x.device)
    wsp = _dev(act_ws, m * inter * 2, 2, "mlp_int4 act_ws", x.device)
    fn = lib.mlp_int4_partial_f32 if partial_f32 else lib.mlp_int4_bf16
    _check(fn(xp, gp, gs, dp, ds, op, wsp, m, h, inter, _stream(stream)), "mlp_int4")
    return out


def rmsnorm(x, weight, norm_style, eps, out=None, stream=None):
    """RMSNorm of the rows of x [rows, cols] (BF16 bits in int16/bfloat16 tensors)."""
    import torch

    rows, cols = x.shape
    if out is None:
        out = torch.empty_like(x)
    xp = _dev(x, rows * cols * 2, 2, "rmsnorm x")
    wp = _dev(weight, cols * 2, 2, "rmsnorm weight", x.device)
    op = _dev(out, rows * cols * 2, 2, "rmsnorm out", x.device)
    _check(lib.w4a16_rmsnorm_bf16(op, xp, wp, cols, rows, norm_style, eps, _stream(stream)),
           "w4a16_rmsnorm_bf16")
    return out


def mlp_int4_norm(residual, norm_w, norm_style, eps, gu, dn, out=None, ws=None, partial_f32=False,
                  stream=None):
    """forward_mlp: RMSNorm of residual [M, H], then the INT4 MLP."""
    import torch

    m, h = residual.shape
    inter = gu.n // 2
    _check_ffn(h, inter, gu, dn, "mlp_int4_norm")
    if ws is None:
        ws = torch.empty((m, h + inter), dtype=residual.dtype, device=residual.device)
    if out is None:
        out = torch.empty((m, h), dtype=torch.float32 if partial_f32 else residual.dtype,
                          device=residual.device)
    dev = residual.device
    osz = 4 if partial_f32 else 2
    rp = _dev(residual, m * h * 2, 2, "mlp_int4_norm residual")
    nwp = _dev(norm_w, h * 2, 2, "mlp_int4_norm norm_w", dev)
    gp, gs = _weight(gu, "mlp_int4_norm gate/up", dev)
    dp, ds = _weight(dn, "mlp_int4_norm down", dev)
    op = _dev(out, m * h * osz, osz, "mlp_int4_norm out", dev)
    wsp = _dev(ws, m * (h + inter) * 2, 2, "mlp_int4_norm ws", dev)
    fn = lib.mlp_int4_norm_partial_f32 if partial_f32 else lib.mlp_int4_norm_bf16
    _check(fn(rp, nwp, norm_style, eps, gp, gs, dp, ds, op, wsp, m, h, inter, _stream(stream)),
           "mlp_int4_norm")
    return out


def mlp_int4_residual_norm(residual, sublayer, norm_w, norm_style, eps, gu, dn, out=None, ws=None,
                           stream=None):
    """Plan F2: residual <- BF16(residual + sublayer); out = MLP(RMSNorm(residual));
    residual <- BF16(residual + out). residual is updated in place; returns out."""
    import torch

    m, h = residual.shape
    inter = gu.n // 2
    _check_ffn(h, inter, gu, dn, "mlp_int4_residual_norm")
    if ws is None:
        ws = torch.empty((m, h + inter), dtype=residual.dtype, device=residual.device)
    if out is None:
        out = torch.empty((m, h), dtype=residual.dtype, device=residual.device)
    dev = residual.device
    rp = _dev(residual, m * h * 2, 2, "mlp_int4_residual_norm residual")
    sp = _dev(sublayer, m * h * 2, 2, "mlp_int4_residual_norm sublayer", dev)
    nwp = _dev(norm_w, h * 2, 2, "mlp_int4_residual_norm norm_w", dev)
    gp, gs = _weight(gu, "mlp_int4_residual_norm gate/up", dev)
    dp, ds = _weight(dn, "mlp_int4_residual_norm down", dev)
    op = _dev(out, m * h * 2, 2, "mlp_int4_residual_norm out", dev)
    wsp = _dev(ws, m * (h + inter) * 2, 2, "mlp_int4_residual_norm ws", dev)
    _check(lib.mlp_int4_residual_norm_bf16(rp, sp, nwp, norm_style, eps, gp, gs, dp, ds, op, wsp,
                                           m, h, inter, _stream(stream)),
           "mlp_int4_residual_norm")
    return out


# ----------------------------------------------------------------------------------------------
# Sidecar and the operand store (engine_load_quantized_ffn)
# ----------------------------------------------------------------------------------------------

MANIFEST_OK, MANIFEST_ERR_ARG, MANIFEST_ERR_SYNTAX, MANIFEST_ERR_FORMAT = 0, 1, 2, 3
MANIFEST_ERR_SHAPE, MANIFEST_ERR_IO, MANIFEST_ERR_HASH = 4, 5, 6


def manifest_check(text):
    """Status of parsing and validating a sidecar document (0 ok; 1-6 as the reference reader)."""
    e, p = _i(0), _i(0)
    st = lib.w4a16_manifest_check(text.encode() if isinstance(text, str) else text,
                                  ctypes.byref(e), ctypes.byref(p))
    return st, e.value, p.value


def artifact_verify(root, file, dtype, nbytes, sha256_hex, want_dtype):
    return lib.w4a16_artifact_verify(root.encode(), file.encode(), dtype.encode(), nbytes,
                                     sha256_hex.encode(), want_dtype.encode() if want_dtype else None)


def sha256_hex(data):
    buf = ctypes.create_string_buffer(65)
    arr = np.frombuffer(data, dtype=np.uint8) if len(data) else np.zeros(1, np.uint8)
    _check(lib.w4a16_sha256_hex(arr.ctypes.data, len(data), buf), "sha256")
    return buf.value.decode()


class _EngineConfig(ctypes.Structure):
    _fields_ = [("num_layers", _i), ("layer_is_dense", ctypes.POINTER(ctypes.c_ubyte)),
                ("hidden", _i), ("intermediate", _i), ("tp_size", _i), ("tp_rank", _i),
                ("ep_size", _i), ("max_tokens", _i), ("int4_max_rows", _i)]


class FfnOperands(ctypes.Structure):
    _fields_ = [("gate_up_packed", _vp), ("gate_up_scales", _vp), ("down_packed", _vp),
                ("down_scales", _vp), ("hidden", _i), ("intermediate", _i), ("group", _i)]


class Engine:
    """The INT4 FFN operand store of one GPU (EngineHandle)."""

    def __init__(self, num_layers, hidden, intermediate, tp_size=1, tp_rank=0, ep_size=1,
                 max_tokens=16, dense=None, int4_max_rows=0):
        """int4_max_rows: verify rows routed to INT4 (0 = decode only, the reference's
        ``tokens == 1`` predicate, csrc/kernels/layers.cu:126); forwards refuse more rows."""
        flags = None
        if dense is not None:
            self._dense = (ctypes.c_ubyte * num_layers)(*[1 if d else 0 for d in dense])
            flags = ctypes.cast(self._dense, ctypes.POINTER(ctypes.c_ubyte))
        cfg = _EngineConfig(num_layers, flags, hidden, intermediate, tp_size, tp_rank, ep_size,
                            max_tokens, int4_max_rows)
        self.handle = lib.w4a16_engine_create(ctypes.byref(cfg))
        if not self.handle:
            raise W4A16Error(W4A16_ERR_CONFIG, f"engine_create: {last_error()}")
        self.hidden, self.intermediate, self.tp_size = hidden, intermediate, tp_size

    def close(self):
        if self.handle and lib is not None:  # lib is None only at interpreter shutdown
            lib.w4a16_engine_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def load_quantized_ffn(self, manifest_dir):
        """engine_load_quantized_ffn: returns the status (0 ok); raises nothing."""
        return lib.engine_load_quantized_ffn(self.handle, manifest_dir.encode())

    @staticmethod
    def last_error():
        return lib.engine_last_error().decode(errors="replace")

    @property
    def quantized_layers(self):
        return lib.engine_quantized_ffn_layers(self.handle)

    def routes_int4(self, layer, tokens, verify_rows=False):
        """engine_ffn_routes_int4: whether mlp_from_normed would take the INT4 branch."""
        return bool(lib.engine_ffn_routes_int4(self.handle, layer, tokens, int(bool(verify_rows))))

    def operands(self, layer):
        op = FfnOperands()
        _check(lib.engine_ffn_operands(self.handle, layer, ctypes.byref(op)), "engine_ffn_operands")
        return op

    def forward(self, layer, normed, out=None, partial_f32=False, stream=None):
        import torch

        m = normed.shape[0]
        if out is None:
            out = torch.empty((m, self.hidden), dtype=torch.float32 if partial_f32 else normed.dtype,
                              device=normed.device)
        osz = 4 if partial_f32 else 2
        np_ = _dev(normed, m * self.hidden * 2, 2, "engine_ffn_forward normed")
        op = _dev(out, m * self.hidden * osz, osz, "engine_ffn_forward out", normed.device)
        fn = lib.engine_ffn_forward_partial_f32 if partial_f32 else lib.engine_ffn_forward
        _check(fn(self.handle, layer, np_, op, m, _stream(stream)), "engine_ffn_forward")
        return out

    def forward_norm(self, layer, residual, norm_w, norm_style, eps, out=None, partial_f32=False,
                     stream=None):
        """forward_mlp: RMSNorm(residual) with norm_w (style 0 Gemma, 1 plain), then the FFN."""
        import torch

        m = residual.shape[0]
        if out is None:
            out = torch.empty((m, self.hidden),
                              dtype=torch.float32 if partial_f32 else residual.dtype,
                              device=residual.device)
        osz = 4 if partial_f32 else 2
        dev = residual.device
        rp = _dev(residual, m * self.hidden * 2, 2, "engine_ffn_forward_norm residual")
        nwp = _dev(norm_w, self.hidden * 2, 2, "engine_ffn_forward_norm norm_w", dev)
        op = _dev(out, m * self.hidden * osz, osz, "engine_ffn_forward_norm out", dev)
        fn = (lib.engine_ffn_forward_norm_partial_f32 if partial_f32
              else lib.engine_ffn_forward_norm)
        _check(fn(self.handle, layer, rp, nwp, norm_style, eps, op, m, _stream(stream)),
               "engine_ffn_forward_norm")
        return out

    def forward_residual_norm(self, layer, residual, sublayer, norm_w, norm_style, eps, out=None,
                              stream=None):
        """Plan F2 (tp = 1): updates residual in place and returns the layer output."""
        import torch

        m = residual.shape[0]
        if out is None:
            out = torch.empty((m, self.hidden), dtype=residual.dtype, device=residual.device)
        dev = residual.device
        rp = _dev(residual, m * self.hidden * 2, 2, "engine_ffn_forward_residual_norm residual")
        sp = _dev(sublayer, m * self.hidden * 2, 2, "engine_ffn_forward_residual_norm sublayer", dev)
        nwp = _dev(norm_w, self.hidden * 2, 2, "engine_ffn_forward_residual_norm norm_w", dev)
        op = _dev(out, m * self.hidden * 2, 2, "engine_ffn_forward_residual_norm out", dev)
        _check(lib.engine_ffn_forward_residual_norm(self.handle, layer, rp, sp, nwp, norm_style,
                                                    eps, op, m, _stream(stream)),
               "engine_ffn_forward_residual_norm")
        return out
