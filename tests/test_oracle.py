"""Pins the CPU oracle (oracle/) before anything is compared against it.

Every oracle function is checked against something other than itself:

* format (bf16, layout, quantize, dequantize, packed_code): the reference's known answers
  (reference tests/quantization_format_test.c:48-245), the reference's --emit fixture and the
  golden vectors its own quantizer/dequantizer wrote (tests/golden/), and - when oracle/_ref is
  built here - the reference's compiled linear_weight.cpp on fresh random tensors;
* gemm_f64 / gemm_bf16: numpy float64 matmul of numpy's own dequantization (an independent
  library routine), plus closed forms: a one-hot activation returns a weight column exactly, a
  zero activation returns zeros, and the product is linear in the activation;
* silu_mul_packed: Python's math.exp at hand-picked points and the limits silu(0) = 0,
  silu(x) -> x, silu(-x) -> 0;
* ffn_bf16 / ffn_partial_f32: stage-by-stage recomposition from the pinned pieces above.
"""

import ctypes
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def vectors():
    return np.load(os.path.join(GOLDEN, "quantize_vectors.npz"), allow_pickle=False)


def golden_weights(vectors, name):
    if f"{name}_weights_bf16" in vectors:
        return oracle.bf16_to_f32(vectors[f"{name}_weights_bf16"])
    if f"{name}_weights_f32bits" in vectors:
        return vectors[f"{name}_weights_f32bits"].view(np.float32)
    # gate cases: the reference kernel gate's frozen legacy stream (seed 11), regenerated.
    rng = np.random.RandomState(11)
    for n, k in ((256, 128), (1024, 256)):
        w = (rng.randn(n, k) * 0.05).astype(np.float32)
        w *= (1.0 + 0.5 * rng.rand(n, k // 128).astype(np.float32)).repeat(128, axis=1)
        if name == f"gate{n}x{k}":
            return w
    raise KeyError(name)


# ---- known answers (reference tests/quantization_format_test.c) --------------------------------

def test_bf16_known_answers():
    assert oracle.lib.orc_f32_to_bf16(1.0) == 0x3F80
    assert oracle.lib.orc_f32_to_bf16(-2.0) == 0xC000
    assert oracle.lib.orc_f32_to_bf16(0.0) == 0x0000
    assert oracle.lib.orc_f32_to_bf16(1.0 + 2.0 ** -8) == 0x3F80        # tie -> even
    assert oracle.lib.orc_f32_to_bf16(1.0 + 3 * 2.0 ** -8) == 0x3F82    # tie -> even (up)
    assert oracle.lib.orc_f32_to_bf16(3.4e38) in (0x7F80, 0x7F7F)
    assert oracle.lib.orc_bf16_to_f32(0x3F80) == 1.0
    # numpy helper and C agree everywhere on a sweep of bit patterns
    pats = np.arange(0, 2 ** 32, 65521, dtype=np.uint64).astype(np.uint32)
    vals = pats.view(np.float32)
    finite = np.isfinite(vals)
    c = np.array([oracle.lib.orc_f32_to_bf16(float(v)) for v in vals[finite][:4000]])
    assert np.array_equal(c, oracle.bf16_bits(vals[finite][:4000]))


def test_layout_refusals():
    assert oracle.layout_check(8, 128) == 0
    assert oracle.layout_check(8, 256) == 0
    assert oracle.layout_check(8, 192) != 0      # 1.5 groups
    assert oracle.layout_check(12, 128) != 0     # 1.5 tiles
    assert oracle.layout_check(0, 128) != 0
    assert oracle.layout_check(8, -128) != 0
    assert oracle.layout_check(8, 128, 64) != 0  # the group is the format's, not a parameter


def test_hand_bytes_and_codes():
    w = np.zeros((8, 128), np.float32)
    w[0, :8] = [0, 1, -1, -7, 7, 3, -3, 2]
    packed, scales = oracle.quantize(w)
    assert oracle.bf16_to_f32(scales[0, 0]) == 1.0
    assert list(packed[0, :4]) == [0x10, 0x9F, 0x37, 0x2D]
    for k, want in enumerate([0, 1, -1, -7, 7, 3, -3, 2]):
        assert oracle.packed_code(packed, 0, k, 128) == want
    back = oracle.dequantize(packed, scales, 8, 128)
    assert np.array_equal(back[0, :8], w[0, :8]) and not back[0, 8:].any()


def test_edge_groups():
    w = np.zeros((8, 128), np.float32)
    packed, scales = oracle.quantize(w)
    assert (oracle.bf16_to_f32(scales) == 1.0).all() and not packed.any()
    w[0, 0], w[0, 1] = 0.7000001, -0.7000001
    packed, scales = oracle.quantize(w)
    assert oracle.packed_code(packed, 0, 0, 128) == 7
    assert oracle.packed_code(packed, 0, 1, 128) == -7
    w[:] = 0
    w[0, 0] = 1e-40                                   # scale rounds to a denormal/zero: refused
    with pytest.raises(oracle.OracleError):
        oracle.quantize(w)
    for bad in (np.nan, np.inf):
        w[:] = 0
        w[0, 5] = bad
        with pytest.raises(oracle.OracleError):
            oracle.quantize(w)
    w[:] = 0
    w[0, 0] = 0.3
    packed, scales = oracle.quantize(w)
    packed[0, 0] = (packed[0, 0] & 0xF0) | 0x08       # reserved code -8
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(packed, scales, 8, 128)
    bad_scale = scales.copy()
    bad_scale[0, 0] = 0x0000
    packed[0, 0] &= 0xF0
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(packed, bad_scale, 8, 128)


def test_requantize_fixed_point(vectors):
    w = golden_weights(vectors, "cfgK2560")
    p, s = oracle.quantize(w)
    back = oracle.dequantize(p, s, *w.shape)
    p2, s2 = oracle.quantize(back)
    assert np.array_equal(p, p2) and np.array_equal(s, s2)


# ---- golden vectors written by the reference's own code -----------------------------------------

def test_emit_fixture():
    with open(os.path.join(GOLDEN, "emit_fixture.json")) as handle:
        fx = json.load(handle)
    n, k = fx["n"], fx["k"]
    w = np.array(fx["weights_f32_bits"], np.uint32).view(np.float32).reshape(n, k)
    packed, scales = oracle.quantize(w)
    assert packed.reshape(-1).tolist() == fx["packed"]
    assert scales.reshape(-1).tolist() == fx["scales_bf16"]
    deq = oracle.dequantize(packed, scales, n, k)
    assert deq.view(np.uint32).reshape(-1).tolist() == fx["dequantized_f32_bits"]


def test_golden_quantize_dequantize(vectors):
    for name in vectors["case_names"]:
        name = str(name)
        w = golden_weights(vectors, name)
        n, k = w.shape
        packed, scales = oracle.quantize(w)
        assert np.array_equal(packed, vectors[f"{name}_packed"]), name
        assert np.array_equal(scales, vectors[f"{name}_scales"]), name
        deq = oracle.dequantize(packed, scales, n, k)
        if f"{name}_dequant_f32bits" in vectors:
            assert np.array_equal(deq.view(np.uint32), vectors[f"{name}_dequant_f32bits"]), name
        # the numpy restatement of the reference test's dequantizer agrees bit for bit
        assert np.array_equal(oracle.dequantize_numpy(packed, scales, n, k).view(np.uint32),
                              deq.view(np.uint32)), name


@pytest.mark.skipif(oracle.ref_binary("libref_format.so") is None,
                    reason="oracle/_ref not built (needs the reference tree)")
def test_against_compiled_reference_random():
    lib = ctypes.CDLL(oracle.ref_binary("libref_format.so"))

    class Layout(ctypes.Structure):
        _fields_ = [(f, ctypes.c_longlong) for f in
                    ("n", "k", "group", "packed_bytes", "scale_count")]

    rng = np.random.Generator(np.random.PCG64(99))
    for n, k, scale in ((16, 384, 0.02), (64, 1024, 3.0), (8, 128, 1e-30)):
        w = (rng.standard_normal((n, k)) * scale).astype(np.float32)
        w[0, :128] = 0.0
        lay = Layout()
        assert lib.linear_layout_init(ctypes.byref(lay), ctypes.c_longlong(n),
                                      ctypes.c_longlong(k), ctypes.c_longlong(128)) == 0
        rp = np.zeros((n, k // 2), np.uint8)
        rs = np.zeros((n, k // 128), np.uint16)
        st = lib.linear_quantize_int4(ctypes.byref(lay), ctypes.c_void_p(w.ctypes.data),
                                      ctypes.c_void_p(rp.ctypes.data),
                                      ctypes.c_void_p(rs.ctypes.data))
        if st != 0:
            with pytest.raises(oracle.OracleError):
                oracle.quantize(w)
            continue
        p, s = oracle.quantize(w)
        assert np.array_equal(p, rp) and np.array_equal(s, rs)


# ---- the matmul, SiLU and FFN -----------------------------------------------------------------

def test_gemm_against_numpy_and_closed_forms(vectors):
    w = golden_weights(vectors, "gate1024x256")
    n, k = w.shape
    p, s = vectors["gate1024x256_packed"], vectors["gate1024x256_scales"]
    x = oracle.synth_activation(3, k, seed=5)
    got = oracle.gemm_f64(x, p, s, n, k)
    deq = oracle.dequantize_numpy(p, s, n, k).astype(np.float64)
    want = oracle.bf16_to_f32(x).astype(np.float64) @ deq.T
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # one-hot activation -> exactly the dequantized column; zero -> zeros
    onehot = np.zeros((1, k), np.uint16)
    onehot[0, 37] = 0x3F80
    col = oracle.gemm_f64(onehot, p, s, n, k)[0]
    assert np.array_equal(col, deq[:, 37])
    assert not oracle.gemm_f64(np.zeros((1, k), np.uint16), p, s, n, k).any()
    # linearity: x1 + x2 (both small integers, exact in BF16)
    a = np.zeros((1, k), np.float32)
    b = np.zeros((1, k), np.float32)
    a[0, ::3], b[0, 1::5] = 2.0, -3.0
    ga = oracle.gemm_f64(oracle.bf16_bits(a), p, s, n, k)
    gb = oracle.gemm_f64(oracle.bf16_bits(b), p, s, n, k)
    gab = oracle.gemm_f64(oracle.bf16_bits(a + b), p, s, n, k)
    np.testing.assert_allclose(gab, ga + gb, rtol=1e-13, atol=1e-13)
    # the BF16 variant is exactly the rounding of the FP64 one through FP32
    gb16 = oracle.gemm_bf16(x, p, s, n, k)
    assert np.array_equal(gb16, oracle.bf16_bits(got.astype(np.float32)))


def test_silu_mul_points():
    pts = [0.0, 1.0, -1.0, 2.5, -2.5, 10.0, -10.0, 30.0, -30.0, 0.125, 88.0, -88.0]
    g = oracle.bf16_bits(np.array(pts, np.float32))
    u = oracle.bf16_bits(np.array([1.0, 0.5, -2.0, 3.0, 1.0, 1.0, 1.0, 2.0, 2.0, -1.0, 1.0, 1.0],
                                  np.float32))
    inter = len(pts)
    packed = np.concatenate([g, u])[None, :]
    act = oracle.silu_mul_packed(packed, 1, inter)[0]
    for i in range(inter):
        gv, uv = float(oracle.bf16_to_f32(g[i])), float(oracle.bf16_to_f32(u[i]))
        want = (gv / (1.0 + math.exp(-gv))) * uv
        assert act[i] == oracle.bf16_bits(np.float32(want)), (pts[i], act[i])
    assert act[0] == 0                                    # silu(0) = 0
    assert oracle.bf16_to_f32(act[7]) == 60.0             # silu(30) * 2 rounds to 60
    assert abs(float(oracle.bf16_to_f32(act[8]))) < 1e-11  # silu(-30) ~ -2.8e-12


def test_ffn_recomposes_from_stages():
    h, inter = 256, 384
    wg = oracle.synth_weight(2 * inter, h, seed=1)
    wd = oracle.synth_weight(h, inter, seed=2)
    gp, gs = oracle.quantize(wg)
    dp, ds = oracle.quantize(wd)
    x = oracle.synth_activation(2, h, seed=7)
    out, mid, act = oracle.ffn_bf16(x, gp, gs, dp, ds, h, inter)
    assert np.array_equal(mid, oracle.gemm_bf16(x, gp, gs, 2 * inter, h))
    assert np.array_equal(act, oracle.silu_mul_packed(mid, 2, inter))
    assert np.array_equal(out, oracle.gemm_bf16(act, dp, ds, h, inter))
    part = oracle.ffn_partial_f32(x, gp, gs, dp, ds, h, inter)
    assert np.array_equal(part, oracle.gemm_f64(act, dp, ds, h, inter).astype(np.float32))
    # the numpy CPU baseline lands within BF16 rounding of the oracle
    base = oracle.ffn_cpu_baseline(x, gp, gs, dp, ds, h, inter)
    d = np.abs(oracle.bf16_to_f32(base) - oracle.bf16_to_f32(out))
    assert d.max() <= 2 ** -6 * np.abs(oracle.bf16_to_f32(out)).max()


def test_rmsnorm_closed_forms():
    """orc_rmsnorm_bf16 against values the formula fixes exactly (FlashInfer RMSNorm behind
    reference csrc/kernels/flashinfer_norm.cu:22-76; bias 1 for norm_style 0 = Gemma):

    * a constant row c with eps negligible normalises to sign(c): out = BF16(b + w) exactly,
      pinning the mean (a sum would scale by 1/sqrt(cols)) and the bias per style;
    * c = 1, eps = 3 gives rsqrt(1 + 3) = 1/2 exactly: eps is added to the mean inside the root;
    * a zero row gives zeros (eps keeps the root positive);
    * scaling a row by a power of two leaves the output bit-identical (homogeneity);
    * a one-hot row v e_j with eps negligible gives sqrt(cols) * sign(v) * (b + w_j) at j.
    """
    cols = 256
    rng = np.random.default_rng(5)
    w = oracle.bf16_bits(rng.normal(0.0, 0.25, cols).astype(np.float32))
    wf = oracle.bf16_to_f32(w).astype(np.float64)
    for style, bias in ((0, 1.0), (1, 0.0)):
        want = oracle.bf16_bits((bias + wf).astype(np.float32))
        for c in (2.0, -0.375, 96.0):
            x = oracle.bf16_bits(np.full(cols, c, np.float32))
            got = oracle.rmsnorm_bf16(x, w, style, 1e-20)[0]
            expect = want if c > 0 else oracle.bf16_bits(-(bias + wf).astype(np.float32))
            assert np.array_equal(got, expect), (style, c)
        x = oracle.bf16_bits(np.ones(cols, np.float32))
        got = oracle.rmsnorm_bf16(x, w, style, 3.0)[0]
        assert np.array_equal(got, oracle.bf16_bits((0.5 * (bias + wf)).astype(np.float32)))
        zero = oracle.rmsnorm_bf16(np.zeros(cols, np.uint16), w, style, 1e-6)[0]
        assert not np.any(zero & 0x7FFF)
        xr = oracle.synth_activation(3, cols, seed=9)
        scaled = oracle.bf16_bits(oracle.bf16_to_f32(xr) * np.float32(8.0))
        assert np.array_equal(oracle.rmsnorm_bf16(xr, w, style, 1e-20),
                              oracle.rmsnorm_bf16(scaled, w, style, 1e-20))
        onehot = np.zeros(cols, np.uint16)
        onehot[17] = oracle.bf16_bits(np.float32([-3.0]))[0]
        got = oracle.rmsnorm_bf16(onehot, w, style, 1e-20)[0]
        assert got[17] == oracle.bf16_bits(np.float32([-16.0 * (bias + wf[17])]))[0]
        assert not np.any(np.delete(got, 17) & 0x7FFF)
    for bad in ((0, 1e-6, 0), (cols, 0.0, 0), (cols, float("nan"), 0), (cols, 1e-6, 2)):
        c_, eps, style = bad
        with pytest.raises(oracle.OracleError):
            oracle.lib_rmsnorm_raw(c_, eps, style)


def test_residual_norm_and_add_closed_forms():
    """Plan F2's residual update and norm (reference csrc/kernels/flashinfer_norm.cu:111-155) and
    the residual add (csrc/kernels/gdn_norm.cu:121-129):

    * the add rounds f32(a) + f32(b) to nearest-even BF16: 1 + 2^-8 -> 1 (tie, even), 1 + 3 * 2^-8
      -> 1 + 2^-6 (tie, even), 1 + 2^-8 + 2^-14 -> 1 + 2^-7 (past the tie), 2^-9 + 2^-9 exact;
    * a zero sublayer leaves the residual unchanged and normalises exactly as orc_rmsnorm_bf16;
    * sublayer = -residual zeroes both;
    * the norm reads the rounded sum: residual = sublayer = the same row gives the RMSNorm of
      2 x (a power of two, so rounding-free) = the RMSNorm of x.
    """
    b = oracle.bf16_bits(np.float32([1.0, 1.0, 1.0, 2.0 ** -9]))
    d = oracle.bf16_bits(np.float32([2.0 ** -8, 3 * 2.0 ** -8, 2.0 ** -8 + 2.0 ** -14, 2.0 ** -9]))
    got = oracle.bf16_to_f32(oracle.residual_add_bf16(b, d))
    assert list(got) == [1.0, 1.0 + 2.0 ** -6, 1.0 + 2.0 ** -7, 2.0 ** -8]
    cols = 512
    rng = np.random.default_rng(12)
    x = oracle.synth_activation(2, cols, seed=21)
    w = oracle.bf16_bits(rng.normal(0.0, 0.3, cols).astype(np.float32))
    for style in (0, 1):
        r, n = oracle.residual_norm_bf16(x, np.zeros_like(x), w, style, 1e-6)
        assert np.array_equal(r, x)
        assert np.array_equal(n, oracle.rmsnorm_bf16(x, w, style, 1e-6))
        neg = x ^ np.uint16(0x8000)
        r, n = oracle.residual_norm_bf16(x, neg, w, style, 1e-6)
        assert not np.any(r & 0x7FFF) and not np.any(n & 0x7FFF)
        r, n = oracle.residual_norm_bf16(x, x, w, style, 1e-20)
        assert np.array_equal(r, oracle.bf16_bits(2 * oracle.bf16_to_f32(x)))
        assert np.array_equal(n, oracle.rmsnorm_bf16(x, w, style, 1e-20))


def test_rmsnorm_f32order_pinned():
    """orc_rmsnorm_f32order_bf16, the reference's in-tree FP32 order (residual_norm_kernel,
    reference csrc/kernels/flashinfer_norm.cu:136-160), against values that only that order
    gives:

    * 4096^2 = 2^24 in column 0 and 1 in columns 1 and 3: the warp tree adds lanes 1 and 3 first
      (offset 2), so the total is exactly 2^24 + 2; a column-sequential FP32 sum gives 2^24
      (2^24 + 1 rounds to even), so a sequential restatement fails here;
    * the same with the ones in columns 33 and 35 (warp 1): the warp totals meet at offset 1,
      again 2^24 + 2;
    * the ones in columns 256 and 512 (thread 0's own stride): fmaf(1, 1, 2^24) rounds to 2^24
      each time, total 2^24 (a tree over columns would give 2^24 + 2);
    * the closed forms of the FP64 form hold here too (constant row -> bias + w, eps inside the
      root, zero row -> zeros), and the two forms agree within one BF16 ULP on random rows.
    """
    cols = 768
    w = oracle.bf16_bits(np.ones(cols, np.float32))
    big = oracle.bf16_bits(np.float32([4096.0]))[0]
    one = oracle.bf16_bits(np.float32([1.0]))[0]
    for ones, total in (((1, 3), 2.0 ** 24 + 2), ((33, 35), 2.0 ** 24 + 2), ((256, 512), 2.0 ** 24)):
        x = np.zeros(cols, np.uint16)
        x[0] = big
        x[list(ones)] = one
        _, rms = oracle.rmsnorm_f32order_bf16(x, w, 1, 1e-6)
        want = np.float32(1.0) / np.sqrt(np.float32(total) / np.float32(cols) + np.float32(1e-6))
        assert rms[0] == want, (ones, rms[0], want)
    rng = np.random.default_rng(6)
    wr = oracle.bf16_bits(rng.normal(0.0, 0.25, 256).astype(np.float32))
    wf = oracle.bf16_to_f32(wr).astype(np.float64)
    for style, bias in ((0, 1.0), (1, 0.0)):
        x = oracle.bf16_bits(np.full(256, 2.0, np.float32))
        got, _ = oracle.rmsnorm_f32order_bf16(x, wr, style, 1e-20)
        assert np.array_equal(got[0], oracle.bf16_bits((bias + wf).astype(np.float32)))
        x = oracle.bf16_bits(np.ones(256, np.float32))
        got, _ = oracle.rmsnorm_f32order_bf16(x, wr, style, 3.0)
        assert np.array_equal(got[0], oracle.bf16_bits((0.5 * (bias + wf)).astype(np.float32)))
        got, _ = oracle.rmsnorm_f32order_bf16(np.zeros(256, np.uint16), wr, style, 1e-6)
        assert not np.any(got & 0x7FFF)


def test_rmsnorm_order_impact():
    """How far the FP64-scale form (what the kernels compute) is from the reference's FP32 order
    on decode-like rows (BF16 ~N(0,1) times a power of two, hidden 2560 and 5120, both styles):
    the per-row FP32 scales differ by at most 3 FP32 ULPs (the FP32 sum's rounding, then the
    FP32 divide, root and reciprocal) and the normalised BF16 values by at most 1 BF16 ULP; the
    share of values that differ is printed."""
    rng = np.random.default_rng(8)
    for hidden in (2560, 5120):
        for style in (0, 1):
            rows = 200
            x = oracle.bf16_to_f32(oracle.synth_activation(rows, hidden, 70 + hidden + style))
            x *= np.float32(2.0) ** rng.integers(-3, 4, size=(rows, 1)).astype(np.float32)
            xb = oracle.bf16_bits(x)
            wb = oracle.bf16_bits(rng.normal(0.0 if style == 0 else 1.0, 0.2, hidden).astype(np.float32))
            f64 = oracle.rmsnorm_bf16(xb, wb, style, 1e-6)
            f32, rms32 = oracle.rmsnorm_f32order_bf16(xb, wb, style, 1e-6)
            ss = (oracle.bf16_to_f32(xb).astype(np.float64) ** 2).sum(axis=1)
            rms64 = (1.0 / np.sqrt(ss / hidden + np.float32(1e-6))).astype(np.float32)
            scale_ulps = np.abs(rms32.view(np.int32).astype(np.int64) - rms64.view(np.int32))
            a = f64.astype(np.int64)
            b = f32.astype(np.int64)
            sa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
            sb = np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
            d = np.abs(sa - sb)
            print(f"H={hidden} style={style}: rows with another scale {int((scale_ulps > 0).sum())}/"
                  f"{rows}, values differing {int((d > 0).sum())}/{d.size}")
            assert scale_ulps.max() <= 3
            assert d.max() <= 1
