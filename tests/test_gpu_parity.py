"""Parity of the HIP path with the CPU oracle, on cuda:0 (marked ``gpu``).

Bars: dequantized tiles bit-exact with the format's dequantizer; FFN and
GEMV outputs within rel-L2 <= 1e-3 and <= 2 BF16 ULP (ULP taken at max(|ref|, rms(ref)/64), see
conftest.parity_metrics) of the oracle's double-accumulated dequant-then-matmul with the
reference's BF16 rounding points. The reference's own kernel gate
(tests/test_quantization_kernel.py:130-136: max_rel <= 8e-3, rms_rel <= 4e-3 of max|ref|) is run
on its own shapes through the same-named bridge symbol test_gemm_int4.
"""

import os
import sys

import numpy as np
import pytest

import w4a16
from conftest import assert_parity, bf16_f32
from oracle import oracle

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def to_dev(arr, cuda):
    import torch

    a = np.ascontiguousarray(arr)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(cuda)


def from_dev(t):
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def make_weight(n, k, seed):
    w = oracle.synth_weight(n, k, seed)
    return oracle.quantize(w)


def make_ffn(hidden, inter, layer=0):
    """Gate/up pair [2I, H] (gate rows then up rows) and down [H, I], seeds 1000+3*layer+role."""
    gp, gs = make_weight(inter, hidden, 1000 + 3 * layer)
    up, us = make_weight(inter, hidden, 1001 + 3 * layer)
    dp, ds = make_weight(hidden, inter, 1002 + 3 * layer)
    return np.concatenate([gp, up]), np.concatenate([gs, us]), dp, ds


# ---- the tile order on the device ---------------------------------------------------------------

def test_tiled_dequant_bit_exact(cuda):
    vec = np.load(os.path.join(GOLDEN, "quantize_vectors.npz"), allow_pickle=False)
    for name in vec["case_names"]:
        name = str(name)
        p, s = vec[f"{name}_packed"], vec[f"{name}_scales"]
        n, k = p.shape[0], p.shape[1] * 2
        for pair in (False, True):
            say(f"tiled dequant {name} n={n} k={k} pair={pair}")
            w = w4a16.TiledWeight.from_artifact(p, s, n, k, pair=pair, device=cuda)
            hp, hs = w4a16.tile_pack_host(p, s, n, k, pair)
            assert np.array_equal(from_dev(w.packed), hp)
            assert np.array_equal(from_dev(w.scales), hs)
            deq = from_dev(w.dequantize()).view(np.uint32)
            want = oracle.dequantize_numpy(p, s, n, k).view(np.uint32)
            assert np.array_equal(deq, want), name
            if f"{name}_dequant_f32bits" in vec:
                assert np.array_equal(deq, vec[f"{name}_dequant_f32bits"].reshape(n, k))


def test_quantize_device_bit_exact(cuda):
    import torch

    gen = torch.Generator(device=cuda)
    gen.manual_seed(5)
    for n, k, std in ((64, 2560, 0.02), (256, 512, 1.0), (8, 128, 1e-3)):
        say(f"quantize_device n={n} k={k}")
        w = (torch.randn(n, k, generator=gen, device=cuda) * std).to(torch.bfloat16).float()
        w[0, :128] = 0.0
        w[1, :8] = torch.tensor([0.0, 1.0, -1.0, -7.0, 7.0, 3.0, -3.0, 2.0], device=cuda)
        p, s = w4a16.quantize_device(w)
        hp, hs = oracle.quantize(w.cpu().numpy())
        assert np.array_equal(from_dev(p).reshape(n, -1), hp)
        assert np.array_equal(from_dev(s).reshape(n, -1), hs)
    bad = torch.zeros(8, 128, device=cuda)
    bad[0, 0] = float("nan")
    with pytest.raises(w4a16.W4A16Error):
        w4a16.quantize_device(bad)


# ---- GEMV (gemm_int4_bf16, M = 1) ----------------------------------------------------------------

@pytest.mark.parametrize("n,k", [(9728, 2560), (2560, 9728), (5120, 17408), (8704, 5120),
                                 (256, 128), (1024, 384), (24, 1152),
                                 # wave-local kernel: an odd group count (13 pairs, one a
                                 # wave), tiles split over three and four blocks (64 and 96
                                 # pairs) and over five (112 and 119 pairs)
                                 (64, 3200), (64, 16384), (32, 24576), (40, 28672), (16, 30464),
                                 # the reference's M = 1 limit (K * 2 = 96 KiB): 8 blocks a tile
                                 (64, 49152),
                                 # wave-local kernel, one pair a wave, 288 and 384 tiles
                                 (2304, 4096), (3072, 4096),
                                 # 7 to 12 group pairs: the matrix-core kernel, five waves of
                                 # two pairs (7-10) and four of three (11-12) a tile, including
                                 # odd group counts
                                 (64, 1792), (64, 2816), (40, 3072), (16, 2944), (56, 1920),
                                 # 37 to 48 pairs: the matrix-core kernel, thirteen waves of
                                 # three pairs to 39, sixteen beyond (75 and 79 groups are odd)
                                 (64, 9472), (48, 9600), (32, 12288), (24, 10112), (40, 9984),
                                 # 33 to 36 pairs: twelve waves of three pairs a tile
                                 (512, 8448 + 128), (128, 8704), (64, 9216),
                                 # 17 to 20 pairs: ten waves of two pairs a tile (the
                                 # reference's published shape first; 35 groups is odd)
                                 (4096, 5120), (64, 4352), (48, 4480)])
def test_gemv_parity(cuda, n, k):
    say(f"gemv n={n} k={k}")
    p, s = make_weight(n, k, seed=n + k)
    x = oracle.synth_activation(1, k, seed=7)
    w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
    out = from_dev(w4a16.gemm_int4_bf16(to_dev(x, cuda), w))
    ref = oracle.gemm_bf16(x, p, s, n, k)
    assert_parity(out, ref, f"gemv {n}x{k}")


@pytest.mark.parametrize("m", [3, 5, 7, 13, 17, 40])
def test_small_m_parity(cuda, m):
    """The MFMA form at row counts between the instantiated ones (3, 5, 7, 13 take the 4-row
    and 16-row A layouts with zero rows) and past 16 (17 and 40 run 16-row slices)."""
    n, k = 2560, 3200  # odd group count: the last group pair is half empty
    say(f"gemm M={m} n={n} k={k}")
    p, s = make_weight(n, k, seed=77)
    x = oracle.synth_activation(m, k, seed=100 + m)
    w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
    out = from_dev(w4a16.gemm_int4_bf16(to_dev(x, cuda), w))
    assert_parity(out, oracle.gemm_bf16(x, p, s, n, k), f"gemm M={m}")


@pytest.mark.parametrize("m,n", [(16, 4096), (32, 4096), (40, 1024), (64, 1024), (64, 4096),
                                 (100, 512), (100, 4096), (128, 1024)])
def test_m_sweep_parity(cuda, m, n):
    """The reference's --time sweep shape (K = 5120; reference tests/test_quantization_kernel.py:
    162-216 times M = 1..128 at N = 4096): at 16 rows the registers-fed long-K kernel (the staged
    rows would not fit LDS), past 16 all the 16-row slices in one launch, on the kernel that runs
    each A operand against two tile pairs (32 rows at N = 4096, 128 rows at N = 1024) or four
    (64 and 100 rows at N = 4096) where that still leaves a block a CU, else one; a ragged last
    slice at 40 and 100 rows."""
    k = 5120
    say(f"gemm M={m} n={n} k={k}")
    p, s = make_weight(n, k, seed=500 + m)
    x = oracle.synth_activation(m, k, seed=600 + m)
    w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
    out = from_dev(w4a16.gemm_int4_bf16(to_dev(x, cuda), w))
    assert_parity(out, oracle.gemm_bf16(x, p, s, n, k), f"gemm M={m} {n}x{k}")


@pytest.mark.parametrize("m", [2, 3, 4, 5, 6, 7, 8, 9, 12, 15, 16])
def test_few_rows_parity(cuda, m):
    """2 <= M <= 16 on the few-row MFMA kernels, through each of their block shapes: 1 group
    pair, an odd group count with a half-filled block of tiles (and, from M = 9, a tile pair
    missing its second tile), 10, 13 (odd), 38 and 68 pairs; the last two take the registers-fed
    long-K kernel from M = 8 to 15 (at 68 pairs with its A loads kept 4 groups ahead of the
    MFMAs) and the split-K MFMA form at M = 16 (their staged rows would pass a block's LDS). The
    gate/up pair with the fused SiLU epilogue at an odd group count."""
    for n, k in [(256, 256), (24, 1152), (2560, 2560), (64, 3200), (640, 9728), (64, 17408)]:
        say(f"gemm M={m} n={n} k={k}")
        p, s = make_weight(n, k, seed=n + k + m)
        x = oracle.synth_activation(m, k, seed=200 + m)
        w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
        out = from_dev(w4a16.gemm_int4_bf16(to_dev(x, cuda), w))
        assert_parity(out, oracle.gemm_bf16(x, p, s, n, k), f"gemm M={m} {n}x{k}")
    # the gate/up pair at an odd group count; at M = 2 also on the matrix-core GEMV (7 to 12
    # group pairs, 23 groups odd), whose long-K down form the 38-pair shape above takes
    for hidden, inter in [(1152, 72)] + ([(2944, 72), (1792, 40)] if m == 2 else []):
        say(f"gate/up M={m} H={hidden} I={inter}")
        gp, gs = make_weight(2 * inter, hidden, seed=300 + m + hidden)
        x = oracle.synth_activation(m, hidden, seed=400 + m)
        gu = w4a16.TiledWeight.from_artifact(gp, gs, 2 * inter, hidden, pair=True, device=cuda)
        act = from_dev(w4a16.gate_up_silu(to_dev(x, cuda), gu))
        mid = oracle.gemm_bf16(x, gp, gs, 2 * inter, hidden)
        assert_parity(act, oracle.silu_mul_packed(mid, m, inter), f"gate/up M={m} H={hidden}")
    # two rows on the matrix-core GEMV's long-K form at odd group counts (75 groups: 38 pairs;
    # 79 groups: 40 pairs, sixteen waves), the last pair's second group past K
    for n, k in ([(48, 9600), (24, 10112)] if m == 2 else []):
        say(f"gemm M={m} n={n} k={k}")
        p, s = make_weight(n, k, seed=n + k + m)
        x = oracle.synth_activation(m, k, seed=200 + m)
        w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
        out = from_dev(w4a16.gemm_int4_bf16(to_dev(x, cuda), w))
        assert_parity(out, oracle.gemm_bf16(x, p, s, n, k), f"gemm M={m} {n}x{k}")


def test_random_shapes_parity(cuda):
    """Seeded random shapes across the routing boundaries (group-pair counts from 1 to 40, the
    staged-row LDS limits, M from 1 to 20 including the 16-row slicing), through gemm_int4_bf16
    and the fused gate/up, each against the oracle."""
    rng = np.random.default_rng(2026)
    for case in range(40):
        m = int(rng.integers(1, 21))
        k = 128 * int(rng.integers(1, 81))
        n = 8 * int(rng.integers(1, 65))
        say(f"random case {case}: M={m} N={n} K={k}")
        p, s = make_weight(n, k, seed=1000 + case)
        x = oracle.synth_activation(m, k, seed=2000 + case)
        w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
        out = from_dev(w4a16.gemm_int4_bf16(to_dev(x, cuda), w))
        assert_parity(out, oracle.gemm_bf16(x, p, s, n, k), f"random gemm M={m} N={n} K={k}")
        if n % 8 == 0 and (n // 2) % 4 == 0:
            inter = n // 2
            gu = w4a16.TiledWeight.from_artifact(p, s, n, k, pair=True, device=cuda)
            act = from_dev(w4a16.gate_up_silu(to_dev(x, cuda), gu))
            mid = oracle.gemm_bf16(x, p, s, n, k)
            assert_parity(act, oracle.silu_mul_packed(mid, m, inter),
                          f"random gate/up M={m} I={inter} K={k}")


def test_random_ffn_shapes_parity(cuda):
    """Seeded random FFN shapes around the chunk-major route (M from 2 to 18, I / 128 from 60 to
    100, hidden from 1 to 12 groups): mlp_int4 against the oracle FFN at the end-to-end bar,
    and its workspace activation against the oracle's."""
    import torch

    rng = np.random.default_rng(2027)
    for case in range(12):
        m = int(rng.integers(2, 19))
        hidden = 128 * int(rng.integers(1, 13))
        inter = 128 * int(rng.integers(60, 101))
        say(f"random ffn case {case}: M={m} H={hidden} I={inter}")
        gup, gus, dp, ds = make_ffn(hidden, inter, layer=20 + case)
        x = oracle.synth_activation(m, hidden, seed=3000 + case)
        gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
        dn = w4a16.TiledWeight.from_artifact(dp, ds, hidden, inter, device=cuda)
        xd = to_dev(x, cuda)
        act_ws = torch.empty((m, inter), dtype=xd.dtype, device=cuda)
        out = from_dev(w4a16.mlp_int4(xd, gu, dn, act_ws=act_ws))
        ref, _, ref_act = oracle.ffn_bf16(x, gup, gus, dp, ds, hidden, inter)
        assert_parity(ws_act(from_dev(act_ws), m, inter), ref_act,
                      f"random ffn act M={m} H={hidden} I={inter}")
        assert_parity(out, ref, f"random ffn M={m} H={hidden} I={inter}", floor_div=16.0)


def test_long_k_routes(cuda):
    """K past the block-staged kernel: a pair operand at M = 1 (hidden 32768) runs the MFMA form
    with one live row; M = 4 at K = 65536 (the MFMA form, 64 K splits)."""
    k, inter = 32768, 64
    say(f"gate/up pair M=1 K={k}")
    gp, gs = make_weight(2 * inter, k, seed=5)
    x = oracle.synth_activation(1, k, seed=8)
    gu = w4a16.TiledWeight.from_artifact(gp, gs, 2 * inter, k, pair=True, device=cuda)
    act = from_dev(w4a16.gate_up_silu(to_dev(x, cuda), gu))
    mid = oracle.gemm_bf16(x, gp, gs, 2 * inter, k)
    assert_parity(act, oracle.silu_mul_packed(mid, 1, inter), f"gate/up K={k}")
    n, k, m = 64, 65536, 4
    say(f"gemm M={m} K={k}")
    p, s = make_weight(n, k, seed=6)
    x = oracle.synth_activation(m, k, seed=9)
    w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
    out = from_dev(w4a16.gemm_int4_bf16(to_dev(x, cuda), w))
    assert_parity(out, oracle.gemm_bf16(x, p, s, n, k), f"gemm M={m} K={k}")


def test_gemv_closed_forms(cuda):
    n, k = 512, 2560
    p, s = make_weight(n, k, seed=3)
    w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
    deq = oracle.dequantize_numpy(p, s, n, k)
    say("gemv zero activation")
    z = from_dev(w4a16.gemm_int4_bf16(to_dev(np.zeros((1, k), np.uint16), cuda), w))
    assert not bf16_f32(z).any()
    for col in (0, 1, 127, 128, 1001, k - 1):
        say(f"gemv one-hot column {col}")
        x = np.zeros((1, k), np.uint16)
        x[0, col] = 0x3F80
        got = from_dev(w4a16.gemm_int4_bf16(to_dev(x, cuda), w))[0]
        assert np.array_equal(got, oracle.bf16_bits(deq[:, col])), col


# ---- SiLU x mul, fused gate/up, whole FFN --------------------------------------------------------

def test_silu_mul_packed(cuda):
    rng = np.random.default_rng(4)
    tokens, inter = 3, 4096
    g = rng.normal(0, 4, size=(tokens, inter)).astype(np.float32)
    g[0, :6] = [0.0, -0.0, 88.0, -88.0, 1e-20, -120.0]
    u = rng.normal(0, 1, size=(tokens, inter)).astype(np.float32)
    packed = np.concatenate([oracle.bf16_bits(g), oracle.bf16_bits(u)], axis=1)
    want = oracle.silu_mul_packed(packed, tokens, inter)
    say("silu_mul_packed kernel")
    import torch

    out = torch.empty((tokens, inter), dtype=torch.int16, device=cuda)
    w4a16.kernel_silu_mul_packed(out, to_dev(packed, cuda), tokens, inter)
    got = from_dev(out)
    m = assert_parity(got, want, "silu_mul_packed", rel_l2=1e-5, max_ulp=1.0)
    assert m["n_over_1ulp"] == 0
    # via the reference-shaped host bridge
    host = np.zeros((tokens, inter), np.uint16)
    assert w4a16.lib.test_silu_mul_packed(host.ctypes.data, packed.ctypes.data, tokens, inter) == 0
    assert np.array_equal(host, got)


@pytest.mark.parametrize("hidden,inter", [(2560, 9728), (1920, 200), (1152, 72), (3072, 40),
                                          (5120, 64)])
def test_gate_up_silu_parity(cuda, hidden, inter):
    """The fused gate/up/SiLU at M = 1 on each of its kernels: C1 and odd group counts on the
    wave-local kernel (8 and 12 pairs), the block-staged one below and above (5 and 20 pairs)."""
    say(f"gate_up_silu H={hidden} I={inter}")
    gup, gus = make_weight(2 * inter, hidden, seed=hidden + inter)
    x = oracle.synth_activation(1, hidden, seed=7)
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
    act = from_dev(w4a16.gate_up_silu(to_dev(x, cuda), gu))
    mid = oracle.gemm_bf16(x, gup, gus, 2 * inter, hidden)
    want = oracle.silu_mul_packed(mid, 1, inter)
    assert_parity(act, want, f"gate_up_silu H={hidden} I={inter}")


@pytest.mark.parametrize("hidden,inter,m", [(2560, 9728, 1), (5120, 17408, 1), (2560, 9728, 2),
                                            (2560, 9728, 4), (2560, 9728, 8), (2560, 9728, 12),
                                            (2560, 9728, 16), (5120, 17408, 16)])
def test_ffn_parity(cuda, hidden, inter, m):
    """End to end and stage by stage.

    Stages: the fused gate/up/SiLU output against the oracle's act, and the down projection
    against the oracle's down applied to the kernel's own act; each at rel-L2 <= 1e-3 and
    <= 2 BF16 ULP (floor rms/64). End to end the same bars hold with the ULP floor at rms/16:
    a one-ULP difference in a BF16 act element (two FP32-accumulated implementations round a
    gate/up value that sits on a BF16 rounding boundary differently) moves every output by about
    2^-8 * |w * act|, which is a BF16 ULP of an output near rms/64.

    From M = 4 the FFN entry keeps its intermediate chunk-major and runs the down projection on
    the registers-fed kernel. From M = 8 to 15 the public entry takes the same kernel on
    row-major rows, which sums in the same order, so the two stages match bit for bit; at M = 4
    to 7 (the LDS-staged few-row kernel) and 16 (the split-K form) the public entry sums in
    another order and the FFN is held to the stage bar against it instead.
    """
    say(f"ffn H={hidden} I={inter} M={m}")
    gup, gus, dp, ds = make_ffn(hidden, inter)
    x = oracle.synth_activation(m, hidden, seed=7 + (m if m > 1 else 0))
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, hidden, inter, device=cuda)
    xd = to_dev(x, cuda)
    out = from_dev(w4a16.mlp_int4(xd, gu, dn))
    act = w4a16.gate_up_silu(xd, gu)
    down = from_dev(w4a16.gemm_int4_bf16(act, dn))
    act = from_dev(act)
    if m < 4 or 8 <= m < 16:
        assert np.array_equal(out, down)             # mlp_int4 is exactly the two stages
    else:
        assert_parity(out, down, f"ffn M={m} against its two stages")
    ref, _, ref_act = oracle.ffn_bf16(x, gup, gus, dp, ds, hidden, inter)
    assert_parity(act, ref_act, f"ffn act stage M={m}")
    assert_parity(down, oracle.gemm_bf16(act, dp, ds, hidden, inter), f"ffn down stage M={m}")
    assert_parity(out, ref, f"ffn H={hidden} I={inter} M={m}", floor_div=16.0)


@pytest.mark.parametrize("hidden,inter,m", [(256, 8192, 4), (256, 8064, 4), (256, 8192, 3),
                                            (384, 24576, 16), (256, 24576, 5)])
def test_ffn_chunk_major_bounds(cuda, hidden, inter, m):
    """The FFN entry's chunk-major route at its edges: I / 128 = 64 (the least K it takes) and
    192 (the most, 12 groups a wave, A loads kept 3 groups ahead), M = 4 (the least M), and
    just outside (I / 128 = 63, M = 3: row-major through the public kernels). Each FFN output
    against the oracle at the end-to-end bar, its workspace activation against the oracle's,
    and the FP32 partial form against the oracle's unrounded partial."""
    import torch

    say(f"ffn chunk-major bounds H={hidden} I={inter} M={m}")
    gup, gus, dp, ds = make_ffn(hidden, inter, layer=5)
    x = oracle.synth_activation(m, hidden, seed=500 + m)
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, hidden, inter, device=cuda)
    xd = to_dev(x, cuda)
    act_ws = torch.empty((m, inter), dtype=xd.dtype, device=cuda)
    out = from_dev(w4a16.mlp_int4(xd, gu, dn, act_ws=act_ws))
    ref, _, ref_act = oracle.ffn_bf16(x, gup, gus, dp, ds, hidden, inter)
    assert_parity(ws_act(from_dev(act_ws), m, inter), ref_act, f"chunk-major act M={m} I={inter}")
    assert_parity(out, ref, f"chunk-major FFN M={m} I={inter}", floor_div=16.0)
    part = w4a16.mlp_int4(xd, gu, dn, act_ws=act_ws, partial_f32=True).cpu().numpy()
    assert np.array_equal(oracle.bf16_bits(part), out)  # the partial rounds to the output


def ws_act(flat, m, inter):
    """The intermediate as the FFN entry points leave it in their workspace: chunk-major
    ([I / 8 chunks][M rows][8 values]) from M = 4 to 16 when I / 128 is 64..192 (the
    registers-fed down kernel reads it so), otherwise row-major; returned as [M, I]."""
    a = np.asarray(flat).reshape(-1)
    if 4 <= m <= 16 and 64 <= inter // 128 <= 192:
        return a.reshape(inter // 8, m, 8).transpose(1, 0, 2).reshape(m, inter)
    return a.reshape(m, inter)


def norm_inputs(rows, hidden, style, seed):
    """A residual with a spread of row scales and a norm weight of the style's shape (Gemma
    weights are offsets around 0, plain ones gains around 1)."""
    rng = np.random.default_rng(seed)
    x = oracle.bf16_to_f32(oracle.synth_activation(rows, hidden, seed))
    x *= np.float32(2.0) ** rng.integers(-3, 4, size=(rows, 1)).astype(np.float32)
    w = rng.normal(0.0 if style == 0 else 1.0, 0.2, hidden).astype(np.float32)
    return oracle.bf16_bits(x), oracle.bf16_bits(w)


def ulp_diff(a, b):
    """|a - b| in BF16 ULPs of the larger magnitude (sign-magnitude bit patterns)."""
    ia = np.where(a & 0x8000, -(a & 0x7FFF).astype(np.int64), (a & 0x7FFF).astype(np.int64))
    ib = np.where(b & 0x8000, -(b & 0x7FFF).astype(np.int64), (b & 0x7FFF).astype(np.int64))
    return np.abs(ia - ib)


@pytest.mark.parametrize("style", [0, 1])
def test_rmsnorm_parity(cuda, style):
    """w4a16_rmsnorm_bf16 against the oracle: within 1 BF16 ULP everywhere (the FP32 sum of
    squares is ordered differently from the oracle's double), and bit-exact for >= 99%."""
    for rows, hidden in ((1, 2560), (5, 5120), (16, 2560)):
        say(f"rmsnorm style={style} rows={rows} H={hidden}")
        x, w = norm_inputs(rows, hidden, style, seed=40 + rows)
        got = from_dev(w4a16.rmsnorm(to_dev(x, cuda), to_dev(w, cuda), style, 1e-6))
        want = oracle.rmsnorm_bf16(x, w, style, 1e-6)
        d = ulp_diff(got, want)
        assert d.max() <= 1, (rows, hidden, int(d.max()))
        assert np.mean(d == 0) >= 0.99
        # the reference's in-tree FP32 order (flashinfer_norm.cu:136-160): within 1 BF16 ULP too
        want32, _ = oracle.rmsnorm_f32order_bf16(x, w, style, 1e-6)
        d32 = ulp_diff(got, want32)
        say(f"  vs FP32-order restatement: max {int(d32.max())} ULP, {int((d32 > 0).sum())}/{d32.size} differ")
        assert d32.max() <= 1, (rows, hidden, int(d32.max()))


@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("m", [1, 2, 16])
def test_ffn_norm_parity(cuda, style, m):
    """mlp_int4_norm (forward_mlp, reference csrc/kernels/layers.cu:150-159) against the
    oracle's RMSNorm followed by the oracle FFN, at the end-to-end bar of test_ffn_parity; at
    M = 1 the norm runs inside the gate/up kernel (the block-staged GEMV's prologue), otherwise in
    its own kernel ahead of the FFN. The FP32 partial form is checked against the oracle's
    unrounded partial."""
    hidden, inter = 2560, 9728
    say(f"ffn norm style={style} M={m}")
    gup, gus, dp, ds = make_ffn(hidden, inter)
    x, w = norm_inputs(m, hidden, style, seed=60 + m)
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, hidden, inter, device=cuda)
    xd, wd = to_dev(x, cuda), to_dev(w, cuda)
    import torch

    ws = torch.empty((m, hidden + inter), dtype=xd.dtype, device=cuda)
    out = from_dev(w4a16.mlp_int4_norm(xd, wd, style, 1e-6, gu, dn, ws=ws))
    normed = oracle.rmsnorm_bf16(x, w, style, 1e-6)
    ref, _, ref_act = oracle.ffn_bf16(normed, gup, gus, dp, ds, hidden, inter)
    act = ws_act(from_dev(ws.reshape(-1)[m * hidden:]), m, inter)  # ws = normed | act
    assert_parity(act, ref_act, f"ffn norm act stage M={m}", floor_div=16.0)
    assert_parity(out, ref, f"ffn norm H={hidden} I={inter} M={m}", floor_div=16.0)
    part = from_dev(w4a16.mlp_int4_norm(xd, wd, style, 1e-6, gu, dn, partial_f32=True))
    want = oracle.ffn_partial_f32(normed, gup, gus, dp, ds, hidden, inter)
    rel = np.linalg.norm(part.astype(np.float64) - want) / np.linalg.norm(want)
    assert rel <= 1e-3, rel


@pytest.mark.parametrize("m", [2, 3, 5, 8])
def test_ffn_norm_fused_rows(cuda, m):
    """mlp_int4_norm for 2 <= M <= 8 against the explicit composition, for both norm styles: the
    standalone RMSNorm then the fused gate/up, act and output bit-identical (the same kernels as
    the call's), and within rel-L2 1e-3 of the oracle end to end. (Against the oracle's
    per-element bar these residual inputs leave a few act values at 3 BF16 ULP at M = 5 and 8:
    one normalised value rounded the other way moves every gate/up sum.)"""
    import torch

    hidden, inter = 2560, 9728
    say(f"ffn fused-rows norm M={m}")
    gup, gus, dp, ds = make_ffn(hidden, inter)
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, hidden, inter, device=cuda)
    for style in (0, 1):
        x, w = norm_inputs(m, hidden, style, seed=60 + m)
        xd, wd = to_dev(x, cuda), to_dev(w, cuda)
        ws = torch.empty((m, hidden + inter), dtype=xd.dtype, device=cuda)
        out = from_dev(w4a16.mlp_int4_norm(xd, wd, style, 1e-6, gu, dn, ws=ws))
        act = ws_act(from_dev(ws.reshape(-1)[m * hidden:]), m, inter)
        normed = w4a16.rmsnorm(xd, wd, style, 1e-6)
        act2 = w4a16.gate_up_silu(normed, gu)
        assert np.array_equal(act, from_dev(act2)), (m, style)
        down2 = from_dev(w4a16.gemm_int4_bf16(act2, dn))
        if m < 4 or m >= 8:  # the same down kernel and summation order
            assert np.array_equal(out, down2), (m, style)
        else:  # chunk-major registers-fed down against the public entry's LDS-staged one
            assert_parity(out, down2, f"norm FFN M={m} against its two stages")
        ref, _, _ = oracle.ffn_bf16(oracle.rmsnorm_bf16(x, w, style, 1e-6), gup, gus, dp, ds,
                                    hidden, inter)
        o, r = bf16_f32(out).astype(np.float64), bf16_f32(ref).astype(np.float64)
        assert np.linalg.norm(o - r) / np.linalg.norm(r) <= 1e-3, (m, style)


def test_f2_separate_norm_m1(cuda):
    """Plan F2 at M = 1 past the fused prologue's hidden size (13 group pairs): the standalone
    norm updates the residual, and the down kernel adds its output into it (no sublayer in its
    epilogue); the layer output against the oracle and the residual bit-exact given it."""
    hidden, inter = 3328, 3328
    say(f"F2 separate norm H={hidden} I={inter}")
    gup, gus = make_weight(2 * inter, hidden, seed=700)
    dp, ds = make_weight(hidden, inter, seed=701)
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, hidden, inter, device=cuda)
    for style in (0, 1):
        x, w = norm_inputs(1, hidden, style, seed=72)
        sub = oracle.synth_activation(1, hidden, seed=73)
        r_mid, normed = oracle.residual_norm_bf16(x, sub, w, style, 1e-6)
        ref, _, _ = oracle.ffn_bf16(normed, gup, gus, dp, ds, hidden, inter)
        res = to_dev(x, cuda)
        got = from_dev(w4a16.mlp_int4_residual_norm(res, to_dev(sub, cuda), to_dev(w, cuda),
                                                    style, 1e-6, gu, dn))
        assert_parity(got, ref, f"F2 H={hidden} style={style}", floor_div=16.0)
        assert np.array_equal(from_dev(res), oracle.residual_add_bf16(r_mid, got))


@pytest.mark.parametrize("hidden", [1152, 1920, 3072])
def test_norm_prologue_shapes(cuda, hidden):
    """The M = 1 norm (and plan-F2) prologue of the block-staged gate/up kernel at 5, 8 (odd
    group count) and 12 group pairs: the act stage and the F2 layer output against the oracle,
    the updated residual bit-exact given the kernel's output."""
    import torch

    inter = 128
    say(f"norm prologue H={hidden}")
    gup, gus = make_weight(2 * inter, hidden, seed=500 + hidden)
    dp, ds = make_weight(hidden, inter, seed=600 + hidden)
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, hidden, inter, device=cuda)
    for style in (0, 1):
        x, w = norm_inputs(1, hidden, style, seed=70 + hidden)
        xd = to_dev(x, cuda)
        ws = torch.empty((1, hidden + inter), dtype=xd.dtype, device=cuda)
        w4a16.mlp_int4_norm(xd, to_dev(w, cuda), style, 1e-6, gu, dn, ws=ws)
        act = from_dev(ws.reshape(-1)[hidden:].reshape(1, inter))
        _, _, ref_act = oracle.ffn_bf16(oracle.rmsnorm_bf16(x, w, style, 1e-6), gup, gus, dp, ds,
                                        hidden, inter)
        assert_parity(act, ref_act, f"norm prologue H={hidden} style={style}", floor_div=16.0)
        sub = oracle.synth_activation(1, hidden, seed=71 + hidden)
        r_mid, normed = oracle.residual_norm_bf16(x, sub, w, style, 1e-6)
        ref, _, _ = oracle.ffn_bf16(normed, gup, gus, dp, ds, hidden, inter)
        res = to_dev(x, cuda)
        got = from_dev(w4a16.mlp_int4_residual_norm(res, to_dev(sub, cuda), to_dev(w, cuda),
                                                    style, 1e-6, gu, dn))
        assert_parity(got, ref, f"F2 H={hidden} style={style}", floor_div=16.0)
        assert np.array_equal(from_dev(res), oracle.residual_add_bf16(r_mid, got))


@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("m", [1, 2, 12, 16])
def test_ffn_residual_norm_parity(cuda, style, m):
    """Plan F2 around the MLP (reference csrc/layer_dispatch.cu:183-209), with the residual added
    in each down kernel's epilogue (M = 12: the registers-fed long-K kernel): the layer output
    against the oracle (residual update, norm, FFN) at the end-to-end bar, and the updated
    residual BF16(BF16(r + s) + out) bit-exact given the kernel's own output; at M = 1 and 2 (the
    two-launch forms) also with the sublayer aliasing the output buffer, as the reference's
    layer_out does."""
    import torch

    hidden, inter = 2560, 9728
    say(f"ffn residual norm style={style} M={m}")
    gup, gus, dp, ds = make_ffn(hidden, inter)
    x, w = norm_inputs(m, hidden, style, seed=80 + m)
    sub = oracle.bf16_bits(oracle.bf16_to_f32(oracle.synth_activation(m, hidden, seed=90 + m)) *
                           np.float32(0.5))
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * inter, hidden, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, hidden, inter, device=cuda)
    r_mid, normed = oracle.residual_norm_bf16(x, sub, w, style, 1e-6)
    ref, _, _ = oracle.ffn_bf16(normed, gup, gus, dp, ds, hidden, inter)
    r_ref = oracle.residual_add_bf16(r_mid, ref)
    for alias in ((False, True) if m <= 2 else (False,)):
        res = to_dev(x, cuda)
        sd = to_dev(sub, cuda)
        out = sd if alias else torch.empty_like(sd)
        got = from_dev(w4a16.mlp_int4_residual_norm(res, sd, to_dev(w, cuda), style, 1e-6, gu, dn,
                                                    out=out))
        assert_parity(got, ref, f"F2 out M={m} alias={alias}", floor_div=16.0)
        # the residual is exact arithmetic on exact inputs: BF16(BF16(r + s) + out) with the
        # kernel's own out must match bit for bit (against the oracle's out it moves by the
        # output's ULPs, which on a cancelling element are many of the residual's)
        assert np.array_equal(from_dev(res), oracle.residual_add_bf16(r_mid, got)), (m, alias)
        assert_parity(from_dev(res), r_ref, f"F2 residual M={m} alias={alias}", floor_div=16.0,
                      max_ulp=16.0)


def test_ffn_tp_slice_partial_f32(cuda):
    """Config 4: rank 0 of tp=2 on the 27B FFN, scales kept global (reference
    csrc/engine.cu:2308-2369: gate/up rows 0..I/2-1 of each half, down columns 0..I/2-1)."""
    hidden, inter = 5120, 17408
    half = inter // 2
    say("ffn tp slice (config 4)")
    gup, gus, dp, ds = make_ffn(hidden, inter)
    sgp = np.concatenate([gup[:half], gup[inter:inter + half]])
    sgs = np.concatenate([gus[:half], gus[inter:inter + half]])
    sdp = np.ascontiguousarray(dp[:, :half // 2])
    sds = np.ascontiguousarray(ds[:, :half // 128])
    x = oracle.synth_activation(1, hidden, seed=7)
    gu = w4a16.TiledWeight.from_artifact(sgp, sgs, 2 * half, hidden, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(sdp, sds, hidden, half, device=cuda)
    got = from_dev(w4a16.mlp_int4(to_dev(x, cuda), gu, dn, partial_f32=True))
    ref = oracle.ffn_partial_f32(x, sgp, sgs, sdp, sds, hidden, half)
    d = np.abs(got.astype(np.float64) - ref)
    rel = np.linalg.norm(d) / np.linalg.norm(ref)
    say(f"tp partial rel_l2={rel:.3g} max_abs={d.max():.3g}")
    assert rel <= 1e-3
    # rounded as the reference's BF16 all-reduce input would be
    assert_parity(oracle.bf16_bits(got), oracle.bf16_bits(ref), "tp partial as BF16")


# ---- the reference's own kernel gate, through its bridge symbol ---------------------------------

def test_reference_kernel_gate_shapes():
    rng = np.random.RandomState(11)
    for n, k in ((256, 128), (1024, 256), (4096, 5120)):
        w = (rng.randn(n, k) * 0.05).astype(np.float32)
        w *= (1.0 + 0.5 * rng.rand(n, k // 128).astype(np.float32)).repeat(128, axis=1)
        packed, scales = oracle.quantize(w)
        deq = oracle.dequantize_numpy(packed, scales, n, k).astype(np.float64)
        for m in (1, 2, 8, 64):
            x = (rng.randn(m, k) * 0.5).astype(np.float32)
            a_bits = np.ascontiguousarray(oracle.bf16_bits(x))
            ref = bf16_f32(a_bits).astype(np.float64) @ deq.T
            out = np.empty((m, n), np.uint16)
            say(f"test_gemm_int4 bridge M={m} N={n} K={k}")
            st = w4a16.lib.test_gemm_int4(out.ctypes.data, a_bits.ctypes.data, packed.ctypes.data,
                                          scales.ctypes.data, m, n, k, 128)
            assert st == 0, w4a16.last_error()
            err = np.abs(bf16_f32(out).astype(np.float64) - ref)
            scale = max(np.abs(ref).max(), 1e-9)
            assert err.max() / scale <= 8e-3 and np.sqrt((err ** 2).mean()) / scale <= 4e-3
            assert_parity(out, oracle.bf16_bits(ref.astype(np.float32)), f"gate M={m} {n}x{k}")
    bad = np.zeros(128 * 192 // 2, np.uint8)
    out = np.zeros((1, 128), np.uint16)
    assert w4a16.lib.test_gemm_int4(out.ctypes.data, out.ctypes.data, bad.ctypes.data,
                                    np.zeros(128, np.uint16).ctypes.data, 1, 128, 192, 128) != 0


def test_wrappers_refuse_short_or_strided_device_buffers(cuda):
    """A caller-supplied output or workspace that is too small, strided or of the wrong element
    width is refused before the kernel is launched (the kernels trust their extents)."""
    import torch

    n, k = 64, 2560
    p, s = make_weight(n, k, seed=3)
    w = w4a16.TiledWeight.from_artifact(p, s, n, k, device=cuda)
    a = to_dev(oracle.synth_activation(2, k, seed=4), cuda)
    with pytest.raises(w4a16.W4A16Error, match="bytes, the call needs"):
        w4a16.gemm_int4_bf16(a, w, out=torch.empty((2, n - 8), dtype=torch.int16, device=cuda))
    with pytest.raises(w4a16.W4A16Error, match="not contiguous"):
        w4a16.gemm_int4_bf16(a, w, out=torch.empty((n, 2), dtype=torch.int16, device=cuda).t())
    with pytest.raises(w4a16.W4A16Error, match="4-byte elements"):
        w4a16.gemm_int4_bf16(a, w, out=torch.empty((2, n), dtype=torch.float32, device=cuda))
    gup, gus, dp, ds = make_ffn(256, 512)
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 1024, 256, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, 256, 512, device=cuda)
    x = to_dev(oracle.synth_activation(4, 256, seed=5), cuda)
    with pytest.raises(w4a16.W4A16Error, match="act_ws"):
        w4a16.mlp_int4(x, gu, dn, act_ws=torch.empty((2, 512), dtype=torch.int16, device=cuda))
    out = from_dev(w4a16.mlp_int4(x, gu, dn))           # the same call with valid buffers
    assert out.shape == (4, 256)
