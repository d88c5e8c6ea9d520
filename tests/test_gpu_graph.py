"""The decode-path entry points captured into a HIP graph (marked ``gpu``).

A decode loop replays captured calls, so every entry point must give, on every replay, the
bits an eager call gives: its kernels may not depend on state that only an eager call sets up
(the split-K combine's arrival counters must be left zero by every launch), and nothing inside
may be a memset node. Each case: one eager call (which also sizes the split-K scratch), capture
of the same call, then three replays, each checked bit for bit against the eager result and each
followed by eager work on other inputs through the same entry point (which shares that scratch).
"""

import numpy as np
import pytest

import w4a16
from oracle import oracle
from test_gpu_parity import from_dev, make_ffn, norm_inputs, say, to_dev

pytestmark = pytest.mark.gpu

HIDDEN, INTER = 2560, 9728


@pytest.fixture(scope="module")
def c1_weights(cuda):
    gup, gus, dp, ds = make_ffn(HIDDEN, INTER)
    gu = w4a16.TiledWeight.from_artifact(gup, gus, 2 * INTER, HIDDEN, pair=True, device=cuda)
    dn = w4a16.TiledWeight.from_artifact(dp, ds, HIDDEN, INTER, device=cuda)
    return gu, dn


def replay_matches_eager(torch, call, outs, reset=None, other=None):
    """call() writes into the static tensors outs; reset() restores in-place inputs."""
    if reset:
        reset()
    call()
    torch.cuda.synchronize()
    want = [from_dev(o).copy() for o in outs]
    graph = torch.cuda.CUDAGraph()
    if reset:
        reset()
    with torch.cuda.graph(graph):
        if reset:
            reset()
        call()
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert np.array_equal(from_dev(o), want[i]), f"replay {rep}, output {i}"
        if other:
            other()
            torch.cuda.synchronize()


@pytest.mark.parametrize("m", [1, 2, 8, 16])
@pytest.mark.parametrize("partial", [False, True])
def test_mlp_graph_replay(cuda, c1_weights, m, partial):
    import torch

    gu, dn = c1_weights
    say(f"graph mlp_int4 M={m} partial_f32={partial}")
    x = to_dev(oracle.synth_activation(m, HIDDEN, seed=300 + m), cuda)
    x2 = to_dev(oracle.synth_activation(m, HIDDEN, seed=400 + m), cuda)
    out = torch.empty((m, HIDDEN), dtype=torch.float32 if partial else torch.int16, device=cuda)
    out2 = torch.empty_like(out)
    act = torch.empty((m, INTER), dtype=torch.int16, device=cuda)
    act2 = torch.empty_like(act)
    replay_matches_eager(
        torch, lambda: w4a16.mlp_int4(x, gu, dn, out=out, act_ws=act, partial_f32=partial),
        [out, act],
        other=lambda: w4a16.mlp_int4(x2, gu, dn, out=out2, act_ws=act2, partial_f32=partial))


@pytest.mark.parametrize("m", [1, 2, 16])
def test_mlp_norm_graph_replay(cuda, c1_weights, m):
    import torch

    gu, dn = c1_weights
    say(f"graph mlp_int4_norm M={m}")
    r, w = norm_inputs(m, HIDDEN, 0, seed=500 + m)
    r2, _ = norm_inputs(m, HIDDEN, 0, seed=600 + m)
    rd, rd2, wd = to_dev(r, cuda), to_dev(r2, cuda), to_dev(w, cuda)
    out = torch.empty((m, HIDDEN), dtype=torch.int16, device=cuda)
    out2 = torch.empty_like(out)
    ws = torch.empty((m, HIDDEN + INTER), dtype=torch.int16, device=cuda)
    ws2 = torch.empty_like(ws)
    replay_matches_eager(
        torch, lambda: w4a16.mlp_int4_norm(rd, wd, 0, 1e-6, gu, dn, out=out, ws=ws), [out],
        other=lambda: w4a16.mlp_int4_norm(rd2, wd, 0, 1e-6, gu, dn, out=out2, ws=ws2))


@pytest.mark.parametrize("m", [1, 2, 16])
def test_residual_norm_graph_replay(cuda, c1_weights, m):
    """Plan F2 updates the residual in place; the graph restores it from a pristine copy (a
    device-to-device copy node) before the call."""
    import torch

    gu, dn = c1_weights
    say(f"graph mlp_int4_residual_norm M={m}")
    r, w = norm_inputs(m, HIDDEN, 1, seed=700 + m)
    sub = oracle.synth_activation(m, HIDDEN, seed=800 + m)
    r0, wd, sd = to_dev(r, cuda), to_dev(w, cuda), to_dev(sub, cuda)
    res = r0.clone()
    res2 = r0.clone()
    out = torch.empty((m, HIDDEN), dtype=torch.int16, device=cuda)
    out2 = torch.empty_like(out)
    ws = torch.empty((m, HIDDEN + INTER), dtype=torch.int16, device=cuda)
    ws2 = torch.empty_like(ws)

    def other():
        res2.copy_(r0)
        w4a16.mlp_int4_residual_norm(res2, sd, wd, 1, 1e-6, gu, dn, out=out2, ws=ws2)

    replay_matches_eager(
        torch, lambda: w4a16.mlp_int4_residual_norm(res, sd, wd, 1, 1e-6, gu, dn, out=out, ws=ws),
        [out, res], reset=lambda: res.copy_(r0), other=other)


def test_graph_survives_scratch_growth(cuda, c1_weights):
    """A graph captured while the split-K scratch was small keeps replaying correctly after an
    eager call of a larger shape grows it (outgrown scratch is never freed)."""
    import torch

    gu, dn = c1_weights
    m = 16
    say("graph replay after split-K scratch growth")
    x = to_dev(oracle.synth_activation(m, HIDDEN, seed=900), cuda)
    out = torch.empty((m, HIDDEN), dtype=torch.float32, device=cuda)
    act = torch.empty((m, INTER), dtype=torch.int16, device=cuda)
    call = lambda: w4a16.mlp_int4(x, gu, dn, out=out, act_ws=act, partial_f32=True)  # noqa: E731
    call()
    torch.cuda.synchronize()
    want = from_dev(out).copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    torch.cuda.synchronize()
    # 16 rows against a 16384 x 16384 operand: 16 K slices x 1024 tile pairs x 1 KiB of FP32
    # partials (16 MiB), more than any other call of the suite asks for
    n = k = 16384
    w = (torch.randn(n, k, device=cuda) * 0.02).to(torch.bfloat16).float()
    p, s = w4a16.quantize_device(w)
    del w
    big = w4a16.TiledWeight.from_device_artifact(p, s, n, k)
    xb = to_dev(oracle.synth_activation(m, k, seed=901), cuda)
    w4a16.gemm_int4_bf16(xb, big)
    torch.cuda.synchronize()
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(out), want), f"replay {rep}"
        w4a16.gemm_int4_bf16(xb, big)
        torch.cuda.synchronize()
