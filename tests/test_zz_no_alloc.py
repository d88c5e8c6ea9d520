"""mlp_int4_bf16_noalloc: the allocation-free variant of mlp_int4_bf16, through the C ABI.

Its split-K partials and counters live in the library's static device array instead of the
growable per-device buffer; the kernels are the same, so its output must equal mlp_int4_bf16's
bit for bit (the split-K combines sum in a fixed order). Checked on calls in a row whose second
input is smaller, on the two routes that use the scratch: the M = 1 down projection split over
three blocks a tile (K = 17408, then K = 13312), config 2 at 16 rows (its gate/up pair on the
split-K MFMA form: the largest partials the bound admits among the BASELINE shapes) and the
16-row split-K MFMA down projection (K = 25600, then 9 rows at K = 17408); then the call
captured into a HIP graph, replayed with eager calls between the replays. Shapes beyond the
array are refused before any launch, and a first call on a device made under graph capture is
refused (it would only record the one-time clear), in a fresh process.
"""

import os
import subprocess
import sys

import ctypes

import numpy as np
import pytest

import w4a16

pytestmark = pytest.mark.gpu


def weights(torch, hidden, inter, seed):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)

    def q(n, k):
        w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(torch.bfloat16).float()
        return w4a16.quantize_device(w)

    gp, gs = q(2 * inter, hidden)
    dp, ds = q(hidden, inter)
    gu = w4a16.TiledWeight.from_device_artifact(gp, gs, 2 * inter, hidden, pair=True)
    dn = w4a16.TiledWeight.from_device_artifact(dp, ds, hidden, inter)
    return gu, dn


def call(fn, torch, x, gu, dn, M, hidden, inter):
    out = torch.full((M, hidden), 0x7FC1, dtype=torch.int16, device="cuda")
    ws = torch.full((M, inter), 0x7FC1, dtype=torch.int16, device="cuda")
    st = fn(x.data_ptr(), gu.packed.data_ptr(), gu.scales.data_ptr(), dn.packed.data_ptr(),
            dn.scales.data_ptr(), out.data_ptr(), ws.data_ptr(), M, hidden, inter,
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, w4a16.last_error()
    return out


# (M, hidden, inter): each second case is the smaller input of its pair
CASES = [(1, 5120, 17408), (1, 2048, 13312), (16, 5120, 17408), (16, 1024, 25600),
         (9, 1024, 17408)]


def test_noalloc_matches_mlp_int4(cuda):
    import torch

    for i, (M, hidden, inter) in enumerate(CASES):
        print(f"noalloc case M={M} hidden={hidden} inter={inter}", flush=True)
        gu, dn = weights(torch, hidden, inter, 77 + i)
        x = (torch.randn(M, hidden, device="cuda")).to(torch.bfloat16).view(torch.int16)
        got = call(w4a16.lib.mlp_int4_bf16_noalloc, torch, x, gu, dn, M, hidden, inter)
        want = call(w4a16.lib.mlp_int4_bf16, torch, x, gu, dn, M, hidden, inter)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, hidden, inter)
        del gu, dn


def test_noalloc_graph_replay(cuda):
    import torch

    M, hidden, inter = 1, 5120, 17408
    print(f"noalloc graph M={M} hidden={hidden} inter={inter}", flush=True)
    gu, dn = weights(torch, hidden, inter, 91)
    x = (torch.randn(M, hidden, device="cuda")).to(torch.bfloat16).view(torch.int16)
    want = call(w4a16.lib.mlp_int4_bf16, torch, x, gu, dn, M, hidden, inter)
    out = torch.zeros((M, hidden), dtype=torch.int16, device="cuda")
    ws = torch.zeros((M, inter), dtype=torch.int16, device="cuda")
    args = (x.data_ptr(), gu.packed.data_ptr(), gu.scales.data_ptr(), dn.packed.data_ptr(),
            dn.scales.data_ptr(), out.data_ptr(), ws.data_ptr(), M, hidden, inter)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        st = w4a16.lib.mlp_int4_bf16_noalloc(*args, ctypes.c_void_p(stream.cuda_stream))
    assert st == 0, w4a16.last_error()
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
        eager = call(w4a16.lib.mlp_int4_bf16_noalloc, torch, x, gu, dn, M, hidden, inter)
        torch.cuda.synchronize()
        assert torch.equal(eager, want), rep


def test_noalloc_refuses_oversized(cuda):
    """A shape whose worst-case split-K partials exceed the 32 MiB array is refused before any
    launch (the output keeps its contents)."""
    import torch

    M, hidden, inter = 16, 8192, 65536
    out = torch.full((M, hidden), 0x1234, dtype=torch.int16, device="cuda")
    st = w4a16.lib.mlp_int4_bf16_noalloc(None, None, None, None, None, out.data_ptr(), None, M,
                                         hidden, inter, None)
    assert st == w4a16.W4A16_ERR_CONFIG and "static scratch" in w4a16.last_error()
    torch.cuda.synchronize()
    assert bool((out == 0x1234).all())


FIRST_CALL_UNDER_CAPTURE = r"""
import ctypes, sys
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/haskell-infer-demo_amd"]
import torch, w4a16
M, hidden, inter = 1, 5120, 17408
gen = torch.Generator(device="cuda"); gen.manual_seed(5)
def q(n, k):
    w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(torch.bfloat16).float()
    return w4a16.quantize_device(w)
gp, gs = q(2 * inter, hidden); dp, ds = q(hidden, inter)
gu = w4a16.TiledWeight.from_device_artifact(gp, gs, 2 * inter, hidden, pair=True)
dn = w4a16.TiledWeight.from_device_artifact(dp, ds, hidden, inter)
x = torch.randn(M, hidden, generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
out = torch.zeros((M, hidden), dtype=torch.int16, device="cuda")
ws = torch.zeros((M, inter), dtype=torch.int16, device="cuda")
args = (x.data_ptr(), gu.packed.data_ptr(), gu.scales.data_ptr(), dn.packed.data_ptr(),
        dn.scales.data_ptr(), out.data_ptr(), ws.data_ptr(), M, hidden, inter)
stream = torch.cuda.Stream()
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=stream):
    st = w4a16.lib.mlp_int4_bf16_noalloc(*args, ctypes.c_void_p(stream.cuda_stream))
print("captured-first", st, w4a16.last_error())
want = torch.zeros_like(out)
st2 = w4a16.lib.mlp_int4_bf16(x.data_ptr(), gu.packed.data_ptr(), gu.scales.data_ptr(),
                              dn.packed.data_ptr(), dn.scales.data_ptr(), want.data_ptr(),
                              ws.data_ptr(), M, hidden, inter, None)
st3 = w4a16.lib.mlp_int4_bf16_noalloc(*args, None)
torch.cuda.synchronize()
print("eager-after", st2, st3, bool(torch.equal(out, want)))
"""


def test_noalloc_first_call_under_capture_refused(cuda):
    """In a fresh process, the first noalloc call on the device made under graph capture is
    refused with W4A16_ERR_STATE (its one-time clear of the static array would only be recorded
    into the graph); an eager call afterwards runs and matches mlp_int4_bf16."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc first call under capture, child process", flush=True)
    proc = subprocess.run([sys.executable, "-c", FIRST_CALL_UNDER_CAPTURE, root],
                          capture_output=True, text=True, timeout=110)
    lines = {ln.split()[0]: ln.split()[1:] for ln in proc.stdout.splitlines() if ln.strip()}
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert lines["captured-first"][0] == str(w4a16.W4A16_ERR_STATE), proc.stdout
    assert "outside graph capture" in proc.stdout
    assert lines["eager-after"] == ["0", "0", "True"], proc.stdout
