"""The loaded path on cuda:0: convert -> engine_load_quantized_ffn -> engine_ffn_forward.

* Every dense layer's operands, dequantized from tile order on the device, equal the oracle's
  dequantization of the artifact bytes bit for bit (tp=1, and each rank's slice at tp=2 with the
  global scales: reference csrc/engine.cu:2308-2395).
* engine_ffn_forward of each layer matches the oracle FFN (rel-L2 <= 1e-3, <= 2 BF16 ULP at
  the rms/16 floor, see test_gpu_parity.test_ffn_parity).
* At tp=2 the two ranks' FP32 partials sum to the full FFN within the same bar, and the sum is
  what a BF16 all-reduce would see.
"""

import ctypes
import os

import numpy as np
import pytest

import convert
import w4a16
from conftest import assert_parity
from oracle import oracle

pytestmark = pytest.mark.gpu

H, I, LAYERS = 2560, 9728, 2


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("int4_model"))
    layers = {}
    for layer in range(LAYERS):
        layers[layer] = {
            "mlpGate": oracle.synth_weight(I, H, 1000 + 3 * layer),
            "mlpUp": oracle.synth_weight(I, H, 1001 + 3 * layer),
            "mlpDown": oracle.synth_weight(H, I, 1002 + 3 * layer),
        }
    convert.write_sidecar(out, layers, "/tmp/synthetic-qwen3-4b-ffn")
    arts = {}
    for layer in range(LAYERS):
        gp, gs = oracle.quantize(layers[layer]["mlpGate"])
        up, us = oracle.quantize(layers[layer]["mlpUp"])
        dp, ds = oracle.quantize(layers[layer]["mlpDown"])
        arts[layer] = (np.concatenate([gp, up]), np.concatenate([gs, us]), dp, ds)
    return out, arts


def dequant_operand(ptr_p, ptr_s, n, k, pair, device):
    import torch

    out = torch.empty((n, k), dtype=torch.float32, device=device)
    st = w4a16.lib.w4a16_dequant_tiled_device(n, k, int(pair), ptr_p, ptr_s, out.data_ptr(),
                                              torch.cuda.current_stream().cuda_stream)
    assert st == 0, w4a16.last_error()
    return out.cpu().numpy()


def test_load_and_forward_tp1(cuda, model):
    import torch

    out, arts = model
    print("engine tp=1 load", flush=True)
    eng = w4a16.Engine(LAYERS, H, I)
    assert eng.load_quantized_ffn(out) == 0, eng.last_error()
    assert eng.quantized_layers == LAYERS
    x = oracle.synth_activation(1, H, 7)
    xd = torch.from_numpy(x.view(np.int16)).to(cuda)
    for layer in range(LAYERS):
        gup, gus, dp, ds = arts[layer]
        op = eng.operands(layer)
        assert (op.hidden, op.intermediate, op.group) == (H, I, 128)
        deq = dequant_operand(op.gate_up_packed, op.gate_up_scales, 2 * I, H, True, cuda)
        assert np.array_equal(deq.view(np.uint32),
                              oracle.dequantize_numpy(gup, gus, 2 * I, H).view(np.uint32))
        deq = dequant_operand(op.down_packed, op.down_scales, H, I, False, cuda)
        assert np.array_equal(deq.view(np.uint32),
                              oracle.dequantize_numpy(dp, ds, H, I).view(np.uint32))
        print(f"engine tp=1 forward layer {layer}", flush=True)
        got = eng.forward(layer, xd).cpu().numpy().view(np.uint16)
        ref, _, _ = oracle.ffn_bf16(x, gup, gus, dp, ds, H, I)
        assert_parity(got, ref, f"engine layer {layer}", floor_div=16.0)
        # forward_mlp: the post-attention RMSNorm folded in (plain style, eps 1e-6)
        print(f"engine tp=1 forward_norm layer {layer}", flush=True)
        nw = oracle.bf16_bits(np.random.default_rng(layer).normal(1.0, 0.2, H).astype(np.float32))
        got = eng.forward_norm(layer, xd, torch.from_numpy(nw.view(np.int16)).to(cuda), 1, 1e-6)
        normed = oracle.rmsnorm_bf16(x, nw, 1, 1e-6)
        ref, _, _ = oracle.ffn_bf16(normed, gup, gus, dp, ds, H, I)
        assert_parity(got.cpu().numpy().view(np.uint16), ref, f"engine norm layer {layer}",
                      floor_div=16.0)
        # plan F2: residual update, norm, FFN, residual add
        print(f"engine tp=1 forward_residual_norm layer {layer}", flush=True)
        sub = oracle.synth_activation(1, H, 30 + layer)
        res = xd.clone()
        got = eng.forward_residual_norm(layer, res, torch.from_numpy(sub.view(np.int16)).to(cuda),
                                        torch.from_numpy(nw.view(np.int16)).to(cuda), 1, 1e-6)
        r_mid, normed = oracle.residual_norm_bf16(x, sub, nw, 1, 1e-6)
        ref, _, _ = oracle.ffn_bf16(normed, gup, gus, dp, ds, H, I)
        assert_parity(got.cpu().numpy().view(np.uint16), ref, f"engine F2 layer {layer}",
                      floor_div=16.0)
        assert_parity(res.cpu().numpy().view(np.uint16), oracle.residual_add_bf16(r_mid, ref),
                      f"engine F2 residual layer {layer}", floor_div=16.0)
    eng.close()


def test_load_and_forward_tp2(cuda, model):
    import torch

    out, arts = model
    li = I // 2
    x = oracle.synth_activation(1, H, 7)
    xd = torch.from_numpy(x.view(np.int16)).to(cuda)
    partials = []
    for rank in range(2):
        print(f"engine tp=2 rank {rank} load", flush=True)
        eng = w4a16.Engine(LAYERS, H, I, tp_size=2, tp_rank=rank)
        assert eng.load_quantized_ffn(out) == 0, eng.last_error()
        gup, gus, dp, ds = arts[0]
        rows = np.r_[rank * li:(rank + 1) * li, I + rank * li:I + (rank + 1) * li]
        sgp, sgs = gup[rows], gus[rows]
        sdp = np.ascontiguousarray(dp[:, rank * li // 2:(rank + 1) * li // 2])
        sds = np.ascontiguousarray(ds[:, rank * li // 128:(rank + 1) * li // 128])
        op = eng.operands(0)
        assert op.intermediate == li
        deq = dequant_operand(op.gate_up_packed, op.gate_up_scales, 2 * li, H, True, cuda)
        assert np.array_equal(deq.view(np.uint32),
                              oracle.dequantize_numpy(sgp, sgs, 2 * li, H).view(np.uint32))
        deq = dequant_operand(op.down_packed, op.down_scales, H, li, False, cuda)
        assert np.array_equal(deq.view(np.uint32),
                              oracle.dequantize_numpy(sdp, sds, H, li).view(np.uint32))
        print(f"engine tp=2 rank {rank} forward", flush=True)
        part = eng.forward(0, xd, partial_f32=True).cpu().numpy()
        with pytest.raises(w4a16.W4A16Error):  # F2 adds the residual after the cross-rank sum
            eng.forward_residual_norm(0, xd.clone(), xd, xd[0], 1, 1e-6)
        want = oracle.ffn_partial_f32(x, sgp, sgs, sdp, sds, H, li)
        rel = np.linalg.norm(part.astype(np.float64) - want) / np.linalg.norm(want)
        assert rel <= 1e-3, rel
        partials.append(part)
        eng.close()
    total = oracle.bf16_bits((partials[0].astype(np.float64) + partials[1]).astype(np.float32))
    ref, _, _ = oracle.ffn_bf16(x, *arts[0], H, I)
    assert_parity(total, ref, "tp=2 partial sum vs full FFN", floor_div=16.0)


def test_engine_rows_and_tp4(cuda, model):
    """Verify rows through the engine (tokens = 4, 16: the MFMA form) at tp = 1, with the
    routing switch on (int4_max_rows = 16), and rank 3 of tp = 4 (slices of 2432 intermediate
    columns = 19 groups, reference csrc/engine.cu:2308-2395) against the oracle on the same
    slice."""
    import torch

    out, arts = model
    gup, gus, dp, ds = arts[1]
    eng = w4a16.Engine(LAYERS, H, I, max_tokens=16, int4_max_rows=16)
    assert eng.load_quantized_ffn(out) == 0, eng.last_error()
    # the routing predicate (reference csrc/kernels/layers.cu:126, extended to verify rows)
    assert eng.routes_int4(1, 1) and eng.routes_int4(1, 1, verify_rows=True)
    assert eng.routes_int4(1, 16, verify_rows=True) and not eng.routes_int4(1, 17, verify_rows=True)
    assert not eng.routes_int4(1, 4)                  # prefill rows stay on BF16
    assert not eng.routes_int4(LAYERS, 1)             # no such layer
    for tokens in (4, 16):
        print(f"engine tokens={tokens}", flush=True)
        x = oracle.synth_activation(tokens, H, 50 + tokens)
        got = eng.forward(1, torch.from_numpy(x.view(np.int16)).to(cuda)).cpu().numpy()
        ref, _, _ = oracle.ffn_bf16(x, gup, gus, dp, ds, H, I)
        assert_parity(got.view(np.uint16), ref, f"engine rows={tokens}", floor_div=16.0)
    eng.close()
    tp, rank = 4, 3
    li = I // tp
    print("engine tp=4 rank 3", flush=True)
    eng = w4a16.Engine(LAYERS, H, I, tp_size=tp, tp_rank=rank)
    assert eng.load_quantized_ffn(out) == 0, eng.last_error()
    rows = np.r_[rank * li:(rank + 1) * li, I + rank * li:I + (rank + 1) * li]
    sgp, sgs = gup[rows], gus[rows]
    sdp = np.ascontiguousarray(dp[:, rank * li // 2:(rank + 1) * li // 2])
    sds = np.ascontiguousarray(ds[:, rank * li // 128:(rank + 1) * li // 128])
    op = eng.operands(1)
    deq = dequant_operand(op.down_packed, op.down_scales, H, li, False, cuda)
    assert np.array_equal(deq.view(np.uint32),
                          oracle.dequantize_numpy(sdp, sds, H, li).view(np.uint32))
    x = oracle.synth_activation(1, H, 7)
    part = eng.forward(1, torch.from_numpy(x.view(np.int16)).to(cuda), partial_f32=True)
    want = oracle.ffn_partial_f32(x, sgp, sgs, sdp, sds, H, li)
    rel = np.linalg.norm(part.cpu().numpy().astype(np.float64) - want) / np.linalg.norm(want)
    assert rel <= 1e-3, rel
    eng.close()


def test_engine_decode_only_default(cuda, model):
    """The default store (int4_max_rows = 0) routes exactly what the reference routes: one
    decode token (reference csrc/kernels/layers.cu:126). Four rows are refused before any launch
    and the output buffer is left untouched; four verify rows run once the switch is on
    (reference tests/test_quantized_ffn.py:196-201: prefill must stay bitwise BF16)."""
    import torch

    out, arts = model
    gup, gus, dp, ds = arts[1]
    eng = w4a16.Engine(LAYERS, H, I, max_tokens=16)
    assert eng.load_quantized_ffn(out) == 0, eng.last_error()
    assert eng.routes_int4(1, 1) and not eng.routes_int4(1, 4, verify_rows=True)
    x = torch.from_numpy(oracle.synth_activation(4, H, 54).view(np.int16)).to(cuda)
    sentinel = torch.full((4, H), 0x1234, dtype=torch.int16, device=cuda)
    with pytest.raises(w4a16.W4A16Error) as err:
        eng.forward(1, x, out=sentinel)
    assert err.value.status == w4a16.W4A16_ERR_CONFIG and "int4_max_rows" in str(err.value)
    torch.cuda.synchronize()
    assert bool((sentinel == 0x1234).all())
    eng.close()
    eng = w4a16.Engine(LAYERS, H, I, max_tokens=16, int4_max_rows=4)
    assert eng.load_quantized_ffn(out) == 0, eng.last_error()
    assert eng.routes_int4(1, 4, verify_rows=True) and not eng.routes_int4(1, 4)
    got = eng.forward(1, x).cpu().numpy()
    ref, _, _ = oracle.ffn_bf16(x.cpu().numpy().view(np.uint16), gup, gus, dp, ds, H, I)
    assert_parity(got.view(np.uint16), ref, "engine verify rows=4", floor_div=16.0)
    eng.close()


def test_engine_loads_converted_checkpoint(cuda, tmp_path):
    """A BF16 safetensors checkpoint -> convert.convert_checkpoint -> engine_load_quantized_ffn ->
    engine_ffn_forward on each dense layer, against the oracle FFN of the same source weights
    (the loaded half of reference tests/test_quantization_converter.py's chain)."""
    import torch

    from test_converter import LAYER_FFNS, make_checkpoint
    from test_converter import H as CH, I as CI

    model, desc, weights = make_checkpoint(str(tmp_path))
    out = str(tmp_path / "int4")
    convert.convert_checkpoint(model, desc, out)
    eng = w4a16.Engine(len(LAYER_FFNS), CH, CI, dense=[f == "dense" for f in LAYER_FFNS])
    assert eng.load_quantized_ffn(out) == 0, eng.last_error()
    assert eng.quantized_layers == 2
    for layer in (0, 2):
        print(f"converted checkpoint layer {layer}", flush=True)
        gp, gs = oracle.quantize(weights[(layer, "gate")])
        up, us = oracle.quantize(weights[(layer, "up")])
        dp, ds = oracle.quantize(weights[(layer, "down")])
        x = oracle.synth_activation(1, CH, 60 + layer)
        got = eng.forward(layer, torch.from_numpy(x.view(np.int16)).to(cuda)).cpu().numpy()
        ref, _, _ = oracle.ffn_bf16(x, np.concatenate([gp, up]), np.concatenate([gs, us]), dp, ds,
                                    CH, CI)
        assert_parity(got.view(np.uint16), ref, f"converted layer {layer}", floor_div=16.0)
    assert not eng.routes_int4(1, 1)                    # the MoE layer keeps BF16
    eng.close()


FIRST_FORWARD_CAPTURED = r"""
import sys, tempfile
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/haskell-infer-demo_amd"]
import numpy as np, torch, convert, w4a16
from oracle import oracle
H, I = 1024, 25600                       # 16 rows: the split-K MFMA down projection
out_dir = tempfile.mkdtemp()
convert.write_sidecar(out_dir, {0: {"mlpGate": oracle.synth_weight(I, H, 11),
                                    "mlpUp": oracle.synth_weight(I, H, 12),
                                    "mlpDown": oracle.synth_weight(H, I, 13)}}, "/tmp/synthetic")
eng = w4a16.Engine(1, H, I, max_tokens=16, int4_max_rows=16)
assert eng.load_quantized_ffn(out_dir) == 0, eng.last_error()
x = torch.from_numpy(oracle.synth_activation(16, H, 21).view(np.int16)).cuda()
got = torch.zeros((16, H), dtype=torch.int16, device="cuda")
stream = torch.cuda.Stream()
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=stream):
    eng.forward(0, x, out=got, stream=stream.cuda_stream)
graph.replay()
torch.cuda.synchronize()
want = eng.forward(0, x)
torch.cuda.synchronize()
print("first-forward-captured", bool(torch.equal(got, want)))
"""


def test_engine_first_forward_under_capture(cuda):
    """In a fresh process, a store's very first forward of its largest shape (16 verify rows on
    the split-K MFMA down projection) is captured into a HIP graph: the loader reserved the
    split-K scratch, so the forward neither allocates nor synchronises, and the replay equals an
    eager forward."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("engine first forward under capture, child process", flush=True)
    proc = subprocess.run([sys.executable, "-c", FIRST_FORWARD_CAPTURED, root],
                          capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "first-forward-captured True" in proc.stdout, proc.stdout + proc.stderr
