"""The converter end to end on the CPU, mirroring reference tests/test_quantization_converter.py
(a synthetic BF16 checkpoint -> convert -> --verify -> the C reader, plus the refusals).

* A two-shard BF16 safetensors checkpoint (8-byte header length, JSON header, raw bytes) and a
  descriptor are written with numpy; one layer is not dense and stays BF16.
* convert_checkpoint writes artifacts that are the quantizer's bytes for each source tensor (and
  the reference's compiled quantizer's, when oracle/_ref is built), the F1 pair, the precision map
  over every (layer, role), and the source and descriptor digests.
* verify() accepts it; this library's reader accepts it; the reference's own reader (compiled
  in oracle/_ref) verifies every artifact; engine_load_quantized_ffn passes every host-side
  check and stops only at the device upload (no GPU here; tests/test_engine_gpu.py loads it).
* Refused: a flipped artifact byte (verify, the library reader's hash check, the reference
  reader), a foreign format block, a pair listing [mlpUp, mlpGate], a source shard changed after
  conversion, an FP16 source tensor, a tensor named in two shards, a missing tensor.
"""

import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import convert
import w4a16
from oracle import oracle

H, I = 256, 384
ROLE_NAMES = ["embed", "inputNorm", "mlpGate", "mlpUp", "mlpDown", "postNorm"]
TEMPLATES = ["model.embed_tokens.weight", "model.layers.%d.input_layernorm.weight",
             "model.layers.%d.mlp.gate_proj.weight", "model.layers.%d.mlp.up_proj.weight",
             "model.layers.%d.mlp.down_proj.weight", "model.layers.%d.post_attention_layernorm.weight"]
LAYER_FFNS = ["dense", "moe", "dense"]


def bf16_bits(a):
    return oracle.bf16_bits(np.asarray(a, np.float32))


def write_safetensors(path, tensors, dtype="BF16"):
    """numpy -> safetensors: u64 header length, JSON header, then the raw little-endian bytes."""
    header, blobs, off = {}, [], 0
    for name, arr in tensors.items():
        raw = (bf16_bits(arr) if dtype == "BF16" else np.asarray(arr, np.float16)).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as handle:
        handle.write(struct.pack("<Q", len(text)) + text + b"".join(blobs))


def make_checkpoint(root, fp16_role=None, duplicate=False):
    model = os.path.join(root, "model")
    os.makedirs(model, exist_ok=True)
    shards = [{}, {}]
    shards[0]["model.embed_tokens.weight"] = oracle.synth_weight(64, H, 5)
    weights = {}
    for layer, ffn in enumerate(LAYER_FFNS):
        shard = shards[layer % 2]
        shard[f"model.layers.{layer}.input_layernorm.weight"] = np.ones(H, np.float32)
        shard[f"model.layers.{layer}.post_attention_layernorm.weight"] = np.ones(H, np.float32)
        if ffn != "dense":
            continue
        for role, (n, k), seed in (("gate", (I, H), 0), ("up", (I, H), 1), ("down", (H, I), 2)):
            w = oracle.synth_weight(n, k, 2000 + 3 * layer + seed)
            weights[(layer, role)] = w
            shard[f"model.layers.{layer}.mlp.{role}_proj.weight"] = w
    if duplicate:
        shards[1]["model.layers.0.mlp.gate_proj.weight"] = weights[(0, "gate")]
    for i, tensors in enumerate(shards):
        if fp16_role and i == 0:
            name = f"model.layers.0.mlp.{fp16_role}_proj.weight"
            f16 = {name: tensors.pop(name)}
            write_safetensors(os.path.join(model, "model-00003.safetensors"), f16, "F16")
        write_safetensors(os.path.join(model, f"model-0000{i + 1}.safetensors"), tensors)
    desc = os.path.join(root, "descriptor.json")
    with open(desc, "w") as handle:
        json.dump({"num_layers": len(LAYER_FFNS), "role_names": ROLE_NAMES,
                   "role_templates": TEMPLATES, "layer_ffns": LAYER_FFNS}, handle)
    return model, desc, weights


@pytest.fixture(scope="module")
def converted(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("ckpt"))
    model, desc, weights = make_checkpoint(root)
    out = os.path.join(root, "int4")
    manifest = convert.convert_checkpoint(model, desc, out)
    return root, model, desc, out, manifest, weights


def test_artifacts_are_the_quantizers_bytes(converted):
    _, model, desc, out, manifest, weights = converted
    names = {"mlpGate": "gate", "mlpUp": "up", "mlpDown": "down"}
    assert {(e["layer"], e["role"]) for e in manifest["entries"]} == \
        {(l, r) for l in (0, 2) for r in names}
    quantizer = oracle.ref_binary("quantization_format_test")
    for e in manifest["entries"]:
        w = weights[(e["layer"], names[e["role"]])]
        p, s = oracle.quantize(w)
        with open(os.path.join(out, e["packed"]["file"]), "rb") as handle:
            assert handle.read() == p.tobytes()
        with open(os.path.join(out, e["scales"]["file"]), "rb") as handle:
            assert handle.read() == s.tobytes()
        assert e["checkpoint_tensor"] == f"model.layers.{e['layer']}.mlp.{names[e['role']]}_proj.weight"
        if quantizer:
            rp, rs = convert._quantize_with(quantizer, w)
            assert rp == p.tobytes() and rs == s.tobytes()
    cells = {(c["layer"], c["role"]): c["precision"] for c in manifest["precision_map"]}
    assert len(cells) == len(LAYER_FFNS) * len(ROLE_NAMES) == len(manifest["precision_map"])
    assert cells[(1, "mlpGate")] == "bf16" and cells[(2, "mlpDown")] == "int4"
    assert cells[(0, "embed")] == "bf16"
    assert [p["layer"] for p in manifest["pairs"]] == [0, 2]
    assert manifest["descriptor"]["sha256"] == convert.sha256_file(desc)
    assert [f["name"] for f in manifest["source"]["files"]] == \
        ["model-00001.safetensors", "model-00002.safetensors"]
    assert manifest["format"] == convert.FORMAT


def test_verify_and_readers_accept(converted):
    _, _, _, out, manifest, _ = converted
    path = os.path.join(out, "weights.manifest.json")
    assert convert.verify(path) == []
    quantizer = oracle.ref_binary("quantization_format_test")
    if quantizer:
        assert convert.verify(path, quantizer) == []
    with open(path) as handle:
        text = handle.read()
    st, entries, pairs = w4a16.manifest_check(text)
    assert (st, entries, pairs) == (0, 6, 2), w4a16.last_error()
    for e in manifest["entries"] + manifest["pairs"]:
        for kind, dtype in (("packed", "u8"), ("scales", "bf16")):
            a = e[kind]
            assert w4a16.artifact_verify(out, a["file"], a["dtype"], a["bytes"], a["sha256"], dtype) == 0
    binary = oracle.ref_binary("quant_manifest_test")
    if binary:
        proc = subprocess.run([binary, "--manifest", path, "--root", out], capture_output=True, text=True)
        assert proc.returncode == 0 and "verified" in proc.stdout, proc.stdout + proc.stderr
    # the loader: every host-side check passes, and a GPU-less store stops at the upload
    eng = w4a16.Engine(len(LAYER_FFNS), H, I, dense=[f == "dense" for f in LAYER_FFNS])
    st = eng.load_quantized_ffn(out)
    if st != 0:
        assert st == w4a16.W4A16_ERR_WEIGHTS and "no device" in eng.last_error(), eng.last_error()
    eng.close()


def copy_out(converted, tmp_path):
    out = converted[3]
    bad = str(tmp_path / "bad")
    shutil.copytree(out, bad)
    return bad, os.path.join(bad, "weights.manifest.json")


def test_flipped_byte_refused(converted, tmp_path):
    bad, path = copy_out(converted, tmp_path)
    manifest = converted[4]
    victim = manifest["entries"][0]["packed"]   # the one the reference binary re-reads
    with open(os.path.join(bad, victim["file"]), "r+b") as handle:
        handle.seek(33)
        b = handle.read(1)
        handle.seek(33)
        handle.write(bytes([b[0] ^ 0x10]))
    problems = convert.verify(path)
    assert any("content hash" in p for p in problems), problems
    assert w4a16.artifact_verify(bad, victim["file"], "u8", victim["bytes"], victim["sha256"], "u8") == 6
    binary = oracle.ref_binary("quant_manifest_test")
    if binary:
        proc = subprocess.run([binary, "--manifest", path, "--root", bad], capture_output=True, text=True)
        assert proc.returncode != 0
    # the loader reads the pair and the down entry: flip a byte of layer 0's pair too
    pair = manifest["pairs"][0]["packed"]
    with open(os.path.join(bad, pair["file"]), "r+b") as handle:
        handle.seek(5)
        b = handle.read(1)
        handle.seek(5)
        handle.write(bytes([b[0] ^ 0x01]))
    eng = w4a16.Engine(len(LAYER_FFNS), H, I, dense=[f == "dense" for f in LAYER_FFNS])
    assert eng.load_quantized_ffn(bad) == w4a16.W4A16_ERR_WEIGHTS
    assert "hashes to" in eng.last_error()
    eng.close()


def test_foreign_format_refused(converted, tmp_path):
    """A foreign format block. --verify compares every key of the block (as the reference's does),
    so a renamed format fails it; the readers, like the reference reader (quant_manifest.c
    parses the name without comparing it), refuse on the numeric keys: abi_version,
    zero_point."""
    bad, path = copy_out(converted, tmp_path)
    with open(path) as handle:
        text = handle.read()
    renamed = text.replace('"name": "int4_symmetric_group_bf16_scale"', '"name": "int4_asymmetric_zp"', 1)
    assert renamed != text
    with open(path, "w") as handle:
        handle.write(renamed)
    assert any("format block: 'name'" in p for p in convert.verify(path))
    lib = oracle.ref_binary("libref_format.so")
    for needle, repl in (('"abi_version": 1', '"abi_version": 2'), ('"zero_point": 0', '"zero_point": 8')):
        foreign = text.replace(needle, repl, 1)
        assert foreign != text
        st, _, _ = w4a16.manifest_check(foreign)
        assert st == 3, w4a16.last_error()
        if lib:
            import ctypes

            ref = ctypes.CDLL(lib)
            buf, err = ctypes.create_string_buffer(8 << 20), ctypes.create_string_buffer(512)
            assert ref.quant_manifest_parse(foreign.encode(), buf, err, 512) == 3
        with open(path, "w") as handle:
            handle.write(foreign)
        assert any("format block" in p for p in convert.verify(path))
        eng = w4a16.Engine(len(LAYER_FFNS), H, I, dense=[f == "dense" for f in LAYER_FFNS])
        assert eng.load_quantized_ffn(bad) == w4a16.W4A16_ERR_WEIGHTS
        assert "format" in eng.last_error(), eng.last_error()
        eng.close()


def test_swapped_pair_members_refused(converted, tmp_path):
    bad, path = copy_out(converted, tmp_path)
    with open(path) as handle:
        doc = json.load(handle)
    doc["pairs"][0]["members"].reverse()
    with open(path, "w") as handle:
        json.dump(doc, handle, indent=2, sort_keys=True)
    assert any("members" in p for p in convert.verify(path))
    eng = w4a16.Engine(len(LAYER_FFNS), H, I, dense=[f == "dense" for f in LAYER_FFNS])
    assert eng.load_quantized_ffn(bad) == w4a16.W4A16_ERR_WEIGHTS
    assert "[mlpGate, mlpUp]" in eng.last_error(), eng.last_error()
    eng.close()


def test_changed_source_refused(converted, tmp_path):
    root, model, desc, out, _, _ = converted
    src = str(tmp_path / "model")
    shutil.copytree(model, src)
    dst = str(tmp_path / "int4")
    convert.convert_checkpoint(src, desc, dst)
    path = os.path.join(dst, "weights.manifest.json")
    assert convert.verify(path) == []
    with open(os.path.join(src, "model-00002.safetensors"), "r+b") as handle:
        handle.seek(-3, os.SEEK_END)
        handle.write(b"\x01\x02\x03")
    assert any("source checkpoint" in p for p in convert.verify(path))


def test_bad_checkpoints_refused(tmp_path):
    model, desc, _ = make_checkpoint(str(tmp_path / "f16"), fp16_role="up")
    with pytest.raises(convert.ConvertError, match="BF16"):
        convert.convert_checkpoint(model, desc, str(tmp_path / "o1"))
    model, desc, _ = make_checkpoint(str(tmp_path / "dup"), duplicate=True)
    with pytest.raises(convert.ConvertError, match="stored by two shards"):
        convert.convert_checkpoint(model, desc, str(tmp_path / "o2"))
    model, desc, _ = make_checkpoint(str(tmp_path / "missing"))
    os.remove(os.path.join(model, "model-00001.safetensors"))
    with pytest.raises(convert.ConvertError, match="not in the checkpoint"):
        convert.convert_checkpoint(model, desc, str(tmp_path / "o3"))


def test_sha256_file_in_blocks(tmp_path):
    import hashlib

    data = np.random.default_rng(3).integers(0, 256, 3 * (1 << 20) + 17, dtype=np.uint8).tobytes()
    p = tmp_path / "blob"
    p.write_bytes(data)
    assert convert.sha256_file(str(p), block=1 << 16) == hashlib.sha256(data).hexdigest()


def test_audit_finds_table_mutants(converted, tmp_path):
    """Mutants that pass the file pass (digests rewritten to match) and are caught by the table
    pass: a pair whose payload is up rows then gate rows, a precision cell listed twice, a cell
    dropped from the descriptor's grid, and an entry listed twice."""
    bad, path = copy_out(converted, tmp_path)
    with open(path) as handle:
        doc = json.load(handle)
    pair = doc["pairs"][0]
    members = {e["role"]: e for e in doc["entries"] if e["layer"] == pair["layer"]}
    swapped = b"".join(open(os.path.join(bad, members[r]["packed"]["file"]), "rb").read()
                       for r in ("mlpUp", "mlpGate"))
    with open(os.path.join(bad, pair["packed"]["file"]), "wb") as handle:
        handle.write(swapped)
    pair["packed"]["sha256"] = convert.sha256_file(os.path.join(bad, pair["packed"]["file"]))
    doc["precision_map"].append(dict(doc["precision_map"][0]))
    dropped = doc["precision_map"].pop(3)
    doc["entries"].append(dict(doc["entries"][1]))
    with open(path, "w") as handle:
        json.dump(doc, handle, indent=2, sort_keys=True)
    found = convert.verify(path)
    assert any("not the gate rows followed by the up rows" in f for f in found), found
    assert any("occurs 2 times" in f for f in found), found
    assert any(f"no cell for the descriptor's layer {dropped['layer']} {dropped['role']}" in f
               for f in found), found
    assert any("more than one entry" in f for f in found), found
    assert not any("content hash" in f for f in found), found
