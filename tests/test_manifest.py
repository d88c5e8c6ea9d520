"""The sidecar path on the CPU: converter -> weights.manifest.json -> reader -> loader refusals.

* SHA-256 against hashlib and the FIPS 180-4 examples.
* A sidecar written by haskell-infer-demo_amd/convert.py is accepted by this library's reader
  and - when oracle/_ref is built - by the reference's own compiled reader (quant_manifest.c via
  libref_format.so, and the quant_manifest_test binary with --manifest/--root).
* The reference reader's refusal classes (reference tests/quant_manifest_test.c:300-380), restated
  as textual mutations of that sidecar: this reader must return the expected status, and the
  reference reader must return the same one.
* Artifact reads: size, dtype, digest and missing-file refusals (quant_manifest_test.c:384-460),
  cross-checked against the reference's quant_artifact_read.
* engine_load_quantized_ffn refusals that happen before any device work (reference
  csrc/engine.cu:2207-2428): null argument, expert parallelism, partial coverage, shape
  mismatch, a tensor-parallel split inside a group, a corrupted artifact.
"""

import ctypes
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

import convert
import w4a16
from oracle import oracle

H, I, LAYERS = 256, 384, 2


@pytest.fixture(scope="module")
def sidecar(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("sidecar"))
    layers = {}
    for layer in range(LAYERS):
        layers[layer] = {
            "mlpGate": oracle.synth_weight(I, H, 1000 + 3 * layer),
            "mlpUp": oracle.synth_weight(I, H, 1001 + 3 * layer),
            "mlpDown": oracle.synth_weight(H, I, 1002 + 3 * layer),
        }
    roles = ["embed", "inputNorm", "mlpGate", "mlpUp", "mlpDown"]
    convert.write_sidecar(out, layers, "/tmp/synthetic-model", role_names=roles)
    with open(os.path.join(out, "weights.manifest.json")) as handle:
        text = handle.read()
    return out, text, layers


def ref_lib():
    path = oracle.ref_binary("libref_format.so")
    return ctypes.CDLL(path) if path else None


def ref_parse(text):
    lib = ref_lib()
    buf = ctypes.create_string_buffer(8 << 20)          # struct QuantManifest is ~1 MiB
    err = ctypes.create_string_buffer(512)
    return lib.quant_manifest_parse(text.encode(), buf, err, 512)


# ---- SHA-256 -----------------------------------------------------------------------------------

def test_sha256_known_answers_and_hashlib():
    assert w4a16.sha256_hex(b"") == \
        "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    assert w4a16.sha256_hex(b"abc") == \
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    msg = b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq"
    assert w4a16.sha256_hex(msg) == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    rng = np.random.default_rng(1)
    for n in (1, 55, 56, 63, 64, 65, 127, 128, 1000, 70000):
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert w4a16.sha256_hex(data) == hashlib.sha256(data).hexdigest(), n


# ---- the converter's sidecar -------------------------------------------------------------------

def test_sidecar_accepted(sidecar):
    out, text, layers = sidecar
    st, entries, pairs = w4a16.manifest_check(text)
    assert (st, entries, pairs) == (0, 3 * LAYERS, LAYERS), w4a16.last_error()
    doc = json.loads(text)
    # the artifacts are the quantizer's bytes, and the pair is gate rows then up rows
    for e in doc["entries"]:
        w = layers[e["layer"]][e["role"]]
        p, s = oracle.quantize(w)
        with open(os.path.join(out, e["packed"]["file"]), "rb") as handle:
            assert handle.read() == p.tobytes()
        with open(os.path.join(out, e["scales"]["file"]), "rb") as handle:
            assert handle.read() == s.tobytes()
    for pair in doc["pairs"]:
        gp, _ = oracle.quantize(layers[pair["layer"]]["mlpGate"])
        upk, _ = oracle.quantize(layers[pair["layer"]]["mlpUp"])
        with open(os.path.join(out, pair["packed"]["file"]), "rb") as handle:
            assert handle.read() == gp.tobytes() + upk.tobytes()


@pytest.mark.skipif(oracle.ref_binary("libref_format.so") is None, reason="oracle/_ref not built")
def test_sidecar_accepted_by_reference_reader(sidecar):
    out, text, _ = sidecar
    assert ref_parse(text) == 0
    binary = oracle.ref_binary("quant_manifest_test")
    proc = subprocess.run([binary, "--manifest", os.path.join(out, "weights.manifest.json"),
                           "--root", out], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "verified" in proc.stdout


def _mutants(text):
    """(label, mutated text, expected status) - the reference reader's refusal classes."""
    doc = json.loads(text)
    gate = [e for e in doc["entries"] if e["role"] == "mlpGate" and e["layer"] == 0][0]
    shape = '"logical_shape": [\n        %d,\n        %d\n      ]' % tuple(gate["logical_shape"])
    bad_k = '"logical_shape": [\n        %d,\n        %d\n      ]' % (gate["logical_shape"][0], 192)
    pshape = '"logical_shape": [\n        %d,\n        %d\n      ]' % tuple(doc["pairs"][0]["logical_shape"])
    pshape_bad = '"logical_shape": [\n        %d,\n        %d\n      ]' % (
        doc["pairs"][0]["logical_shape"][0] - 1, doc["pairs"][0]["logical_shape"][1])
    gate_bytes = '"bytes": %d' % gate["packed"]["bytes"]
    gate_count = '"count": %d' % gate["scales"]["count"]
    digest = gate["packed"]["sha256"]
    cases = [
        ("a version this reader does not speak", '"manifest_version": 1', '"manifest_version": 2', 3),
        ("a qmin that is not the frozen one", '"qmin": -7', '"qmin": -6', 3),
        ("a foreign group", '"group": 128,\n      "group_axis"', '"group": 64,\n      "group_axis"', 4),
        ("a K that is not a whole number of groups", shape, bad_k, 4),
        ("a group axis that is not K", '"group_axis": "k"', '"group_axis": "n"', 3),
        ("packed bytes that disagree with the shape", gate_bytes, '"bytes": %d' % (gate["packed"]["bytes"] + 1), 4),
        ("a scale count that disagrees with the shape", gate_count, '"count": %d' % (gate["scales"]["count"] - 1), 4),
        ("a malformed digest", digest, "z" + digest[1:], 3),
        ("a packed dtype that is not u8", '"dtype": "u8"', '"dtype": "f16"', 3),
        ("an entry with no int4 precision cell", '"precision": "int4"', '"precision": "bf16"', 4),
        ("a pair whose rows are not its members'", pshape, pshape_bad, 4),
        ("a pair member that is not an entry", '"role": "mlpUp",\n          "role_index"',
         '"role": "mlpXx",\n          "role_index"', 4),
        ("a duplicate key", '"manifest_version": 1', '"manifest_version": 1,\n  "manifest_version": 1', 2),
        ("a missing required section", '"entries":', '"entries_x":', 2),
    ]
    out = []
    for label, needle, repl, want in cases:
        assert needle in text, f"anchor for {label!r} not found"
        out.append((label, text.replace(needle, repl, 1), want))
    out.append(("a truncated document", text[:-20], 2))
    out.append(("an empty document", "", 2))
    out.append(("a document that is not an object", "[]", 2))
    out.append(("a precision cell that is neither int4 nor bf16",
                text.replace('"precision": "bf16"', '"precision": "fp8"', 1), 3))
    return out


def test_refusals_match_the_reference_classes(sidecar):
    _, text, _ = sidecar
    have_ref = oracle.ref_binary("libref_format.so") is not None
    for label, mutant, want in _mutants(text):
        st, _, _ = w4a16.manifest_check(mutant)
        assert st == want, (label, st, w4a16.last_error())
        if have_ref:
            assert ref_parse(mutant) == want, (label, "reference reader disagrees")


def test_artifact_reads(tmp_path):
    root = str(tmp_path)
    payload = bytes((i * 7 + 1) & 0xFF for i in range(64))
    with open(os.path.join(root, "one.packed"), "wb") as handle:
        handle.write(payload)
    digest = hashlib.sha256(payload).hexdigest()
    assert w4a16.artifact_verify(root, "one.packed", "u8", 64, digest, "u8") == 0
    assert w4a16.artifact_verify(root, "one.packed", "u8", 65, digest, "u8") == 5      # size
    assert w4a16.artifact_verify(root, "one.packed", "u8", 64, digest, "bf16") == 3    # dtype
    assert w4a16.artifact_verify(root, "two.packed", "u8", 64, digest, "u8") == 5      # missing
    bad = bytearray(payload)
    bad[3] ^= 0xFF
    with open(os.path.join(root, "one.packed"), "wb") as handle:
        handle.write(bytes(bad))
    assert w4a16.artifact_verify(root, "one.packed", "u8", 64, digest, "u8") == 6      # hash
    assert "hashes to" in w4a16.last_error()
    lib = ref_lib()
    if lib is not None:
        class Art(ctypes.Structure):
            _fields_ = [("file", ctypes.c_char * 512), ("dtype", ctypes.c_char * 64),
                        ("bytes", ctypes.c_longlong), ("count", ctypes.c_longlong),
                        ("sha256", ctypes.c_char * 65)]
        art = Art(b"one.packed", b"u8", 64, -1, digest.encode())
        out, n = ctypes.c_void_p(), ctypes.c_size_t()
        err = ctypes.create_string_buffer(512)
        assert lib.quant_artifact_read(root.encode(), ctypes.byref(art), b"u8", ctypes.byref(out),
                                       ctypes.byref(n), err, 512) == 6


# ---- engine_load_quantized_ffn refusals before any device work ----------------------------------

def test_loader_refusals(sidecar, tmp_path):
    out, text, _ = sidecar
    import shutil

    assert w4a16.lib.engine_load_quantized_ffn(None, out.encode()) == w4a16.W4A16_ERR_CONFIG
    eng = w4a16.Engine(LAYERS, H, I, ep_size=2)
    assert eng.load_quantized_ffn(out) == w4a16.W4A16_ERR_WEIGHTS
    assert "expert-parallel" in eng.last_error()
    eng = w4a16.Engine(LAYERS + 1, H, I)
    assert eng.load_quantized_ffn(out) == w4a16.W4A16_ERR_WEIGHTS
    assert "covers 2 of 3" in eng.last_error()
    eng = w4a16.Engine(LAYERS, 2 * H, I)
    assert eng.load_quantized_ffn(out) == w4a16.W4A16_ERR_WEIGHTS
    assert "checkpoint" in eng.last_error()
    eng = w4a16.Engine(LAYERS, H, I, tp_size=3, tp_rank=1)       # 128-wide slices: allowed
    eng = w4a16.Engine(LAYERS, H, I, tp_size=2, tp_rank=0)       # 192-wide slices: inside a group
    assert eng.load_quantized_ffn(out) == w4a16.W4A16_ERR_WEIGHTS
    assert "group boundary" in eng.last_error()
    # a corrupted artifact byte
    bad = str(tmp_path / "bad")
    shutil.copytree(out, bad)
    doc = json.loads(text)
    victim = os.path.join(bad, doc["pairs"][0]["packed"]["file"])
    with open(victim, "r+b") as handle:
        handle.seek(17)
        b = handle.read(1)
        handle.seek(17)
        handle.write(bytes([b[0] ^ 0x40]))
    eng = w4a16.Engine(LAYERS, H, I)
    assert eng.load_quantized_ffn(bad) == w4a16.W4A16_ERR_WEIGHTS
    assert "hashes to" in eng.last_error()
    assert eng.quantized_layers == 0                             # all-or-nothing
    # a tampered format block
    with open(os.path.join(bad, "weights.manifest.json"), "w") as handle:
        handle.write(text.replace('"qmax": 7', '"qmax": 8', 1))
    assert eng.load_quantized_ffn(bad) == w4a16.W4A16_ERR_WEIGHTS
    assert "frozen format" in eng.last_error()
    assert eng.load_quantized_ffn(str(tmp_path / "missing")) == w4a16.W4A16_ERR_WEIGHTS
