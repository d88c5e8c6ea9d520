#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ from the reference's own CPU code.

The reference's C format sources are compiled (not copied) into oracle/_ref/ by
``make -C oracle ref``; this script runs that build's ``quantization_format_test`` binary:

* ``--emit PATH`` writes the reference's canonical [8, 256] fixture (weights, packed bytes,
  BF16 scales, dequantized FP32 bits) -> ``emit_fixture.json`` (copied verbatim: it is data the
  reference's own tool produces);
* ``--quantize in.f32 out.packed out.scales N K`` quantizes seeded tensors -> the packed bytes
  and scales in ``quantize_vectors.npz``, together with the inputs (as BF16 bits: every synthetic
  weight is BF16-valued) and the reference's dequantization (``libref_format.so``'s
  ``linear_dequantize_int4``) as FP32 bits.

Cases: one 8-row tile at each distinct K of the path's configurations (2560, 9728, 5120, 17408,
8704) with BF16 ~N(0, 0.02) weights; the reference kernel gate's distribution
(tests/test_quantization_kernel.py:100-104: randn*0.05 times a per-group factor, RandomState(11))
at its two small shapes; and edge groups (all zero, a clipped extreme, exact ties).

Run from the repository root:  python tests/golden/make_golden.py
"""

import ctypes
import json
import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle  # noqa: E402  (test infrastructure: bf16 helpers and generators)

OUT = os.path.dirname(os.path.abspath(__file__))
REF = os.path.join(ROOT, "oracle", "_ref")


def ref_quantize(binary, weights, workdir, tag):
    n, k = weights.shape
    fin = os.path.join(workdir, tag + ".f32")
    fp = os.path.join(workdir, tag + ".packed")
    fs = os.path.join(workdir, tag + ".scales")
    np.ascontiguousarray(weights, np.float32).tofile(fin)
    subprocess.run([binary, "--quantize", fin, fp, fs, str(n), str(k)], check=True)
    return np.fromfile(fp, np.uint8).reshape(n, k // 2), np.fromfile(fs, np.uint16).reshape(n, -1)


def ref_dequantize(lib, packed, scales, n, k):
    class Layout(ctypes.Structure):
        _fields_ = [(f, ctypes.c_longlong) for f in
                    ("n", "k", "group", "packed_bytes", "scale_count")]

    lay = Layout()
    assert lib.linear_layout_init(ctypes.byref(lay), ctypes.c_longlong(n), ctypes.c_longlong(k),
                                  ctypes.c_longlong(128)) == 0
    out = np.zeros((n, k), np.float32)
    p = np.ascontiguousarray(packed)
    s = np.ascontiguousarray(scales)
    st = lib.linear_dequantize_int4(ctypes.byref(lay), ctypes.c_void_p(p.ctypes.data),
                                    ctypes.c_void_p(s.ctypes.data),
                                    ctypes.c_void_p(out.ctypes.data))
    assert st == 0, st
    return out


def edge_weights():
    w = np.zeros((8, 256), np.float32)
    w[0, :8] = [0.0, 1.0, -1.0, -7.0, 7.0, 3.0, -3.0, 2.0]          # hand bytes 0x10 0x9F 0x37 0x2D
    w[1, 0], w[1, 1] = 0.7000001, -0.7000001                        # clipped extremes
    w[2, :128] = np.linspace(-7.0, 7.0, 128, dtype=np.float32)      # scale 1, many exact ties
    w[2, 128:136] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 7.0]     # half-way cases, RNE
    w[3, :] = 1e-3                                                   # constant group
    w[4, ::2] = -0.02                                                # alternating signs
    w[4, 1::2] = 0.02
    return w                                                         # rows 5..7 all zero


def main():
    binary = os.path.join(REF, "quantization_format_test")
    lib_path = os.path.join(REF, "libref_format.so")
    if not (os.path.exists(binary) and os.path.exists(lib_path)):
        sys.exit("build the reference oracle first: make -C oracle ref")
    lib = ctypes.CDLL(lib_path)
    arrays = {}
    with tempfile.TemporaryDirectory() as work:
        subprocess.run([binary, "--emit", os.path.join(work, "emit.json")], check=True)
        shutil.copyfile(os.path.join(work, "emit.json"), os.path.join(OUT, "emit_fixture.json"))

        cases = []
        for i, k in enumerate((2560, 9728, 5120, 17408, 8704)):
            cases.append((f"cfgK{k}", oracle.synth_weight(8, k, seed=500 + i)))
        rng = np.random.RandomState(11)
        for n, k in ((256, 128), (1024, 256)):
            w = (rng.randn(n, k) * 0.05).astype(np.float32)
            w *= (1.0 + 0.5 * rng.rand(n, k // 128).astype(np.float32)).repeat(128, axis=1)
            cases.append((f"gate{n}x{k}", w))
        cases.append(("edge", edge_weights()))

        names = []
        for name, w in cases:
            n, k = w.shape
            packed, scales = ref_quantize(binary, w, work, name)
            deq = ref_dequantize(lib, packed, scales, n, k)
            if name.startswith("cfg"):
                # BF16-valued inputs: their top halves are the whole value.
                assert np.array_equal(oracle.bf16_to_f32(oracle.bf16_bits(w)), w)
                arrays[f"{name}_weights_bf16"] = oracle.bf16_bits(w)
            elif name == "edge":
                arrays[f"{name}_weights_f32bits"] = w.view(np.uint32)
            # The gate cases' inputs are not stored: numpy's legacy RandomState stream is frozen,
            # so the tests regenerate them from seed 11 in the order above.
            arrays[f"{name}_packed"] = packed
            arrays[f"{name}_scales"] = scales
            if not name.startswith("gate"):
                arrays[f"{name}_dequant_f32bits"] = deq.view(np.uint32)
            names.append(name)
        arrays["case_names"] = np.array(names)
    np.savez_compressed(os.path.join(OUT, "quantize_vectors.npz"), **arrays)
    with open(os.path.join(OUT, "README.json"), "w") as handle:
        json.dump({"source": "oracle/_ref/quantization_format_test (--emit, --quantize) and "
                             "oracle/_ref/libref_format.so linear_dequantize_int4",
                   "cases": names}, handle, indent=2)
    print("wrote", sorted(arrays))


if __name__ == "__main__":
    main()
