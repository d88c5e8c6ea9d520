"""The drop-in boundary on the CPU: the export list, and an engine that keeps its own
engine_load_quantized_ffn (reference csrc/include/engine.h:98) linked beside this library.

* libw4a16.so exports exactly the functions include/w4a16.h declares, nothing else.
* A stub engine library (tests/stub/engine_stub.c, the pattern of reference
  tests/generation_engine_stub.c) defines engine_load_quantized_ffn and engine_last_error, links
  against libw4a16.so and is loaded RTLD_GLOBAL before it, in a fresh process. Refused loads
  (a missing directory; the expert-parallel refusal of reference csrc/engine.cu:2231-2236) go
  stub -> w4a16_load_quantized_ffn and return ENGINE_ERR_WEIGHTS (-3) with the library's own
  reason, and the library never calls back into the stub's definitions.
"""

import os
import shutil
import subprocess
import sys

import pytest

import convert
import w4a16
from oracle import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = w4a16.LIB_PATH

CHILD = r'''
import ctypes, os, sys
stub = ctypes.CDLL(sys.argv[1], mode=os.RTLD_NOW | os.RTLD_GLOBAL)
lib = ctypes.CDLL(sys.argv[2])          # already mapped as the stub's dependency
sidecar = sys.argv[3].encode()

class Cfg(ctypes.Structure):
    _fields_ = [("num_layers", ctypes.c_int), ("layer_is_dense", ctypes.c_void_p),
                ("hidden", ctypes.c_int), ("intermediate", ctypes.c_int),
                ("tp_size", ctypes.c_int), ("tp_rank", ctypes.c_int), ("ep_size", ctypes.c_int),
                ("max_tokens", ctypes.c_int), ("int4_max_rows", ctypes.c_int)]

for f in (lib.w4a16_engine_create,):
    f.restype = ctypes.c_void_p
lib.w4a16_last_error.restype = ctypes.c_char_p
lib.engine_last_error.restype = ctypes.c_char_p
stub.engine_last_error.restype = ctypes.c_char_p
for f in (stub.engine_load_quantized_ffn, lib.engine_load_quantized_ffn,
          lib.w4a16_load_quantized_ffn):
    f.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
lib.w4a16_engine_destroy.argtypes = [ctypes.c_void_p]

def store(ep):
    cfg = Cfg(2, None, 256, 384, 1, 0, ep, 1, 0)
    h = lib.w4a16_engine_create(ctypes.byref(cfg))
    assert h, lib.w4a16_last_error()
    return h

reent = ctypes.c_int.in_dll(stub, "stub_reentries")
loads = ctypes.c_int.in_dll(stub, "stub_loads")
h = store(1)
print("missing", stub.engine_load_quantized_ffn(h, b"/nonexistent/int4"),
      lib.w4a16_last_error().decode())
h2 = store(2)
print("ep2", stub.engine_load_quantized_ffn(h2, sidecar), lib.w4a16_last_error().decode())
print("direct", lib.engine_load_quantized_ffn(h2, sidecar), lib.w4a16_last_error().decode())
print("prefixed", lib.w4a16_load_quantized_ffn(h2, sidecar))
print("errors", stub.engine_last_error().decode(), "|", lib.engine_last_error().decode())
print("counts", loads.value, reent.value)
lib.w4a16_engine_destroy(h)
lib.w4a16_engine_destroy(h2)
'''


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True,
                         text=True).stdout
    return sorted(line.split()[-1] for line in out.splitlines() if line.strip())


def test_exports_are_the_header():
    assert exported(LIB) == w4a16.header_symbols()


@pytest.fixture(scope="module")
def stub_engine(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not available")
    d = tmp_path_factory.mktemp("stub")
    so = str(d / "libengine_stub.so")
    libdir = os.path.dirname(LIB)
    subprocess.run(["gcc", "-shared", "-fPIC", "-O1", "-o", so,
                    os.path.join(HERE, "stub", "engine_stub.c"), "-L" + libdir, "-l:libw4a16.so",
                    "-Wl,-rpath," + libdir, "-Wl,--no-as-needed"], check=True)
    side = str(d / "sidecar")
    layers = {l: {"mlpGate": oracle.synth_weight(384, 256, 1000 + 3 * l),
                  "mlpUp": oracle.synth_weight(384, 256, 1001 + 3 * l),
                  "mlpDown": oracle.synth_weight(256, 384, 1002 + 3 * l)} for l in range(2)}
    convert.write_sidecar(side, layers, "/tmp/synthetic-model")
    return so, side


def test_engine_keeps_its_own_loader(stub_engine):
    so, side = stub_engine
    env = dict(os.environ)
    env["HIP_VISIBLE_DEVICES"] = env.get("HIP_VISIBLE_DEVICES", "")  # no GPU work is done
    res = subprocess.run([sys.executable, "-c", CHILD, so, LIB, side], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    lines = {ln.split(" ", 1)[0]: ln.split(" ", 1)[1] for ln in res.stdout.splitlines() if " " in ln}
    status, why = lines["missing"].split(" ", 1)
    assert int(status) == w4a16.W4A16_ERR_WEIGHTS and "cannot open" in why
    status, why = lines["ep2"].split(" ", 1)
    assert int(status) == w4a16.W4A16_ERR_WEIGHTS and "expert-parallel" in why
    status, why = lines["direct"].split(" ", 1)
    assert int(status) == w4a16.W4A16_ERR_WEIGHTS and "expert-parallel" in why
    assert int(lines["prefixed"]) == w4a16.W4A16_ERR_WEIGHTS
    stub_err, lib_err = lines["errors"].split(" | ")
    assert stub_err == "the stub engine's own error string"
    assert "expert-parallel" in lib_err        # the library's alias, not the stub's
    assert lines["counts"] == "2 0"            # two stub loads, no re-entry from the library


def test_int4_row_switch_refusals():
    """The routing switch on the host: int4_max_rows outside 0..min(16, max_tokens) is refused at
    create;
    a store routes one decode row by default (reference csrc/kernels/layers.cu:126) and refuses
    more rows before any device work; an unloaded layer is never routed."""
    with pytest.raises(w4a16.W4A16Error):
        w4a16.Engine(2, 256, 384, max_tokens=4, int4_max_rows=5)
    with pytest.raises(w4a16.W4A16Error):
        w4a16.Engine(2, 256, 384, max_tokens=4, int4_max_rows=-1)
    with pytest.raises(w4a16.W4A16Error, match="min\\(16"):   # the small-M kernels stop at 16
        w4a16.Engine(2, 256, 384, max_tokens=32, int4_max_rows=17)
    w4a16.Engine(2, 256, 384, max_tokens=32, int4_max_rows=16).close()
    eng = w4a16.Engine(2, 256, 384, max_tokens=16)
    assert not eng.routes_int4(0, 1) and not eng.routes_int4(0, 4, verify_rows=True)
    for tokens in (2, 4, 16):
        st = w4a16.lib.engine_ffn_forward(eng.handle, 0, None, None, tokens, None)
        assert st == w4a16.W4A16_ERR_CONFIG and "int4_max_rows" in w4a16.last_error()
    eng.close()
    eng = w4a16.Engine(2, 256, 384, max_tokens=16, int4_max_rows=8)
    st = w4a16.lib.engine_ffn_forward_norm(eng.handle, 0, None, None, 0, 1e-6, None, 9, None)
    assert st == w4a16.W4A16_ERR_CONFIG and "at most 8 rows" in w4a16.last_error()
    eng.close()
