"""The kernels that stage activation rows into LDS by direct-to-LDS buffer loads wait for them
with a count-based s_waitcnt: "at most N vector memory operations outstanding", N being the
weight and scale loads issued after the staging loads. That is only right if those N loads are
really issued between the staging loads and the wait; if the compiler sinks some of them past
the wait (into the branch that uses them), the wait no longer covers the staging and the first
LDS reads can see stale data (a race that shows up as wrong results only now and then).

This CPU test compiles the kernels to gfx950 assembly and checks, for every kernel that issues
such loads, that before its first LDS read some vmcnt wait allows no more outstanding operations
than were issued after the last staging load (a straight-line scan of the listing).

The same listing also guards the load order of the streaming kernels: loads complete in issue
order, so every 2-byte scale load has to be issued before the first weight piece (the
non-temporal 16-byte loads); issued after them, the first pair's scale multiply waits for the
wave's whole weight stream."""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "haskell-infer-demo_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def uncovered_kernels(asm):
    bad = []
    for m in re.finditer(r"^(_Z\w+):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        body = [ln.strip() for ln in asm[m.end():end].split("\n")]
        body = [ln for ln in body if ln and not ln.startswith((";", "."))]
        if not any(ln.startswith("buffer_load") and " lds" in ln for ln in body):
            continue
        since, covered, seen = 0, False, False
        for ln in body:
            if ln.startswith(("buffer_load", "global_load")):
                if " lds" in ln:
                    seen, since, covered = True, 0, False
                else:
                    since += 1
            elif seen and ln.startswith("s_waitcnt") and "vmcnt" in ln:
                covered |= int(re.search(r"vmcnt\((\d+)\)", ln).group(1)) <= since
            elif seen and ln.startswith("ds_read"):
                break
        if not covered:
            bad.append(m.group(1))
    return bad


STREAMING = re.compile(r"gemv_(xwave|mfma1|tiles|rows16x?)_kernel|mfma_gemm_kernel")


def late_scale_kernels(asm):
    """Streaming kernels in which a scale load (buffer_load_ushort) follows a weight load."""
    bad, seen = [], 0
    for m in re.finditer(r"^(_Z\w+):", asm, re.M):
        if not STREAMING.search(m.group(1)):
            continue
        end = asm.find(".Lfunc_end", m.end())
        body = [ln.strip() for ln in asm[m.end():end].split("\n")]
        weights = [i for i, ln in enumerate(body)
                   if ln.startswith("buffer_load_dwordx4") and ln.endswith(" nt")]
        scales = [i for i, ln in enumerate(body) if ln.startswith("buffer_load_ushort")]
        if not weights:
            continue
        seen += 1
        if not scales or max(scales) > weights[0]:
            bad.append(m.group(1))
    return seen, bad


@pytest.fixture(scope="module")
def kernels_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc is not installed")
    out = tmp_path_factory.mktemp("asm") / "kernels.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-kernarg-preload-count=16", "-mllvm",
           "-amdgpu-sched-strategy=max-ilp", "-I", CSRC, "--cuda-device-only", "-S",
           os.path.join(CSRC, "kernels.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


def test_staging_waits_cover_the_direct_loads(kernels_asm):
    assert "lds" in kernels_asm  # the staging kernels are there
    assert uncovered_kernels(kernels_asm) == []


def test_scales_are_issued_before_the_weights(kernels_asm):
    seen, bad = late_scale_kernels(kernels_asm)
    assert seen > 50  # every instantiation of the streaming kernels is checked
    assert bad == []


def test_the_order_check_finds_a_late_scale():
    listing = """_ZN12_GLOBAL__N_117gemv_xwave_kernelIbad:
    buffer_load_dwordx4 v[2:5], v6, s[4:7], 0 offen nt
    buffer_load_ushort v7, v8, s[8:11], 0 offen
.Lfunc_end0:
_ZN12_GLOBAL__N_117gemv_mfma1_kernelIok:
    buffer_load_ushort v7, v8, s[8:11], 0 offen
    buffer_load_dwordx4 v[2:5], v6, s[4:7], 0 offen nt
.Lfunc_end1:
"""
    assert late_scale_kernels(listing) == (2, ["_ZN12_GLOBAL__N_117gemv_xwave_kernelIbad"])


def test_the_check_finds_an_uncovered_wait():
    listing = """_Zk:
    buffer_load_dwordx4 v1, s[0:3], 0 offen lds
    buffer_load_dwordx4 v[2:5], v6, s[4:7], 0 offen
    s_waitcnt vmcnt(2)
    ds_read_b128 v[8:11], v12
.Lfunc_end0:
_Zok:
    buffer_load_dwordx4 v1, s[0:3], 0 offen lds
    buffer_load_dwordx4 v[2:5], v6, s[4:7], 0 offen
    buffer_load_dwordx4 v[2:5], v6, s[4:7], 0 offen
    s_waitcnt vmcnt(2)
    ds_read_b128 v[8:11], v12
.Lfunc_end1:
"""
    assert uncovered_kernels(listing) == ["_Zk"]
