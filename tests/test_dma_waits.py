"""The kernels that stage activation rows into LDS by direct-to-LDS buffer loads wait for them
with a count-based s_waitcnt: "at most N vector memory operations outstanding", N being the
weight and scale loads issued after the staging loads. That is only right if those N loads are
really issued between the staging loads and the wait; if the compiler sinks some of them past
the wait (into the branch that uses them), the wait no longer covers the staging and the first
LDS reads can see stale data (a race that shows up as wrong results only now and then).

This CPU test compiles the kernels to gfx950 assembly and checks, for every kernel that issues
such loads, that before its first LDS read some vmcnt wait allows no more outstanding operations
than were issued after the last staging load (a straight-line scan of the listing)."""

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


def test_staging_waits_cover_the_direct_loads(tmp_path):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc is not installed")
    out = tmp_path / "kernels.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-kernarg-preload-count=16", "-mllvm",
           "-amdgpu-sched-strategy=max-ilp", "-I", CSRC, "--cuda-device-only", "-S",
           os.path.join(CSRC, "kernels.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    asm = out.read_text()
    assert "lds" in asm  # the staging kernels are there
    assert uncovered_kernels(asm) == []


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
