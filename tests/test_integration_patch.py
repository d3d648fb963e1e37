"""The libshield_av "hip" video backend (shield-sisa_amd/integration/shield_av_hip.patch): the patch applies to the
reference service (service/src/shield_av.cpp, service/include/shield_av.h), the patched translation unit compiles
against the reference's own headers and include/shv_hip.h (compile only: nothing of the reference is built or run),
and every shv_hip_* function it calls is exported by libshield_v_hip.so.  The selector sites it changes:
shield_av.cpp:160 (backend 3), 192-217 (pinned crop pool), 540-611 (submit + completion), 806-869 (selector and
load), 880 (completion thread), 907-909 (teardown), 962 (video_predict), 1013 (device token slots)."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = Path("/root/reference")
PATCH = ROOT / "shield-sisa_amd" / "integration" / "shield_av_hip.patch"

pytestmark = pytest.mark.skipif(not (REF / "service" / "src" / "shield_av.cpp").exists(),
                                reason="the reference tree is not present")


def exported(lib: Path) -> set:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.split()}


def test_hip_selector_patch_applies_and_compiles(tmp_path, shv):
    shv.library()   # built
    work = tmp_path / "ref"
    shutil.copytree(REF / "service", work / "service")
    r = subprocess.run(["patch", "-p1", "-d", str(work), "-i", str(PATCH)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    src = work / "service" / "src" / "shield_av.cpp"
    text = src.read_text()
    assert 'backend != "hip"' in text and "shv_hip_load_ex" in text
    obj = tmp_path / "shield_av.o"
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-c", "-o", str(obj),
                        "-I", str(work / "service" / "include"), "-I", str(REF / "engine" / "audio" / "include"),
                        "-I", str(REF / "engine" / "include"), "-I", str(ROOT / "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    # the HIP entry points the object needs, and the library's exports
    und = subprocess.run(["nm", "-u", str(obj)], capture_output=True, text=True, check=True).stdout
    needed = {s for s in re.findall(r"\b(shv_hip_\w+)", und)}
    called = set(re.findall(r"\b(shv_hip_\w+)\s*\(", text))
    assert called and called <= needed | {"shv_hip_default_options"}
    assert needed <= exported(ROOT / "shield-sisa_amd" / "lib" / "libshield_v_hip.so"), needed
    # the unpatched service keeps compiling without the HIP header (the patch is the only change)
    assert "shv_hip" not in (REF / "service" / "src" / "shield_av.cpp").read_text()
