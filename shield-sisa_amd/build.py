"""Build the SHIELD-V HIP engine for gfx950 in-tree.

Outputs (shield-sisa_amd/lib/):
  libshield_v_hip.so               production library (approximate modes need a certificate)
  libshield_v_hip_experimental.so  same, without the certificate check (offline certification only)
  libshv_synth.so                  seeded synthetic weights / crops (host only, gcc)

The compute revision (shv_hip_compute_revision) is "hip-" + the first 16 hex digits of the SHA-256 over the
SHA-256 digests of the numeric sources, in a fixed order, followed by the build recipe that turns them into machine
code (target architecture, compiler path and version, every flag and the per-source flag choices), so a change to
kernel or layout code, to a flag or to the compiler invalidates certificates (the reference hashes its CUDA sources
and its CMakeLists.txt: engine/cuda/gen_revision.cmake:1-17, engine/cuda/CMakeLists.txt:20-25).
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_obj"
LIB = PKG / "lib"
INCLUDE = PKG.parent / "include"

NUMERIC_SOURCES = ["dev_common.hpp", "mfma.hpp", "kernels.hpp", "gemm.hip", "cnn.hip", "fused.hip", "strip.hip", "seq.hip",
                   "engine.hpp", "engine.hip", "stack.hpp", "audio.hpp", "audio.hip", "afront.hip",
                   "host_model.hpp", "host_model.cpp"]
DEVICE_SOURCES = ["gemm.hip", "cnn.hip", "fused.hip", "strip.hip", "seq.hip", "engine.hip", "audio.hip", "afront.hip",
                  "crop.hip"]
HOST_SOURCES = ["host_model.cpp", "sched.cpp", "cert.cpp"]
HIP_HOST_SOURCES = ["lanes.cpp"]          # host code that calls the HIP runtime
API_SOURCE = "capi.cpp"                   # built twice: certified and experimental
C_SOURCES = ["sha256.c"]

ARCH = os.environ.get("SHV_HIP_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-fPIC", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-fvisibility=hidden",
          "-Wall", "-Wno-unused-function", "-Wno-unused-result"]
# no packed-fp32 instructions anywhere in the device code
DEVICE_FLAGS = ["--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# MFMA accumulators in ordinary VGPRs instead of AGPRs (the unified register file holds them either way; the AGPR
# form adds v_accvgpr moves around every accumulation chain and costs registers).  Only for sources where no inline
# asm reads an MFMA result: the compiler inserts the MFMA-to-VALU wait states for its own instructions but not for
# an asm operand, and an empty asm is counted as one wait state.  In these two files every asm operand is a loaded
# value or a VALU result; tests/test_mfma_asm_hazard.py checks that on the built code objects (no inline-asm DPP
# instruction reads a VGPR that an MFMA write can reach).
VGPR_FORM_SOURCES = {"strip.hip", "gemm.hip"}
VGPR_FORM_FLAGS = ["-mllvm", "-amdgpu-mfma-vgpr-form"]


def _compiler_version() -> str:
    try:
        r = subprocess.run([HIPCC, "--version"], capture_output=True, text=True, timeout=60)
        return r.stdout.strip()
    except (OSError, subprocess.SubprocessError):
        return "unknown"


def recipe() -> str:
    """The part of the build that decides the numerics besides the sources: one canonical text."""
    lines = ["arch=" + ARCH, "hipcc=" + HIPCC, "compiler=" + _compiler_version(), "common=" + " ".join(COMMON),
             "device=" + " ".join(DEVICE_FLAGS)]
    for src in DEVICE_SOURCES:
        extra = VGPR_FORM_FLAGS if src in VGPR_FORM_SOURCES else []
        lines.append(f"{src}: " + " ".join(extra))
    return "\n".join(lines)


def revision() -> str:
    h = hashlib.sha256()
    for name in NUMERIC_SOURCES:
        h.update(hashlib.sha256((CSRC / name).read_bytes()).hexdigest().encode())
    h.update(hashlib.sha256(recipe().encode()).hexdigest().encode())
    return "hip-" + h.hexdigest()[:16]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)


def build(verbose: bool = False) -> dict:
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    rev = revision()
    revdef = f'-DSHV_HIP_REVISION="{rev}"'
    jobs: list[list[str]] = []
    objs: list[Path] = []
    for src in DEVICE_SOURCES:
        o = OBJ / (src + ".o")
        extra = VGPR_FORM_FLAGS if src in VGPR_FORM_SOURCES else []
        jobs.append([HIPCC, *COMMON, *DEVICE_FLAGS, *extra, "-c", str(CSRC / src), "-o", str(o)])
        objs.append(o)
    for src in HOST_SOURCES:
        o = OBJ / (src + ".o")
        jobs.append([HIPCC, *COMMON, "-x", "c++", "-c", str(CSRC / src), "-o", str(o)])
        objs.append(o)
    for src in C_SOURCES:
        o = OBJ / (src + ".o")
        jobs.append(["gcc", "-O2", "-fPIC", "-fvisibility=hidden", "-c", str(CSRC / src), "-o", str(o)])
        objs.append(o)
    host_hip = ["-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include", "-I", str(INCLUDE), revdef]
    for src in HIP_HOST_SOURCES:
        o = OBJ / (src + ".o")
        jobs.append([HIPCC, *COMMON, *host_hip, "-c", str(CSRC / src), "-o", str(o)])
        objs.append(o)
    api = OBJ / "capi.cpp.o"
    api_exp = OBJ / "capi_experimental.cpp.o"
    jobs.append([HIPCC, *COMMON, *host_hip, "-c", str(CSRC / API_SOURCE), "-o", str(api)])
    jobs.append([HIPCC, *COMMON, *host_hip, "-DSHV_HIP_EXPERIMENTAL=1", "-c", str(CSRC / API_SOURCE), "-o",
                 str(api_exp)])
    synth = LIB / "libshv_synth.so"
    jobs.append(["gcc", "-O2", "-fPIC", "-shared", "-fvisibility=hidden", "-o", str(synth) + ".tmp",
                 str(CSRC / "synth.c"), str(CSRC / "sha256.c")])
    workers = int(os.environ.get("MAX_JOBS", "8"))
    with ThreadPoolExecutor(max_workers=max(1, min(workers, 16))) as ex:
        list(ex.map(_run, jobs))
    os.replace(str(synth) + ".tmp", synth)
    outs = {}
    for name, apio in (("libshield_v_hip.so", api), ("libshield_v_hip_experimental.so", api_exp)):
        out = LIB / name
        _run([HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", str(out) + ".tmp", str(apio),
              *[str(o) for o in objs], "-lpthread"])
        os.replace(str(out) + ".tmp", out)
        outs[name] = str(out)
    outs["libshv_synth.so"] = str(synth)
    outs["revision"] = rev
    if verbose:
        print(outs)
    return outs


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
