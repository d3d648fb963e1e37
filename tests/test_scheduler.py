"""The batched API's host side (shield-sisa_amd/csrc/sched.cpp: request validation, FIFO coalescing, the token-slot
hazard rule, two-lane pipelining, NaN on failure and on non-finite logits, callback / job_free ordering, closing with
queued jobs, jobs outliving the model) on a CPU stub device, built with g++ under the thread sanitizer and under the
address + undefined-behaviour sanitizers.  A sanitizer report fails the run (TSan exits 66, ASan / UBSan abort).

The reference's fixed races this guards against: notify-while-holding the job mutex because job_free may delete the
job (engine/cuda/api.cu:194-203, 630-637), free-while-queued (api.cu:515-519), non-finite -> NaN (api.cu:334-338).
"""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = [ROOT / "tests" / "native" / "sched_check.cpp", ROOT / "shield-sisa_amd" / "csrc" / "sched.cpp"]


def _build_and_run(tmp_path, name, flags, scale):
    exe = tmp_path / name
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Wextra", "-Werror", *flags, "-I", str(ROOT / "include"),
           *map(str, SRC), "-o", str(exe), "-lpthread"]
    b = subprocess.run(cmd, capture_output=True, text=True)
    assert b.returncode == 0, b.stderr
    r = subprocess.run([str(exe), str(scale)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-6000:]
    assert "PASS: 0 failed checks" in r.stdout
    assert "WARNING" not in r.stderr and "ERROR" not in r.stderr, r.stderr[-6000:]


def test_scheduler_under_thread_sanitizer(tmp_path):
    _build_and_run(tmp_path, "sched_tsan", ["-fsanitize=thread"], 1)


def test_scheduler_under_address_sanitizer(tmp_path):
    _build_and_run(tmp_path, "sched_asan", ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"], 2)
