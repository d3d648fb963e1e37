"""The C-ABI boundary (include/shv_hip.h) on the CPU: every declared symbol is exported, defaults and revision
match the contract, and every load-time validation that precedes device work fails with the reference's
messages (engine/cuda/model.cpp:137-179, engine/cuda/api.cu:397-499)."""
import re
import shutil
import struct
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "shv_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(shv_hip_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(shv):
    lib = shv.library()
    names = declared_functions()
    assert len(names) == 52
    for n in names:
        assert hasattr(lib, n), n
    exp = shv.library(experimental=True)
    for n in names:
        assert hasattr(exp, n), n


def test_defaults_and_revision(shv):
    o = shv.default_options()
    assert (o.max_frames, o.max_windows, o.max_host_tokens, o.token_slots, o.use_graphs, o.max_delay_us) == \
        (640, 512, 2048, 0, 1, 0)
    rev = shv.library().shv_hip_compute_revision().decode()
    assert re.fullmatch(r"hip-[0-9a-f]{16}", rev)
    import importlib.util
    spec = importlib.util.spec_from_file_location("shv_build", ROOT / "shield-sisa_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    assert rev == b.revision(), "library built from other sources than the tree (rebuild)"


def load_err(shv, path, mode="fp32", **opts):
    with pytest.raises(shv.ShvError) as e:
        shv.Model(path, mode, **opts)
    return str(e.value)


def copy_weights(weights, tmp_path, name="w.weights"):
    dst = tmp_path / name
    shutil.copy(weights, dst)
    shutil.copy(str(weights) + ".json", str(dst) + ".json")
    return dst


def test_load_rejects_bad_files(shv, weights, tmp_path):
    assert "cannot open weights" in load_err(shv, tmp_path / "missing.weights")
    bad = tmp_path / "bad.weights"
    bad.write_bytes(b"NOTSHLDV" + b"\0" * 64)
    assert "not a SHLDV001 file" in load_err(shv, bad)
    data = Path(weights).read_bytes()
    trunc = tmp_path / "trunc.weights"
    trunc.write_bytes(data[: len(data) // 2])
    assert "truncated" in load_err(shv, trunc)
    trail = tmp_path / "trail.weights"
    trail.write_bytes(data + b"\0")
    assert "trailing data" in load_err(shv, trail)
    # first tensor's first value -> NaN (header: magic 8, count 4, name_len 4, name, rank 4, dims 4*rank, n 8)
    nl = struct.unpack_from("<I", data, 12)[0]
    rank = struct.unpack_from("<I", data, 16 + nl)[0]
    off = 16 + nl + 4 + 4 * rank + 8
    nan = bytearray(data)
    nan[off:off + 4] = struct.pack("<f", float("nan"))
    p = tmp_path / "nan.weights"
    p.write_bytes(bytes(nan))
    assert "non-finite" in load_err(shv, p)


def test_sidecar_rules(shv, weights, tmp_path):
    w = copy_weights(weights, tmp_path)
    side = Path(str(w) + ".json")
    text = side.read_text()
    side.write_text(text.replace('"output_sha256": "', '"output_sha256": "0'))
    assert "does not match the weights' SHA-256" in load_err(shv, w)
    side.write_text(re.sub(r'"output_sha256": "[0-9a-f]+"', '"x": 1', text))
    assert "no output_sha256" in load_err(shv, w)
    side.write_text(re.sub(r'"threshold": [0-9.e+-]+', '"threshold": 1.5', text))
    assert "threshold out of (0,1)" in load_err(shv, w)
    side.write_text(re.sub(r'"threshold": [0-9.e+-]+,', "", text))
    assert "no threshold" in load_err(shv, w)
    side.unlink()
    assert "cannot open" in load_err(shv, w)


def test_modes_and_certificates(shv, weights, tmp_path):
    w = copy_weights(weights, tmp_path)
    assert "unknown mode" in load_err(shv, w, "int8")
    assert "no certificate file at" in load_err(shv, w, "fp16")
    cert = Path(str(w) + ".hip.cert")
    cert.write_text("SHIELDV_CUDA_CERT_V2\n")
    assert "lacks the SHIELDV_HIP_CERT_V2 header" in load_err(shv, w, "bf16")
    sha = shv.write_weights(tmp_path / "other.weights", seed=2)
    rev = shv.library().shv_hip_compute_revision().decode()
    cert.write_text(f"SHIELDV_HIP_CERT_V2\n{sha} fp16 {rev} PASS c.json 0 threshold=0.5\n")
    assert "has no PASS line" in load_err(shv, w, "fp16")
    mine = Path(w).read_bytes()
    import hashlib
    msha = hashlib.sha256(mine).hexdigest()
    cert.write_text(f"SHIELDV_HIP_CERT_V2\n{msha} fp16 {rev} PASS c.json 0 threshold=0.25\n")
    assert "uncertified at this threshold" in load_err(shv, w, "fp16")
    cert.write_text(f"SHIELDV_HIP_CERT_V2\n{msha} fp16 hip-0000000000000000 PASS c.json 0 threshold=0.5\n")
    assert "has no PASS line" in load_err(shv, w, "fp16")


def test_invalid_options(shv, weights):
    assert "invalid options" in load_err(shv, weights, max_frames=0)
    assert "invalid options" in load_err(shv, weights, max_windows=5000)
    assert "invalid options" in load_err(shv, weights, token_slots=-1)


def test_null_arguments(shv):
    lib = shv.library()
    assert lib.shv_hip_load_ex(None, None, 0, None) is None
    assert "null weights path" in shv.last_error()
    assert lib.shv_hip_submit(None, None) is None
    assert lib.shv_hip_job_status(None) == -1
    assert lib.shv_hip_job_wait(None) == -1
    assert lib.shv_hip_limits(None, None, None, None, None) == -1
    assert np.isnan(lib.shv_hip_threshold(None))
    assert lib.shv_hip_mode(None) == b""
    lib.shv_hip_job_free(None)
    lib.shv_hip_free(None)


def test_gemm_tool_rejects_bad_arguments(shv):
    """The GEMM microbench entry points validate before any device work (NULL / -1 plus last_error)."""
    lib = shv.library()
    assert not lib.shv_hip_gemm_create(b"fp8", 16, 16, 1, None)
    assert "unknown mode" in shv.last_error()
    assert not lib.shv_hip_gemm_create(b"fp16", 16, 12, 1, None)
    assert "K % 8" in shv.last_error()
    assert not lib.shv_hip_gemm_create(b"fp32", 16, 16, None, None)
    assert "invalid argument" in shv.last_error()
    assert lib.shv_hip_gemm_run(None, 1, 1, None, 0, 1, 0, None) == -1
    assert "invalid argument" in shv.last_error()
    lib.shv_hip_gemm_free(None)
