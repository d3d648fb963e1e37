"""Certification tool (shield-sisa_amd/certify.py): criteria, certificate file format, and the loader's acceptance
of what it writes.  The line format and the loader's rules mirror the reference's SHIELDV_CUDA_CERT_V2 contract
(engine/cuda/api.cu:423-461, bench/gpu_certify.sh:1-9)."""
import hashlib
import importlib.util
import shutil
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def cert(shv):
    spec = importlib.util.spec_from_file_location("shv_certify", ROOT / "shield-sisa_amd" / "certify.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["shv_certify"] = mod
    spec.loader.exec_module(mod)
    return mod


def _copy(weights, tmp_path):
    dst = tmp_path / "w.weights"
    shutil.copy(weights, dst)
    shutil.copy(str(weights) + ".json", str(dst) + ".json")
    return dst


def test_criteria(cert):
    exact = np.array([-1.5, -0.2, 0.05, 0.8, 1.9])
    ok = cert.evaluate(exact, exact + 3e-3, 0.5, 1e-2)
    assert ok["verdict"] == "PASS" and ok["flips"] == 0 and abs(ok["max_abs_dlogit"] - 3e-3) < 1e-12
    assert cert.evaluate(exact, exact + 2e-2, 0.5, 1e-2)["verdict"] == "FAIL"          # tolerance
    flipped = exact.copy()
    flipped[2] = -0.001                                                                 # sigmoid crosses 0.5
    r = cert.evaluate(exact, flipped, 0.5, 1.0)
    assert r["verdict"] == "FAIL" and r["flips"] == 1
    bad = exact.copy()
    bad[0] = np.nan
    assert cert.evaluate(exact, bad, 0.5, 1.0)["verdict"] == "FAIL"                    # every logit finite
    # the decision is sigmoid(logit) >= threshold in double precision: logit 0 sits exactly on threshold 0.5
    assert cert.decisions(np.array([0.0, -1e-12]), 0.5).tolist() == [True, False]


def test_certificate_merge(cert, tmp_path):
    p = tmp_path / "x.hip.cert"
    p.write_text("SHIELDV_HIP_CERT_V2\n"
                 "aaa fp16 hip-1 PASS a.json 0 threshold=0.5\n"      # same weights + revision + mode: replaced
                 "aaa bf16 hip-1 PASS b.json 0 threshold=0.5\n"      # another mode: kept
                 "aaa fp16 hip-0 PASS c.json 0 threshold=0.5\n"      # another revision: kept
                 "bbb fp16 hip-1 PASS d.json 0 threshold=0.5\n")     # other weights: kept
    new = cert.cert_line("aaa", "fp16", "hip-1", "n.json", "f" * 64, 0.37)
    lines = cert.merge_certificate(p, "aaa", "hip-1", {"fp16": new}).splitlines()
    assert lines[0] == "SHIELDV_HIP_CERT_V2"
    assert lines[1:] == ["aaa bf16 hip-1 PASS b.json 0 threshold=0.5", "aaa fp16 hip-0 PASS c.json 0 threshold=0.5",
                         "bbb fp16 hip-1 PASS d.json 0 threshold=0.5", new]
    assert new.endswith("threshold=0.37")
    p.write_text("SHIELDV_CUDA_CERT_V2\nzzz fp16 r PASS j 0 threshold=0.5\n")             # foreign header: replaced
    assert cert.merge_certificate(p, "aaa", "hip-1", {"fp16": new}).splitlines() == ["SHIELDV_HIP_CERT_V2", new]


def test_loader_accepts_written_line(shv, cert, weights, tmp_path):
    """A line written by the tool passes shv_hip_load's certificate check (which runs before the device is
    touched); without it the load stops at the check."""
    w = _copy(weights, tmp_path)
    with pytest.raises(shv.ShvError) as e:
        shv.Model(w, "fp16", max_frames=20, max_windows=1)
    assert "certificate" in str(e.value)
    import json
    thr = json.loads(Path(str(w) + ".json").read_text())["threshold"]
    sha = hashlib.sha256(w.read_bytes()).hexdigest()
    rev = shv.library().shv_hip_compute_revision().decode()
    Path(str(w) + ".hip.cert").write_text(
        cert.merge_certificate(Path(str(w) + ".hip.cert"), sha, rev,
                               {"fp16": cert.cert_line(sha, "fp16", rev, "w.json", "0" * 64, thr)}))
    try:
        shv.Model(w, "fp16", max_frames=20, max_windows=1).close()   # a GPU box loads it
    except shv.ShvError as err:                                        # no GPU: fails past the check
        assert "certificate" not in str(err) and "threshold" not in str(err), str(err)
    # the certificate covers fp16 only
    with pytest.raises(shv.ShvError) as e:
        shv.Model(w, "bf16", max_frames=20, max_windows=1)
    assert "has no PASS line" in str(e.value)


@pytest.mark.gpu
def test_certify_then_load(shv, cert, weights, tmp_path):
    print("[gpu] certify fp16 on 4 synthetic clips, then load through the checking library", flush=True)
    w = _copy(weights, tmp_path)
    clips = shv.synth_clips(4, 1000)
    res = cert.certify(w, ["fp16"], clips, 1e-2, 4, "test clips")
    assert res["fp16"]["verdict"] == "PASS", res["fp16"]
    text = Path(str(w) + ".hip.cert").read_text().splitlines()
    assert text[0] == "SHIELDV_HIP_CERT_V2" and len(text) == 2 and " fp16 " in text[1]
    with shv.Model(w, "fp16", max_frames=80, max_windows=4) as m, \
            shv.Model(w, "fp16", experimental=True, max_frames=80, max_windows=4) as mx:
        a, b = m.predict(clips), mx.predict(clips)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
