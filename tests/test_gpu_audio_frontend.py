"""SHIELD-A from PCM on the GPU (shv_hip_audio_predict / _predict_device / _frontend) against the reference engine
compiled from its own sources (oracle/_ref/libshield_a_ref.so, exact mode) and its golden fixture
(tests/golden/audio_frontend_golden.json), in every tier.

  mel      : the log-mel image of window 0 (dump "mel", the reference's [80][997] layout) within MEL_TOL of the
             reference's dump -- the FFT, power spectrum and filterbank chains perform the reference's operations in its
             order, so only the device logf differs (an ulp or two).
  tokens   : the frontend's tokens within TOKEN_REL_TOL[tier] of the largest reference token (the 1x1 layers run on the
             tier's matrix cores with BatchNorm folded into their weights, the reference on its CPU GEMM: the order
             and rounding of those sums differ).
  logits   : PCM -> logit within LOGIT_TOL[tier] of the reference's, 0 decision flips.
  entries  : the device entry bitwise equal to the host entry (graph capture, then replay); 20 windows in host
             batches of 8 through chunks of the frontend bitwise equal to window-by-window calls; PCM that is not
             finite or outside [-1, 1] rejected with NaN logits; a sequence-only weight file refuses PCM.
"""
import tempfile
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MEL_TOL = 2e-5
# every tier within the bound of the sequence stages alone (1e-4): measured 3.6e-6 / 4.6e-6 / 5.6e-6 (tokens) and
# 7.6e-6 / 9.9e-6 / 1.4e-5 (logits) for fp32 / fp16 / bf16
TOKEN_REL_TOL = {"fp32": 1e-4, "fp16": 1e-4, "bf16": 1e-4}
LOGIT_TOL = {"fp32": 1e-4, "fp16": 1e-4, "bf16": 1e-4}
N_WINDOWS = 6


@pytest.fixture(scope="module")
def model_weights(shv, tmp_path_factory):
    p = tmp_path_factory.mktemp("agpu") / "audio_model.shlda"
    shv.write_audio_model_weights(p, 5)
    return p


@pytest.fixture(scope="module")
def pcm(shv):
    return shv.audio_pcm(N_WINDOWS, 23)


@pytest.fixture(scope="module")
def aref(orc, model_weights):
    if not orc.AUDIO_SO.exists():
        pytest.skip("the reference audio engine (oracle/_ref) is not built")
    r = orc.AudioReference(model_weights)
    yield r
    r.close()


@pytest.fixture(scope="module")
def ref_out(aref, pcm):
    print(f"[gpu] reference SHIELD-A engine on {N_WINDOWS} PCM windows", flush=True)
    with tempfile.TemporaryDirectory() as d:
        tok0 = aref.frontend(pcm[0], d)
        mel0 = np.fromfile(Path(d) / "mel.f32", np.float32)
    toks = np.stack([tok0] + [aref.frontend(pcm[w]) for w in range(1, N_WINDOWS)])
    return {"mel0": mel0, "tokens": toks, "logits": aref.predict(pcm)}


def flips(a, b):
    return int(((np.asarray(a) >= 0) != (np.asarray(b) >= 0)).sum())


@pytest.mark.parametrize("mode", ["fp32", "fp16", "bf16"])
def test_audio_pcm_to_logit(shv, model_weights, pcm, ref_out, mode, margin):
    print(f"[gpu] audio {mode}: PCM -> mel, tokens, logits ({N_WINDOWS} windows)", flush=True)
    with shv.AudioModel(model_weights, mode, max_windows=8, experimental=mode != "fp32") as m:
        assert m.has_frontend
        with tempfile.TemporaryDirectory() as d:
            m.set_dump_dir(d)
            m.frontend(pcm[:1])
            m.set_dump_dir("")
            mel0 = np.fromfile(Path(d) / "mel.f32", np.float32)
        toks = m.frontend(pcm)
        lg = m.predict(pcm)
    dm = float(np.abs(mel0 - ref_out["mel0"]).max())
    scale = float(np.abs(ref_out["tokens"]).max())
    dt = float(np.abs(toks - ref_out["tokens"]).max()) / scale
    dl = float(np.abs(lg - ref_out["logits"]).max())
    nf = flips(lg, ref_out["logits"])
    print(f"[gpu] audio {mode}: mel max|d| {dm:.3e}, tokens max|d|/max|token| {dt:.3e}, logits max|d| {dl:.3e}, "
          f"flips {nf}", flush=True)
    margin(f"audio {mode} log-mel (window 0) vs reference", dm, MEL_TOL)
    margin(f"audio {mode} frontend tokens vs reference (relative)", dt, TOKEN_REL_TOL[mode])
    margin(f"audio {mode} PCM -> logit vs reference", dl, LOGIT_TOL[mode])
    assert np.all(np.isfinite(toks)) and np.all(np.isfinite(lg))
    assert dm <= MEL_TOL
    assert dt <= TOKEN_REL_TOL[mode]
    assert dl <= LOGIT_TOL[mode] and nf == 0


def test_audio_golden_windows(shv, model_weights, pcm):
    """The fixture's three windows: tokens and logits against the stored reference values (no compiled reference
    needed)."""
    import json
    root = Path(__file__).resolve().parents[1]
    g = json.loads((root / "tests" / "golden" / "audio_frontend_golden.json").read_text())
    assert shv.sha256_bytes(shv.audio_pcm(g["windows"], g["pcm_seed"])) == g["pcm_sha256"]
    print("[gpu] audio fp32: golden PCM windows", flush=True)
    with shv.AudioModel(model_weights, "fp32", max_windows=8) as m:
        toks = m.frontend(pcm[:g["windows"]])
        lg = m.predict(pcm[:g["windows"]])
    for w, pw in enumerate(g["per_window"]):
        sample = toks[w].reshape(-1)[::g["token_step"]]
        scale = float(np.abs(toks[w]).max())
        assert np.abs(sample - np.array(pw["token_sample"])).max() <= TOKEN_REL_TOL["fp32"] * scale
        assert abs(float(lg[w]) - pw["logit"]) <= LOGIT_TOL["fp32"]


def test_audio_device_entry_and_batching(shv, model_weights, pcm):
    print("[gpu] audio fp32: predict_device vs predict, host batches vs single windows", flush=True)
    many = np.concatenate([pcm, pcm, pcm, pcm[:2]])   # 20 windows: more than one frontend chunk and host batch
    hip = shv.Hip()
    with shv.AudioModel(model_weights, "fp32", max_windows=8) as m:
        host = m.predict(pcm)
        d_pcm = hip.upload(pcm)
        d_lg = hip.malloc(N_WINDOWS * 4)
        s = hip.stream()
        try:
            runs = []
            for _ in range(2):   # graph capture, then replay
                hip.memset(d_lg, 0xFF, N_WINDOWS * 4)
                m.predict_device(d_pcm, N_WINDOWS, d_lg, stream=s)
                hip.stream_sync(s)
                runs.append(hip.download(d_lg, N_WINDOWS, np.float32))
        finally:
            hip.stream_destroy(s)
            hip.free(d_pcm)
            hip.free(d_lg)
        batched = m.predict(many)
        single = np.concatenate([m.predict(pcm[w:w + 1]) for w in range(N_WINDOWS)])
    for r in runs:
        assert np.array_equal(r.view(np.uint32), host.view(np.uint32))
    assert np.array_equal(single.view(np.uint32), host.view(np.uint32))
    assert np.array_equal(batched.view(np.uint32), np.concatenate([host, host, host, host[:2]]).view(np.uint32))


def test_audio_pcm_checks(shv, model_weights, pcm, tmp_path):
    print("[gpu] audio: PCM range checks and a sequence-only weight file", flush=True)
    with shv.AudioModel(model_weights, "fp32", max_windows=4) as m:
        for bad in (np.nan, 1.5, -np.inf):
            x = pcm[:2].copy()
            x[1, 777] = bad
            out = np.zeros(2, np.float32)
            rc = m.lib.shv_hip_audio_predict(m.h, x.ctypes.data, 2, 160000, out.ctypes.data)
            assert rc != 0 and np.all(np.isnan(out))
            assert "[-1,1]" in m._err()
    seq_only = tmp_path / "seq.shlda"
    shv.write_audio_weights(seq_only, 5)
    with shv.AudioModel(seq_only, "fp32", max_windows=4) as m:
        assert not m.has_frontend
        with pytest.raises(shv.ShvError, match="frontend"):
            m.predict(pcm[:1])
