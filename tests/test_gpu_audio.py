"""GPU parity of the SHIELD-A sequence stages (shv_hip_audio_*, through the C-ABI) against the reference engine's
golden fixture (tests/golden/audio_golden.json; the reference's exact mode, compiled from its own sources).

Bars, every tier (fp32: the reference's GEMM operand order with the device's elementwise functions; fp16 / bf16:
split-operand matrix cores with fp32-level operand precision):
  logits     : max |logit - reference| <= LOGIT_TOL on the 8 seeded windows
  stages     : relative L2 error of the dumped stage tensors (windows 0 and 5) <= STAGE_TOL; the assembled input
               (tokens + readout) bit for bit
  batching   : a window's logit is bitwise the same alone, in any batch, past max_windows, and from strided device
               memory
"""
import json
import tempfile
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
# the float64 restatement sits 6e-6 from the reference's fp32 logits: the fp32 rounding band of this model
LOGIT_TOL = 1e-4
STAGE_TOL = {"tokens": 0.0, "gdn_a": 1e-5, "gdn_b": 1e-5, "sisa_last": 5e-5}
MODES = ["fp32", "fp16", "bf16"]


@pytest.fixture(scope="module")
def agold():
    return json.loads((ROOT / "tests" / "golden" / "audio_golden.json").read_text())


@pytest.fixture(scope="module")
def aweights(tmp_path_factory, shv, agold):
    p = tmp_path_factory.mktemp("audio") / "seed5.shlda"
    assert shv.write_audio_weights(p, agold["weights_seed"]) == agold["weights_sha256"]
    return p


@pytest.fixture(scope="module")
def atokens(shv, agold):
    t = shv.audio_tokens(agold["windows"], agold["tokens_seed"])
    assert shv.sha256_bytes(t) == agold["tokens_sha256"]
    return t


@pytest.fixture(scope="module")
def models(shv, aweights):
    out = {}
    for mode in MODES:
        print(f"[gpu] audio load {mode}", flush=True)
        out[mode] = shv.AudioModel(aweights, mode, max_windows=8, experimental=mode != "fp32")
    yield out
    for m in out.values():
        m.close()


def gold_logits(agold):
    return np.array([int(b, 16) for b in agold["logit_bits"]], np.uint32).view(np.float32)


@pytest.mark.parametrize("mode", MODES)
def test_audio_logits(models, atokens, agold, mode, margin):
    print(f"[gpu] audio {mode} sequence of 8 windows", flush=True)
    got = models[mode].sequence(atokens)
    assert got.shape == (8,) and np.all(np.isfinite(got))
    d = float(np.abs(got.astype(np.float64) - gold_logits(agold)).max())
    margin(f"audio {mode} logits vs reference", d, LOGIT_TOL)
    assert d <= LOGIT_TOL, (got, gold_logits(agold))


@pytest.mark.parametrize("mode", MODES)
def test_audio_stages(models, atokens, agold, mode, margin):
    m = models[mode]
    step = agold["sample_step"]
    for w, gold in agold["stages"].items():
        with tempfile.TemporaryDirectory() as d:
            print(f"[gpu] audio {mode} stage dump window {w}", flush=True)
            m.set_dump_dir(d)
            try:
                m.sequence(atokens[int(w):int(w) + 1])
            finally:
                m.set_dump_dir("")
            for name, g in gold.items():
                a = np.fromfile(Path(d) / f"{name}.f32", np.float32)
                assert a.size == g["size"], name
                sample = (a if name == "sisa_last" else a[::step]).astype(np.float64)
                ref = np.array(g["sample"], np.float64)
                if name == "tokens":
                    assert np.array_equal(sample.astype(np.float32), ref.astype(np.float32))
                    continue
                e = float(np.linalg.norm(sample - ref) / np.linalg.norm(ref))
                margin(f"audio {mode} {name} (window {w}) rel L2", e, STAGE_TOL[name])
                assert e <= STAGE_TOL[name], (name, e)


@pytest.mark.parametrize("mode", ["fp32", "fp16"])
def test_audio_batch_independence(models, atokens, mode):
    m = models[mode]
    print(f"[gpu] audio {mode} batch independence", flush=True)
    full = m.sequence(atokens)
    for lo, hi in [(0, 1), (2, 5), (7, 8), (1, 8)]:
        part = m.sequence(atokens[lo:hi])
        assert np.array_equal(part.view(np.uint32), full[lo:hi].view(np.uint32)), (lo, hi)
    # 20 windows through a model of max_windows 8: three batches (8, 8, 4)
    idx = np.arange(20) % 8
    many = m.sequence(atokens[idx])
    assert np.array_equal(many.view(np.uint32), full[idx].view(np.uint32))


def test_audio_device_path_strided(shv, models, atokens):
    m = models["fp32"]
    hip = shv.Hip()
    stride = shv.AUDIO_WINDOW_FLOATS + 4
    padded = np.full((8, stride), np.nan, np.float32)
    padded[:, :shv.AUDIO_WINDOW_FLOATS] = atokens.reshape(8, -1)
    print("[gpu] audio device path, strided windows", flush=True)
    d_tok = hip.upload(padded)
    d_out = hip.malloc(8 * 4)
    try:
        m.sequence_device(d_tok, 8, d_out, stride=stride)
        hip.sync()
        got = hip.download(d_out, (8,), np.float32)
        host = m.sequence(padded.reshape(-1), stride=stride)
    finally:
        hip.free(d_tok)
        hip.free(d_out)
    full = m.sequence(atokens)
    assert np.array_equal(got.view(np.uint32), full.view(np.uint32))
    assert np.array_equal(host.view(np.uint32), full.view(np.uint32))


@pytest.mark.parametrize("mode", ["fp32", "fp16"])
def test_audio_calls_ordered_across_streams(shv, models, atokens, agold, mode):
    """Calls of one handle share its activation buffers.  A device call on a user stream returns before its kernels
    end; a host call issued at once, and a device call on a second stream, must still run after it: every result is
    bitwise the one of an isolated call (windows are independent rows, so the reversed batch is the reversed
    logits)."""
    m = models[mode]
    full = m.sequence(atokens)
    rev = np.ascontiguousarray(atokens[::-1])
    hip = shv.Hip()
    s1, s2 = hip.stream(), hip.stream()
    d_a, d_b = hip.upload(atokens), hip.upload(rev)
    d_oa, d_ob = hip.malloc(8 * 4), hip.malloc(8 * 4)
    try:
        for rep in range(3):
            print(f"[gpu] audio {mode} calls on two streams and the host path, round {rep}", flush=True)
            hip.memset(d_oa, 0xFF, 8 * 4)
            hip.memset(d_ob, 0xFF, 8 * 4)
            m.sequence_device(d_a, 8, d_oa, stream=s1)
            host = m.sequence(rev)
            m.sequence_device(d_b, 8, d_ob, stream=s2)
            hip.stream_sync(s1)
            hip.stream_sync(s2)
            ga = hip.download(d_oa, (8,), np.float32)
            gb = hip.download(d_ob, (8,), np.float32)
            assert np.array_equal(ga.view(np.uint32), full.view(np.uint32)), rep
            assert np.array_equal(host.view(np.uint32), full[::-1].view(np.uint32)), rep
            assert np.array_equal(gb.view(np.uint32), full[::-1].view(np.uint32)), rep
    finally:
        for b in (d_a, d_b, d_oa, d_ob):
            hip.free(b)
        hip.sync()
    assert float(np.max(np.abs(full - gold_logits(agold)))) <= LOGIT_TOL


@pytest.mark.parametrize("mode", ["fp16", "bf16"])
def test_audio_large_batches(shv, aweights, atokens, agold, mode, margin):
    """Past 16 windows per launch the chunked delta-rule scan takes 64-column value blocks and the sequence GEMMs
    larger-M tile plans: 40 windows in one launch (the golden windows repeated) give bitwise the logits of launches
    of 8, through the host and the device entry points, within the golden bound."""
    print(f"[gpu] audio {mode} 40-window launches", flush=True)
    n = 40
    idx = np.arange(n) % 8
    many = np.ascontiguousarray(atokens[idx])
    with shv.AudioModel(aweights, mode, max_windows=n, experimental=True) as big, \
            shv.AudioModel(aweights, mode, max_windows=8, experimental=True) as small:
        ref = small.sequence(atokens)
        got = big.sequence(many)
        hip = shv.Hip()
        d_t, d_o = hip.upload(many), hip.malloc(n * 4)
        try:
            big.sequence_device(d_t, n, d_o)
            hip.sync()
            dev = hip.download(d_o, (n,), np.float32)
        finally:
            hip.free(d_t)
            hip.free(d_o)
    assert np.array_equal(got.view(np.uint32), ref[idx].view(np.uint32))
    assert np.array_equal(dev.view(np.uint32), ref[idx].view(np.uint32))
    err = float(np.max(np.abs(ref - gold_logits(agold))))
    margin(f"audio {mode} 40-window launch vs reference", err, LOGIT_TOL)
    assert err <= LOGIT_TOL


def test_audio_argument_errors(shv, models, atokens):
    m = models["fp32"]
    lib = m.lib
    out = np.empty(1, np.float32)
    assert lib.shv_hip_audio_sequence(m.h, atokens.ctypes.data, 0, shv.AUDIO_WINDOW_FLOATS, out.ctypes.data) == -1
    assert "empty" in m._err()
    assert lib.shv_hip_audio_sequence(m.h, atokens.ctypes.data, 1, 100, out.ctypes.data) == -1
    assert "stride" in m._err()
    assert lib.shv_hip_audio_sequence_device(m.h, 16, 9, shv.AUDIO_WINDOW_FLOATS, 16, None) == -1
    assert "window count" in m._err()
    assert m.fingerprint and m.mode == "fp32" and m.device_bytes() > 0


def test_audio_profile_families(models, atokens):
    m = models["fp16"]
    m.profile_enable(True)
    try:
        m.sequence(atokens)
        fams = m.profile_families()
        for fam in ("window_input", "gdn_prep", "delta", "gated_norm", "sisa", "head"):
            assert fam in fams
            st = m.profile_read(fam)
            assert st and st["launches"] >= 1 and st["ms"] > 0, fam
        assert any(f.startswith("gemm_seq:") for f in fams)
    finally:
        m.profile_enable(False)
