"""SHIELD-A sequence stages on the CPU: the golden fixture (tests/golden/audio_golden.json, written by the
reference engine compiled from its own sources) is pinned three ways -- the compiled reference reproduces it bit for
bit where it is built, the float64 restatement (oracle/audio_seq.py) agrees with it to fp32 rounding noise, and
plausible mistakes planted in the restatement move it far outside that band -- and the C-ABI's load-time checks of
the audio entry point fail with clear messages before any device work."""
import json
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]

# float64 restatement vs the reference's fp32 engine: measured max 6.0e-6 on the 8 logits
RESTATE_LOGIT_TOL = 5e-5
# relative L2 error of a stage's sampled values; measured 4.8e-7 (gdn_a), 7.3e-7 (gdn_b), 3.7e-6 (sisa_last)
RESTATE_STAGE_TOL = {"tokens": 0.0, "gdn_a": 5e-6, "gdn_b": 5e-6, "sisa_last": 3e-5}


@pytest.fixture(scope="module")
def agold():
    return json.loads((ROOT / "tests" / "golden" / "audio_golden.json").read_text())


@pytest.fixture(scope="module")
def aweights(tmp_path_factory, shv, agold):
    p = tmp_path_factory.mktemp("audio") / "seed5.shlda"
    assert shv.write_audio_weights(p, agold["weights_seed"]) == agold["weights_sha256"], \
        "synthetic audio weight generator drifted from the golden fixture"
    return p


@pytest.fixture(scope="module")
def atokens(shv, agold):
    t = shv.audio_tokens(agold["windows"], agold["tokens_seed"])
    assert shv.sha256_bytes(t) == agold["tokens_sha256"], "token generator drifted from the golden fixture"
    return t


@pytest.fixture(scope="module")
def restated(aweights, atokens):
    import audio_seq
    w = audio_seq.load_shlda(aweights)
    return w, [audio_seq.sequence(w, atokens[i]) for i in range(len(atokens))]


def fixture_logits(agold):
    return np.array([int(b, 16) for b in agold["logit_bits"]], np.uint32).view(np.float32)


def test_fixture_bits_match_values(agold):
    assert np.array_equal(fixture_logits(agold), np.array(agold["logits"], np.float32))


def test_compiled_reference_reproduces_fixture(agold, aweights, atokens):
    import oracle
    if not oracle.AUDIO_SO.exists():
        pytest.skip("oracle/_ref/libshield_a_ref.so not built (needs /root/reference)")
    ref = oracle.AudioReference(aweights)
    try:
        got = np.array([ref.sequence(atokens[i]) for i in range(len(atokens))], np.float32)
    finally:
        ref.close()
    assert np.array_equal(got.view(np.uint32), fixture_logits(agold).view(np.uint32))


def stage_errors(st, gold, step):
    out = {}
    for name, g in gold.items():
        a = np.asarray(st[name], np.float64).ravel()
        assert a.size == g["size"]
        sample = a if name == "sisa_last" else a[::step]
        ref = np.array(g["sample"], np.float64)
        out[name] = float(np.linalg.norm(sample - ref) / np.linalg.norm(ref))
    return out


def test_restatement_matches_fixture(agold, restated, margin):
    _, runs = restated
    d = np.abs(np.array([r[0] for r in runs]) - fixture_logits(agold).astype(np.float64)).max()
    margin("audio restatement logits vs reference", d, RESTATE_LOGIT_TOL)
    assert d <= RESTATE_LOGIT_TOL
    for w, gold in agold["stages"].items():
        errs = stage_errors(runs[int(w)][1], gold, agold["sample_step"])
        for name, e in errs.items():
            assert e <= RESTATE_STAGE_TOL[name], (w, name, e)


@pytest.mark.parametrize("mistake", ["gdn_b_unscaled", "tanh_for_erf", "l2_scaled", "conv_taps_reversed"])
def test_planted_mistakes_leave_the_band(agold, restated, atokens, monkeypatch, mistake):
    import audio_seq
    w, _ = restated
    if mistake == "gdn_b_unscaled":      # GDN-B residual h + branch instead of h + 0.70710678 * branch
        orig = audio_seq._block
        monkeypatch.setattr(audio_seq, "_block", lambda w_, n, h, r, s: orig(w_, n, h, r, 1.0))
    elif mistake == "tanh_for_erf":      # tanh-approximate GELU shape instead of the exact erf GELU
        monkeypatch.setattr(audio_seq, "erf", np.tanh)
    elif mistake == "l2_scaled":         # SHIELD-V's 0.125 q scale carried over into the audio L2 norm
        orig = audio_seq._l2
        monkeypatch.setattr(audio_seq, "_l2", lambda x: orig(x) * 0.125)
    elif mistake == "conv_taps_reversed":   # short-conv tap j paired with row t - j instead of t + j - 3
        orig = audio_seq._short_conv

        def flipped(w_, name, x):
            w2 = dict(w_)
            w2[name + ".weight"] = w_[name + ".weight"][:, :, ::-1]
            return orig(w2, name, x)
        monkeypatch.setattr(audio_seq, "_short_conv", flipped)
    got = np.array([audio_seq.sequence(w, atokens[i])[0] for i in range(4)])
    d = np.abs(got - fixture_logits(agold)[:4].astype(np.float64)).max()
    assert d > 100 * RESTATE_LOGIT_TOL, (mistake, d)


def test_audio_load_rejections(shv, tmp_path, weights):
    lib = shv.library()
    def load(path, mode="fp32", maxw=8):
        h = lib.shv_hip_audio_load(str(path).encode(), mode.encode(), 0, maxw)
        assert not h
        return lib.shv_hip_last_error().decode()
    ok = tmp_path / "a.shlda"
    shv.write_audio_weights(ok, 5)
    assert "experimental" in load(ok, "fp16")
    assert "experimental" in load(ok, "bf16")
    assert "unknown mode" in load(ok, "int8")
    assert "max_windows" in load(ok, "fp32", 0)
    assert "max_windows" in load(ok, "fp32", 5000)
    assert "not a SHLDA001 file" in load(weights)              # a SHIELD-V file
    assert "cannot open" in load(tmp_path / "missing.shlda")
    raw = ok.read_bytes()
    (tmp_path / "trunc.shlda").write_bytes(raw[:-3])
    assert "truncated" in load(tmp_path / "trunc.shlda")
    (tmp_path / "trail.shlda").write_bytes(raw + b"\0")
    assert "trailing" in load(tmp_path / "trail.shlda")
