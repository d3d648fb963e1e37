"""SHIELD-A frontend on the CPU: the float64 restatement (oracle/audio_front.py) pinned against the golden fixture the
reference engine wrote (tests/golden/audio_frontend_golden.json: log-mel and token samples, logits of 3 seeded PCM
windows), against the compiled reference engine itself when it is built, and its DFT step against the direct sum
and Parseval's identity.  Planted mistakes in the restatement (strides swapped, the 3x3 kernel transposed, the
residual dropped, the attention softmax over time instead of frequency) each move the tokens far past the bound.

Bounds: the reference computes in fp32 (the restatement in float64): log-mel within 2e-5 absolute (|mel| <= ~6),
tokens within 2e-5 of the largest token, logits within 2e-5 -- a few times the fp32 rounding noise measured between
the two (mel 2.3e-6, tokens 4.9e-6 relative, logit 6e-7)."""
import json
import sys
import tempfile
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "oracle"))

import audio_front  # noqa: E402
import audio_seq  # noqa: E402

MEL_TOL, TOKEN_REL_TOL, LOGIT_TOL = 2e-5, 2e-5, 2e-5


@pytest.fixture(scope="module")
def fgold():
    return json.loads((ROOT / "tests" / "golden" / "audio_frontend_golden.json").read_text())


@pytest.fixture(scope="module")
def model_weights(shv, fgold, tmp_path_factory):
    p = tmp_path_factory.mktemp("afront") / "audio_model.shlda"
    assert shv.write_audio_model_weights(p, fgold["weights_seed"]) == fgold["weights_sha256"], \
        "synthetic audio model generator drifted from the golden fixture"
    return p


@pytest.fixture(scope="module")
def pcm(shv, fgold):
    x = shv.audio_pcm(fgold["windows"], fgold["pcm_seed"])
    assert shv.sha256_bytes(x) == fgold["pcm_sha256"], "PCM generator drifted from the golden fixture"
    return x


@pytest.fixture(scope="module")
def W(model_weights):
    return audio_seq.load_shlda(model_weights)


@pytest.fixture(scope="module")
def oracle_out(W, pcm):
    return [audio_front.frontend(W, pcm[w]) for w in range(len(pcm))]


def test_sequence_tensors_match_sequence_only_file(shv, W, tmp_path):
    """The whole-model file draws the sequence tensors exactly as the sequence-only file of the same seed."""
    p = tmp_path / "seq.shlda"
    shv.write_audio_weights(p, 5)
    seq = audio_seq.load_shlda(p)
    for name, v in seq.items():
        assert np.array_equal(v, W[name]), name


def test_dft_against_direct_sum_and_parseval():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, audio_front.NFFT))
    p = audio_front.power_spectrum(x)
    n = np.arange(audio_front.NFFT)
    for k in (0, 1, 37, 128, 256):
        direct = (x * np.exp(-2j * np.pi * k * n / audio_front.NFFT)).sum(axis=1)
        assert np.allclose(p[:, k], np.abs(direct) ** 2, rtol=1e-10, atol=1e-9)
    # Parseval over the full spectrum: the rfft half counts bins 1..255 twice
    full = p[:, 0] + p[:, 256] + 2.0 * p[:, 1:256].sum(axis=1)
    assert np.allclose(full, audio_front.NFFT * (x ** 2).sum(axis=1), rtol=1e-10)


def test_oracle_matches_golden(fgold, W, pcm, oracle_out):
    for w, g in enumerate(fgold["per_window"]):
        mel, tok = oracle_out[w]
        mel_nchw = mel.T.reshape(-1)
        assert abs(np.linalg.norm(mel_nchw) - g["mel_l2"]) <= 1e-5 * g["mel_l2"]
        assert np.abs(mel_nchw[::fgold["mel_step"]] - np.array(g["mel_sample"])).max() <= MEL_TOL
        scale = np.abs(tok).max()
        d = np.abs(tok.reshape(-1)[::fgold["token_step"]] - np.array(g["token_sample"])).max()
        assert d <= TOKEN_REL_TOL * scale, (w, d / scale)
        logit, _ = audio_seq.sequence(W, tok.astype(np.float32))
        assert abs(logit - g["logit"]) <= LOGIT_TOL, (w, logit, g["logit"])


def test_oracle_matches_compiled_reference(orc, model_weights, W, pcm, oracle_out):
    if not orc.AUDIO_SO.exists():
        pytest.skip("the reference audio engine (oracle/_ref) is not built")
    ref = orc.AudioReference(model_weights)
    try:
        with tempfile.TemporaryDirectory() as d:
            tok = ref.frontend(pcm[1], d)
            mel = np.fromfile(Path(d) / "mel.f32", np.float32).reshape(80, 997)
        m64, t64 = oracle_out[1]
        assert np.abs(m64.T - mel).max() <= MEL_TOL
        assert np.abs(t64 - tok).max() <= TOKEN_REL_TOL * np.abs(tok).max()
        lg = ref.predict(pcm[1:2])[0]
        l64, _ = audio_seq.sequence(W, tok)
        assert abs(l64 - lg) <= LOGIT_TOL
    finally:
        ref.close()


def _planted(W, m, mistake):
    """tokens of the restatement with one mistake planted (the checker must reject each)"""
    orig_conv, orig_block, orig_tokens = audio_front._conv3, audio_front._block, audio_front.tokens
    try:
        if mistake == "strides_swapped":
            audio_front._conv3 = lambda x, k, sf, st: orig_conv(x, k, st, sf)
        elif mistake == "kernel_transposed":
            audio_front._conv3 = lambda x, k, sf, st: orig_conv(x, np.swapaxes(k, 1, 2), sf, st)
        elif mistake == "residual_dropped":
            def block(w, x, out, sf, st, name):
                y = orig_block(w, x, out, sf, st, name)
                return y - x if (x.shape[-1] == out and sf == 1 and st == 1) else y
            audio_front._block = block
        elif mistake == "softmax_over_time":
            h = audio_front.cnn_image(W, m)
            logits = h @ W["cnn.freq_attn.weight"].reshape(192) + W["cnn.freq_attn.bias"].reshape(())
            a = np.exp(logits - logits.max(axis=0, keepdims=True))
            a = a / a.sum(axis=0, keepdims=True)
            return (h * a[:, :, None]).sum(axis=1) @ W["cnn.proj.weight"].reshape(384, 192).T
        return audio_front.tokens(W, m)
    finally:
        audio_front._conv3, audio_front._block, audio_front.tokens = orig_conv, orig_block, orig_tokens


@pytest.mark.parametrize("mistake", ["strides_swapped", "kernel_transposed", "residual_dropped", "softmax_over_time"])
def test_planted_mistakes_fail_the_golden(fgold, W, oracle_out, mistake):
    m, tok = oracle_out[0]
    try:
        bad = _planted(W, m, mistake)
    except ValueError:
        return   # a shape error is a failure the checker sees too
    if bad.shape != tok.shape:
        return   # so is a token image of the wrong size (strides swapped: 250 time steps)
    g = fgold["per_window"][0]
    d = np.abs(bad.reshape(-1)[::fgold["token_step"]] - np.array(g["token_sample"])).max()
    assert d > 100 * TOKEN_REL_TOL * np.abs(tok).max(), (mistake, d)
