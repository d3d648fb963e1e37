"""TEST INFRASTRUCTURE ONLY.  A float64 numpy restatement of the SHIELD-A frontend (the reference's
engine/audio/frontend.cpp: log-mel frames, then the CNN with frequency attention and the token projection), used by
tests/ as a checker of the compiled reference and of the HIP path, never as the product.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module.

Pinned by tests/test_audio_frontend_oracle.py: against the reference engine compiled from its own sources
(oracle/_ref/libshield_a_ref.so, its mel and token dumps and its PCM -> logit), against the golden fixture that
engine wrote (tests/golden/audio_frontend_golden.json), and the DFT step against a direct O(N^2) sum and Parseval's
identity; planted mistakes (strides swapped, the kernel transposed, the residual dropped, the attention softmax over
time instead of frequency) each fail the comparison.
"""
from __future__ import annotations

import numpy as np

NT, NF = 997, 80                       # mel frames per window, mel bins (frontend.cpp:85)
HOP, NFFT, WIN, OFF = 160, 512, 400, 56  # frame t reads pcm[t*160 + 56 .. + 400) into FFT slots 56.. (frontend.cpp:247)
CHANNELS = (48, 96, 160, 192)          # stage outputs (frontend.cpp:215)
BN_EPS = 1e-5                          # frontend.cpp:141


def _bn(w: dict, name: str):
    """Folded BatchNorm (frontend.cpp:136-144): scale = gamma / sqrt(var + eps), shift = beta - mean * scale."""
    scale = w[name + ".weight"] / np.sqrt(w[name + ".running_var"] + BN_EPS)
    return scale, w[name + ".bias"] - w[name + ".running_mean"] * scale


def _silu(x):
    return x / (1.0 + np.exp(-x))


def window_and_fb(w: dict):
    """The analysis window [400] and filterbank [80][257]: the file's (export.py:35) or the reference's defaults
    (frontend.cpp:127-135: periodic Hann, HTK mel triangles from 20 to 7600 Hz on 31.25 Hz bins)."""
    if "frontend.window" in w:
        win = w["frontend.window"].reshape(WIN)
    else:
        j = np.arange(WIN)
        win = 0.5 * (1.0 - np.cos(2.0 * np.pi * j / WIN))
    if "frontend.fb" in w:
        fb = w["frontend.fb"].reshape(NF, NFFT // 2 + 1)
    else:
        m0, m1 = 2595.0 * np.log10(1.0 + 20.0 / 700.0), 2595.0 * np.log10(1.0 + 7600.0 / 700.0)
        hz = 700.0 * (10.0 ** ((m0 + (m1 - m0) * np.arange(82) / 81.0) / 2595.0) - 1.0)
        k = np.arange(NFFT // 2 + 1) * 31.25
        fb = np.zeros((NF, NFFT // 2 + 1))
        for m in range(NF):
            up = (k - hz[m]) / (hz[m + 1] - hz[m])
            down = (hz[m + 2] - k) / (hz[m + 2] - hz[m + 1])
            fb[m] = np.maximum(0.0, np.minimum(up, down))
    return win, fb


def power_spectrum(frames: np.ndarray) -> np.ndarray:
    """|DFT_512|^2 at bins 0..256 of real frames [n][512] (frontend.cpp:248-252: the radix-2 FFT with
    e^{-2 pi i j / 512} twiddles computes this DFT)."""
    spec = np.fft.rfft(frames, n=NFFT, axis=-1)
    return spec.real ** 2 + spec.imag ** 2


def mel(w: dict, pcm: np.ndarray) -> np.ndarray:
    """160,000 samples -> normalised log-mel [997][80] (frontend.cpp:245-256)."""
    win, fb = window_and_fb(w)
    x = np.asarray(pcm, np.float64).reshape(-1)
    idx = np.arange(NT)[:, None] * HOP + OFF + np.arange(WIN)[None, :]
    frames = np.zeros((NT, NFFT))
    frames[:, OFF:OFF + WIN] = x[idx] * win[None, :]
    energy = power_spectrum(frames) @ fb.T
    return (np.log(energy + 1e-6) - w["frontend.mean"].reshape(NF)) / w["frontend.std"].reshape(NF)


def _conv3(x: np.ndarray, k: np.ndarray, sf: int, st: int) -> np.ndarray:
    """Depthwise 3x3 over an image [time][freq][c] with strides (time st, freq sf), zero padding 1; k [c][3 freq][3
    time] (the PyTorch weight [c][1][kf][kt], frontend.cpp:32-39)."""
    t, f, c = x.shape
    ot, of = (t + st - 1) // st, (f + sf - 1) // sf
    xp = np.zeros((t + 2, f + 2, c))
    xp[1:-1, 1:-1] = x
    out = np.zeros((ot, of, c))
    for kf in range(3):
        for kt in range(3):
            tap = xp[kt:kt + st * (ot - 1) + 1:st, kf:kf + sf * (of - 1) + 1:sf]
            out += tap * k[:, kf, kt][None, None, :]
    return out


def _pointwise(w: dict, name: str, x: np.ndarray, act: bool) -> np.ndarray:
    """1x1 convolution + BatchNorm (+ SiLU) (frontend.cpp:183-187)."""
    wt = w[name + ".0.weight"].reshape(w[name + ".0.weight"].shape[0], -1)
    s, b = _bn(w, name + ".1")
    y = (x @ wt.T) * s + b
    return _silu(y) if act else y


def _block(w: dict, x: np.ndarray, out: int, sf: int, st: int, name: str) -> np.ndarray:
    """pw1 (x2, BN, SiLU) -> depthwise 3x3 (BN, SiLU) -> pw2 (BN), + the input when the shape is kept
    (frontend.cpp:193-204)."""
    e = _pointwise(w, name + ".pw1", x, True)
    k = w[name + ".dw.0.weight"].reshape(-1, 3, 3)
    s, b = _bn(w, name + ".dw.1")
    d = _silu(_conv3(e, k, sf, st) * s + b)
    y = _pointwise(w, name + ".pw2", d, False)
    if x.shape[-1] == out and sf == 1 and st == 1:
        y = y + x
    return y


def cnn_image(w: dict, m: np.ndarray) -> np.ndarray:
    """log-mel [997][80] -> feature image [125][20][192] (frontend.cpp:205-221)."""
    k = w["cnn.stem.0.weight"].reshape(32, 3, 3)
    s, b = _bn(w, "cnn.stem.1")
    h = _silu(_conv3(np.repeat(m[:, :, None], 32, axis=2), k, 1, 1) * s + b)
    for st_i, co in enumerate(CHANNELS):
        base = f"cnn.stages.{st_i}"
        h = _block(w, h, co, 2 if st_i < 2 else 1, 2 if st_i < 3 else 1, base + ".0")
        h = _block(w, h, co, 1, 1, base + ".1")
    return h


def tokens(w: dict, m: np.ndarray) -> np.ndarray:
    """Frequency attention (a softmax over the 20 frequency rows of each time step) pooling the image, then the
    projection 192 -> 384: tokens [125][384] (frontend.cpp:222-232)."""
    h = cnn_image(w, m)
    logits = h @ w["cnn.freq_attn.weight"].reshape(192) + w["cnn.freq_attn.bias"].reshape(())
    a = np.exp(logits - logits.max(axis=1, keepdims=True))
    a = a / a.sum(axis=1, keepdims=True)
    pooled = (h * a[:, :, None]).sum(axis=1)
    return pooled @ w["cnn.proj.weight"].reshape(384, 192).T


def frontend(w: dict, pcm: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """160,000 samples -> (log-mel [997][80], tokens [125][384]).  The reference computes the tokens in five time
    slabs with 40-frame halos (frontend.cpp:233-244); the receptive field is 77 frames with a time stride of 8, so
    the slabs give the whole window's result, which is what this computes."""
    m = mel(w, pcm)
    return m, tokens(w, m)
