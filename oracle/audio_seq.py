"""TEST INFRASTRUCTURE ONLY.  A float64 numpy restatement of the SHIELD-A sequence stages (the reference's
engine/audio/sequence.cpp), used by tests/ as a checker of the compiled reference and of the HIP path, never as the
product.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module.

Pinned by tests/test_audio_oracle.py against the reference engine compiled from its own sources
(oracle/_ref/libshield_a_ref.so): per-stage tensors and logits agree to the fp32 rounding noise of the reference.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
from scipy.special import erf

T, D, H, K, V, VD, FF, S = 126, 384, 6, 64, 128, 768, 960, 32   # sequence.cpp:20


def load_shlda(path) -> dict[str, np.ndarray]:
    """Every tensor of a SHLDA001 file as float64 (container: engine/audio/weights.cpp:16-48)."""
    raw = Path(path).read_bytes()
    if raw[:8] != b"SHLDA001":
        raise ValueError("not a SHLDA001 file")
    (count,), off = struct.unpack_from("<I", raw, 8), 12
    out = {}
    for _ in range(count):
        (n,) = struct.unpack_from("<I", raw, off); off += 4
        name = raw[off:off + n].decode(); off += n
        (rank,) = struct.unpack_from("<I", raw, off); off += 4
        dims = struct.unpack_from(f"<{rank}I", raw, off); off += 4 * rank
        (elems,) = struct.unpack_from("<Q", raw, off); off += 8
        a = np.frombuffer(raw, "<f4", elems, off).astype(np.float64).reshape(dims)
        off += 4 * elems
        out[name] = a
    if off != len(raw):
        raise ValueError("trailing data")
    return out


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _softplus(x):                        # sequence.cpp:24
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def _norm(x, w, eps=1e-6):               # sequence.cpp:29-36
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _lin(w, name, x, bias=False):        # y = x W^T (+ b), W [out][in] (sequence.cpp:26-28, kernels.cpp:105-113)
    y = x @ w[name + ".weight"].T
    return y + w[name + ".bias"] if bias else y


def _short_conv(w, name, x):             # causal 4 taps + bias, SiLU (sequence.cpp:127-139)
    wt = w[name + ".weight"][:, 0, :]    # [channels][4], tap j pairs with row t + j - 3
    y = np.broadcast_to(w[name + ".bias"], x.shape).copy()
    for j in range(4):
        sh = 3 - j
        y[sh:] += x[:T - sh] * wt[:, j]
    return _silu(y)


def _l2(x):                              # per head, 1 / max(|x|, 1e-12) (sequence.cpp:140-148)
    x = x.reshape(T, H, K)
    return (x / np.maximum(np.sqrt(np.sum(x * x, -1, keepdims=True)), 1e-12)).reshape(T, H * K)


def _mixer(w, n, x):                     # sequence.cpp:173-215 (no cache)
    q, k, v = _lin(w, n + ".q_proj", x), _lin(w, n + ".k_proj", x), _lin(w, n + ".v_proj", x)
    a, b, g = _lin(w, n + ".a_proj", x), _lin(w, n + ".b_proj", x), _lin(w, n + ".g_proj", x)
    rates = np.exp(w[n + ".A_log"])                                         # transform_gates, :152-159
    a = np.exp(-rates * _softplus(a + w[n + ".dt_bias"]))
    b = _sigmoid(b)
    g = _silu(g)
    q = _l2(_short_conv(w, n + ".q_conv1d", q))
    k = _l2(_short_conv(w, n + ".k_conv1d", k))
    v = _short_conv(w, n + ".v_conv1d", v)
    ow = w[n + ".o_norm.weight"]
    o = np.zeros((T, VD))
    for h in range(H):                                                      # delta rule, :57-68, 201-213
        st = np.zeros((K, V))
        for t in range(T):
            kt, qt, vt = k[t, h * K:(h + 1) * K], q[t, h * K:(h + 1) * K], v[t, h * V:(h + 1) * V]
            st *= a[t, h]
            u = b[t, h] * (vt - kt @ st)
            st += np.outer(kt, u)
            out = (qt @ st) * 0.125
            inv = 1.0 / np.sqrt(np.mean(out * out) + 1e-5)
            o[t, h * V:(h + 1) * V] = out * inv * ow * g[t, h * V:(h + 1) * V]
    return _lin(w, n + ".o_proj", o)


def _ffn(w, n, x):                       # sequence.cpp:216-221
    return _lin(w, n + ".w_down", _silu(_lin(w, n + ".w_gate", x)) * _lin(w, n + ".w_up", x))


def _block(w, n, h, repeats, scale):     # sequence.cpp:222-231
    for _ in range(repeats):
        h = h + scale * _mixer(w, n + ".mixer", _norm(h, w[n + ".mixer_norm.weight"]))
    return h + _ffn(w, n + ".ffn", _norm(h, w[n + ".ffn_norm.weight"]))


def _sisa_last(w, h):                    # sequence.cpp:232-287
    n = "sisa.attn"
    x = _norm(h, w["sisa.attn_norm.weight"])
    q, c = _lin(w, n + ".W_Q", x[-1]), _lin(w, n + ".W_C", x[-1])
    kk, vv, bb = _lin(w, n + ".W_K", x), _lin(w, n + ".W_V", x), _lin(w, n + ".W_B", x)
    theta = _lin(w, n + ".theta_proj", x)
    decay = -np.cumsum(_softplus(_lin(w, n + ".alpha_proj", x, True)), axis=0)
    forget = -np.cumsum(_softplus(-_lin(w, n + ".forget_proj", x, True)), axis=0)
    phi = np.cumsum(theta, axis=0).reshape(T, H, S // 2)
    co, si = np.cos(phi), np.sin(phi)
    bb = bb.reshape(T, H, S // 2, 2)
    br = np.stack([bb[..., 0] * co - bb[..., 1] * si, bb[..., 0] * si + bb[..., 1] * co], -1).reshape(T, H, S)
    c = c.reshape(H, S // 2, 2)
    cr = np.stack([c[..., 0] * co[-1] - c[..., 1] * si[-1], c[..., 0] * si[-1] + c[..., 1] * co[-1]], -1)
    cr = cr.reshape(H, S)
    lam = _softplus(w[n + ".lambda_raw"])
    att = np.zeros(D)
    for hh in range(H):
        content = kk[:, hh * K:(hh + 1) * K] @ q[hh * K:(hh + 1) * K]
        ssm = br[:, hh] @ cr[hh]
        score = content * 0.125 + lam[hh] * np.exp(decay[-1, hh] - decay[:, hh]) * ssm + (forget[-1, hh] - forget[:, hh])
        p = np.exp(score - score.max())
        p /= p.sum()
        att[hh * K:(hh + 1) * K] = p @ vv[:, hh * K:(hh + 1) * K]
    last = h[-1] + _lin(w, n + ".W_O", att)
    return last + _ffn(w, "sisa.ffn", _norm(last, w["sisa.ffn_norm.weight"]))


def sequence(w: dict, tokens: np.ndarray) -> tuple[float, dict[str, np.ndarray]]:
    """tokens [125][384] -> (logit, stages) with stages tokens/gdn_a/gdn_b [126][384], sisa_last [384]
    (sequence.cpp:319-348)."""
    h = np.concatenate([np.asarray(tokens, np.float64).reshape(T - 1, D), w["readout"].reshape(1, D)])
    st = {"tokens": h}
    h = _block(w, "gdn_a", h, 1, 1.0)
    st["gdn_a"] = h
    h = _block(w, "gdn_b", h, 2, 0.7071067811865475244)
    st["gdn_b"] = h
    last = _sisa_last(w, h)
    st["sisa_last"] = last
    z = _lin(w, "head.0", _norm(last, w["head_norm.weight"]), True)
    z = 0.5 * z * (1.0 + erf(z / np.sqrt(2.0)))
    logit = float(_lin(w, "head.3", z, True)[0])
    return logit, st
