"""The oracle (oracle/shv_oracle.c) pinned against the reference CPU engine's golden fixtures and against the
mathematics.  CPU only."""
import hashlib
import math

import numpy as np
import pytest


def digest(a):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    d = a.astype(np.float64)
    return {"n": int(a.size), "sum": float(d.sum()), "abs": float(np.abs(d).sum()), "sq": float((d * d).sum()),
            "head": [int(x) for x in a[:16].view(np.uint32)]}


def test_generator_matches_fixture(shv, weights, golden, clips):
    # SHA-256 of generated weights and every clip equal the fixture (checked by the fixtures themselves too)
    for i in range(0, len(golden["clip_sha256"]), 9):
        assert shv.sha256_bytes(clips[i]) == golden["clip_sha256"][i]
    import json
    side = json.loads(open(str(weights) + ".json").read())
    assert side["parameters"] == 9884507 and side["tensor_count"] == 331   # oracle/shieldv_ref.py:66 PARAMETERS


def test_sha256_fips(shv):
    rng = np.random.default_rng(5)
    for n in (0, 1, 55, 56, 63, 64, 65, 1000, 4097):
        data = rng.integers(0, 256, n, dtype=np.uint8)
        assert shv.sha256_bytes(data) == hashlib.sha256(data.tobytes()).hexdigest()


@pytest.fixture(scope="module")
def oracle_clip0(orc, weights, clips):
    o = orc.Oracle(weights)
    toks = []
    cnn = {}
    for f in range(20):
        toks.append(o.encode_frame(clips[0][f], cnn if f == 19 else None))
    toks = np.stack(toks)
    seq = {}
    logit = o.classify(toks, seq)
    return logit, toks, cnn, seq


def test_oracle_logit_bitwise(oracle_clip0, golden_logits):
    logit = oracle_clip0[0]
    assert logit.view(np.uint32)[0] == golden_logits[:1].view(np.uint32)[0]


def test_oracle_tokens_bitwise(oracle_clip0, golden_tokens):
    toks = oracle_clip0[1]
    assert np.array_equal(toks[0], golden_tokens[0])
    assert np.array_equal(toks[19], golden_tokens[1])


def test_oracle_every_stage_matches_reference(oracle_clip0, golden):
    _, _, cnn, seq = oracle_clip0
    stages = golden["stages_clip0"]
    seen = 0
    for name, d in {**cnn, **seq}.items():
        g = stages[name]
        mine = digest(d)
        assert mine["n"] == g["n"], name
        assert mine["head"] == g["head"], name
        assert mine["sum"] == g["sum"] and mine["sq"] == g["sq"], name
        seen += 1
    assert seen == len(stages) == 25


def test_gemm_against_float64(orc):
    o = orc.Oracle(None)
    rng = np.random.default_rng(1)
    for (M, N, K) in [(3, 17, 5), (7, 33, 64), (5, 40, 65), (4, 24, 200), (2, 960, 160)]:
        A = rng.standard_normal((M, K)).astype(np.float32)
        W = rng.standard_normal((N, K)).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32)
        C = o.gemm(A, W, b, "store")
        ref = A.astype(np.float64) @ W.astype(np.float64).T + b
        bound = (np.abs(A).astype(np.float64) @ np.abs(W).astype(np.float64).T + np.abs(b)) * (K + 2) * 2 ** -23
        assert np.all(np.abs(C - ref) <= bound), (M, N, K)
        # a transposed operand or a dropped K block is far outside the bound
        assert not np.allclose(o.gemm(A, W[:, ::-1], b, "store"), ref, atol=1e-3)


def test_gemm_epilogues(orc):
    o = orc.Oracle(None)
    rng = np.random.default_rng(2)
    M, N, K = 6, 32, 70
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = rng.standard_normal((N, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    R = rng.standard_normal((M, N)).astype(np.float32)
    base = o.gemm(A, W, b, "store").astype(np.float64)
    x = base
    np.testing.assert_allclose(o.gemm(A, W, b, "relu"), np.maximum(x, 0), rtol=0, atol=0)
    np.testing.assert_allclose(o.gemm(A, W, b, "hs"), x * np.clip(x + 3, 0, 6) / 6, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(o.gemm(A, W, b, "hsig"), np.clip(x + 3, 0, 6) / 6, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(o.gemm(A, W, b, "silu"), x / (1 + np.exp(-x)), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(o.gemm(A, W, b, "res", R=R), x + R, rtol=1e-6, atol=1e-6)
    nob = o.gemm(A, W, None, "store").astype(np.float64)
    np.testing.assert_allclose(o.gemm(A, W, None, "acc", C=R.copy()), R + nob, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(o.gemm(A, W, None, "acc_div2", C=R.copy()), R + nob / math.sqrt(2), rtol=1e-6,
                               atol=1e-6)
    sw = o.gemm(A, W, None, "swiglu")
    g, u = nob[:, 0::2], nob[:, 1::2]
    np.testing.assert_allclose(sw, g / (1 + np.exp(-g)) * u, rtol=1e-5, atol=1e-5)


def test_exp_and_silu_ulp(orc):
    o = orc.Oracle(None)
    xs = np.concatenate([np.linspace(-87, 88, 2001), np.linspace(-2, 2, 1001)]).astype(np.float32)
    for x in xs:
        got = o.lib.orc_exp(float(x))
        want = math.exp(float(x))
        ulp = np.spacing(np.float32(want))
        assert abs(got - want) <= 2.0 * ulp, x
    assert abs(o.lib.orc_silu(0.0)) == 0.0
    assert abs(o.lib.orc_silu(10.0) - 10.0 / (1 + math.exp(-10.0))) < 1e-5


def delta_f64(q, k, v, a, b):
    S = np.zeros((64, 128))
    out = np.zeros((q.shape[0], 128))
    for t in range(q.shape[0]):
        S = S * a[t]
        pred = k[t] @ S
        u = (v[t] - pred) * b[t]
        S = S + np.outer(k[t], u)
        out[t] = q[t] @ S
    return out


def test_delta_rule(orc):
    o = orc.Oracle(None)
    rng = np.random.default_rng(3)
    T = 40
    q = rng.standard_normal((T, 64)).astype(np.float32)
    k = rng.standard_normal((T, 64)).astype(np.float32)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    q = (q / np.linalg.norm(q, axis=1, keepdims=True) * 0.125).astype(np.float32)
    v = rng.standard_normal((T, 128)).astype(np.float32)
    a = rng.uniform(0.5, 1.0, T).astype(np.float32)
    b = rng.uniform(0.0, 1.0, T).astype(np.float32)
    got = o.delta_rule(q, k, v, a, b)
    ref = delta_f64(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), a.astype(np.float64),
                    b.astype(np.float64))
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-5)
    # beta = 0: the state never leaves zero
    assert np.all(o.delta_rule(q, k, v, a, np.zeros(T, np.float32)) == 0)
    # one token: o = beta (q . k) v
    one = o.delta_rule(q[:1], k[:1], v[:1], a[:1], b[:1])
    np.testing.assert_allclose(one[0], b[0] * float(q[0] @ k[0]) * v[0], rtol=1e-5, atol=1e-6)
