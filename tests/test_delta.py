"""The gated delta rule of config 3 on its own, through the C-ABI entry point shv_hip_delta_rule, against the oracle's
restatement of the CPU engine's recurrence (orc_delta_rule, engine/model/isa_impl.hpp:911-947; pinned to a float64
recurrence and closed forms in tests/test_oracle.py).

  fp32 (token by token, the reference's order; variant 1) : bitwise equal to the oracle.
  fp32 (token by token, keys split over lane groups; variant 3) : within 1e-5 of the largest output.
  fp32 chunked (variants 0, 2: fp32 matrix cores), fp16 / bf16 token by token and chunked :
      max |o - oracle| <= 1e-4 max |o| per (window, head) -- rounding only; a wrong decay, beta, key or chunk
      boundary moves o by O(1).
Inputs follow config 3: q, k l2-normalised N(0,1) rows (q scaled by 1/8), v ~ N(0,1), beta = sigmoid(N(0,1)),
decay = exp(-exp(A_log) softplus(N(0,1))) with A_log = ln U[1,16] per head; window 2 has strongly correlated keys
(the worst conditioning for the chunked scan's (I + L)^-1).
"""
import numpy as np
import pytest

T, H = 321, 6


def inputs(n_windows, seed):
    rng = np.random.default_rng(seed)
    rows = n_windows * T

    def l2(x):
        return (x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)).astype(np.float32)

    q = l2(rng.standard_normal((rows, H, 64))) * np.float32(0.125)
    kraw = rng.standard_normal((rows, H, 64))
    if n_windows > 2:   # window 2: keys close to one direction per head
        kraw[2 * T:3 * T] = 0.3 * kraw[2 * T:3 * T] + rng.standard_normal((1, H, 64)) * 3.0
    k = l2(kraw)
    v = rng.standard_normal((rows, H * 128)).astype(np.float32)
    a_log = np.log(rng.uniform(1.0, 16.0, H))
    sp = np.log1p(np.exp(rng.standard_normal((rows, H))))
    dec = np.zeros((rows, 8), np.float32)
    beta = np.zeros((rows, 8), np.float32)
    dec[:, :H] = np.exp(-np.exp(a_log) * sp)
    beta[:, :H] = 1.0 / (1.0 + np.exp(-rng.standard_normal((rows, H))))
    return q.reshape(rows, H * 64), k.reshape(rows, H * 64), v, dec, beta


def oracle_o(orc, weights, q, k, v, dec, beta, n_windows):
    o = orc.Oracle(weights)
    out = np.zeros((n_windows * T, H * 128), np.float32)
    for w in range(n_windows):
        rs = slice(w * T, (w + 1) * T)
        for h in range(H):
            out[rs, h * 128:(h + 1) * 128] = o.delta_rule(q[rs, h * 64:(h + 1) * 64], k[rs, h * 64:(h + 1) * 64],
                                                          v[rs, h * 128:(h + 1) * 128], dec[rs, h], beta[rs, h])
    o.close()
    return out


@pytest.mark.gpu
def test_delta_rule_kernels_against_oracle(shv, orc, weights):
    n = 3
    q, k, v, dec, beta = inputs(n, 11)
    ref = oracle_o(orc, weights, q, k, v, dec, beta, n)
    hip = shv.Hip()
    bufs = [hip.upload(x) for x in (q, k, v, dec, beta)]
    d_o = hip.malloc(n * T * H * 128 * 4)
    try:
        for mode, variant in (("fp32", 1), ("fp32", 0), ("fp32", 2), ("fp32", 3), ("fp16", 1), ("fp16", 2),
                              ("bf16", 1), ("bf16", 2)):
            print(f"[gpu] delta rule {mode} variant {variant}, {n} windows", flush=True)
            hip.memset(d_o, 0xFF, n * T * H * 128 * 4)
            shv.delta_rule(mode, *bufs, n, d_o, variant)
            hip.sync()
            got = hip.download(d_o, (n * T, H * 128), np.float32)
            bad = ~np.isfinite(got)
            if bad.any():
                rr, cc = np.nonzero(bad)
                print(f"[gpu]   non-finite: {bad.sum()} values, rows {rr.min()}..{rr.max()}, cols {cc.min()}..{cc.max()}",
                      flush=True)
            assert not bad.any()
            if mode == "fp32" and variant == 1:   # the reference's operation order
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
                continue
            # key split (fp32: fp32 operations in another order), the chunked scans and the half tiers' kernels:
            # per (window, head), relative to the largest output; a wrong decay, beta, key or chunk boundary moves
            # outputs by O(1)
            tol = 1e-5 if (mode == "fp32" and variant == 3) else 1e-4
            for w in range(n):
                for h in range(H):
                    g = got[w * T:(w + 1) * T, h * 128:(h + 1) * 128]
                    r = ref[w * T:(w + 1) * T, h * 128:(h + 1) * 128]
                    err = float(np.abs(g - r).max()) / float(np.abs(r).max())
                    assert err <= tol, (mode, variant, w, h, err)
            print(f"[gpu]   max rel err {max(float(np.abs(got - ref).max() / np.abs(ref).max()), 0):.2e}", flush=True)
    finally:
        for p in bufs + [d_o]:
            hip.free(p)



@pytest.mark.gpu
def test_delta_rule_fp32_row_independence(shv):
    """A window's exact-tier recurrence does not depend on the other windows of the launch: the first 3 of 17 windows
    equal the 3-window run bitwise (the 3-window run is pinned to the oracle by the test above)."""
    n_big, n_small = 17, 3
    q, k, v, dec, beta = inputs(n_big, 12)
    hip = shv.Hip()
    bufs = [hip.upload(x) for x in (q, k, v, dec, beta)]
    d_big = hip.malloc(n_big * T * H * 128 * 4)
    d_small = hip.malloc(n_small * T * H * 128 * 4)
    try:
        print(f"[gpu] fp32 delta rule: {n_big} windows vs {n_small}", flush=True)
        shv.delta_rule("fp32", *bufs, n_big, d_big, 0)
        shv.delta_rule("fp32", *bufs, n_small, d_small, 0)
        hip.sync()
        big = hip.download(d_big, (n_big * T, H * 128), np.float32)[:n_small * T]
        small = hip.download(d_small, (n_small * T, H * 128), np.float32)
        assert np.all(np.isfinite(small))
        assert np.array_equal(big.view(np.uint32), small.view(np.uint32))
    finally:
        for p in bufs + [d_big, d_small]:
            hip.free(p)
