"""Pointwise-conv GEMM (the wide 1x1-conv workload, the reference's bench/gpu_gemm_bench.cu) through the C-ABI tool entry
points shv_hip_gemm_*: the literal config shapes at full M, bias + hardswish fused, A and W ~ 0.1 N(0,1) from a seed.

  fp32        : the engine's CNN kernels (the CPU engine's K-block-64 order) bitwise equal to the oracle's GEMM on
                sampled rows; the fp32 matrix-core kernel (variant 4, the sequence stages') within
                |C - C_float64| <= 1.5 (K + 8) 2^-24 (sum_k |a_k w_k| + |b|).
  fp16 / bf16 : |C - C_float64| <= 2^-17 (sum_k |a_k w_k| + |b|) on sampled rows -- the split-operand bound; plain
                half-precision operands miss it by ~30x (checked on the CPU below, so the bar pins the split).
  variants    : every kernel variant gives bitwise the automatic choice's outputs (the reference's variant check);
                the fp32 GEMV variant on a 65,536-row prefix, the fp32 K-block variant on an 8,192-row prefix.
"""
import numpy as np
import pytest

SHAPES = [("b2.expand literal", 2560 * 28 * 28, 120, 40), ("b14.expand literal", 2560 * 7 * 7, 960, 160),
          # the short-K routes of the half tiers' planner (K < 64): streaming kernel (<= 5 column tiles), direct kernel
          # at 2 tiles per wave (6), wide kernel (> 10), as the SHIELD-A frontend and the layer path meet them
          ("short-K streaming", 200_000, 64, 32), ("short-K direct", 100_000, 96, 48), ("short-K wide", 100_000, 240, 40)]
SPLIT_TOL = 2.0 ** -17


def operands(M, N, K, seed):
    rng = np.random.default_rng(seed)
    A = (rng.standard_normal((M, K), dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    W = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    b = (rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    return A, W, b


def hswish64(x):
    return x * np.clip(x + 3.0, 0.0, 6.0) / 6.0


def sample_rows(M, rng):
    return np.unique(np.concatenate([np.arange(64), np.arange(M - 64, M), rng.integers(0, M, 4096)]))


def split_bound(A, W, b):
    return np.abs(A).astype(np.float64) @ np.abs(W).astype(np.float64).T + np.abs(b).astype(np.float64)


def test_split_bound_rejects_plain_half_operands():
    """CPU check of the bar itself: rounding A and W to fp16 (one part) breaks the bound on these shapes."""
    A, W, b = operands(512, 120, 40, 7)
    ref = A.astype(np.float64) @ W.astype(np.float64).T + b
    half = A.astype(np.float16).astype(np.float64) @ W.astype(np.float16).astype(np.float64).T + b
    ratio = np.abs(half - ref) / split_bound(A, W, b)
    assert ratio.max() > 8 * SPLIT_TOL


def f32_tol(K):
    """fp32 accumulation of K products in any order, plus the bias add and the hardswish (slope <= 1.5, a few
    roundings): |C - C_float64| <= 1.5 (K + 8) 2^-24 (sum_k |a_k w_k| + |b|).  A dropped or transposed term
    (|a_k w_k| ~ 1e-2 here) misses it by orders of magnitude."""
    return 1.5 * (K + 8) * 2.0 ** -24


def test_f32_bound_rejects_a_dropped_term():
    """CPU check of the fp32 bar: dropping one product of the sum breaks it, fp32 summation in any order meets it."""
    A, W, b = operands(256, 120, 40, 9)
    ref = A.astype(np.float64) @ W.astype(np.float64).T + b
    rev = (A[:, ::-1].astype(np.float32) @ W[:, ::-1].T.astype(np.float32) + b).astype(np.float64)
    scale = split_bound(A, W, b)
    assert (np.abs(rev - ref) / scale).max() <= f32_tol(40)
    dropped = A[:, 1:].astype(np.float64) @ W[:, 1:].astype(np.float64).T + b
    assert (np.abs(dropped - ref) / scale).max() > 100 * f32_tol(40)


@pytest.mark.gpu
@pytest.mark.parametrize("name,M,N,K", SHAPES)
@pytest.mark.parametrize("mode", ["fp32", "fp16", "bf16"])
def test_pw_gemm_parity_and_variants(shv, orc, weights, name, M, N, K, mode):
    """fp32: the engine's own kernel choice for the CNN (the reference CPU order) bitwise equal to the oracle, with
    every CPU-order variant bitwise equal to it; the fp32 matrix-core kernel (the sequence stages') within the fp32
    rounding bound.  fp16 / bf16: the split bound, every variant bitwise equal to the automatic choice."""
    print(f"[gpu] gemm {name} {mode} M={M} N={N} K={K}", flush=True)
    hip = shv.Hip()
    A, W, b = operands(M, N, K, 1 + K)
    dA, dW, db = hip.upload(A), hip.upload(W), hip.upload(b)
    dC = hip.malloc(M * N * 4)
    dV = hip.malloc(M * N * 4)
    try:
        with shv.PwGemm(mode, dW, N, K) as g:
            g.run(dA, M, dC, db, shv.ACT_HSWISH)
            hip.sync()
            C = hip.download(dC, (M, N), np.float32)
            assert np.all(np.isfinite(C))
            rows = sample_rows(M, np.random.default_rng(5))
            x = A[rows].astype(np.float64) @ W.astype(np.float64).T + b
            if mode == "fp32":
                o = orc.Oracle(weights)
                ref = o.gemm(A[rows], W, b, "hs")
                o.close()
                assert np.array_equal(C[rows].view(np.uint32), ref.view(np.uint32))
                g.run(dA, M, dV, db, shv.ACT_HSWISH, variant=4)
                hip.sync()
                mf = hip.download(dV, (M, N), np.float32)
                ratio = np.abs(mf[rows] - hswish64(x)) / split_bound(A[rows], W, b)
                print(f"[gpu]   fp32 matrix cores: max error / bound-scale {ratio.max():.3e} (bar {f32_tol(K):.3e})",
                      flush=True)
                assert np.all(np.isfinite(mf)) and ratio.max() <= f32_tol(K)
            else:
                ratio = np.abs(C[rows] - hswish64(x)) / split_bound(A[rows], W, b)
                print(f"[gpu]   max error / bound-scale {ratio.max():.3e} (bar {SPLIT_TOL:.3e})", flush=True)
                assert ratio.max() <= SPLIT_TOL
            for v in shv.GEMM_VARIANTS[mode]:
                if (v in shv.GEMM_NARROW_VARIANTS and N > 160 and mode != "fp32") or (mode == "fp32" and v == 4):
                    continue
                if mode == "fp32" and v == 5 and (K, N) != (40, 120):   # the narrow kernel's shapes only
                    continue
                m = min(M, 65536) if (mode == "fp32" and v == 1) else min(M, 8192) if (mode == "fp32" and v == 3) else M
                hip.memset(dV, 0xFF, m * N * 4)
                g.run(dA, m, dV, db, shv.ACT_HSWISH, variant=v)
                hip.sync()
                got = hip.download(dV, (m, N), np.float32)
                assert np.array_equal(got.view(np.uint32), C[:m].view(np.uint32)), f"variant {v} differs"
    finally:
        for p in (dA, dW, db, dC, dV):
            hip.free(p)
