"""GPU parity of the HIP engine against the reference CPU engine's golden fixtures (through the C-ABI).

Bars (the path's stated tolerances):
  fp32  : tokens bitwise equal to the reference (the CNN keeps the reference CPU order); logits within 4e-4 absolute,
          no decision flips -- both with the engine's own sequence-stage arithmetic (fp32 matrix-core GEMMs,
          key-split delta rule) and with the reference order there too (SHV_HIP_F32_CPU_ORDER=1).
  fp16  : max |logit - exact| <= FP16_TOL on the 64-clip seeded set, 0 flips at the sidecar threshold.
  bf16  : max |logit - exact| <= BF16_TOL, 0 flips.
Row independence: a window's logit and a frame's tokens are bitwise identical whatever else is in the batch.
"""
import ctypes
import os
import sys
import tempfile
import threading
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FP32_TOL = 4e-4
# half tiers: split-operand MFMA (fp32-level operand precision; fp16 weights pre-scaled by a power of two); measured
# max 2.3e-3 (fp16), 4.0e-3 (bf16) on 64 clips
FP16_TOL = 1e-2
BF16_TOL = 1e-2
CNN_STAGES = ["cnn%02d" % i for i in range(17)]


def flips(a, b, thr):
    from math import exp
    sa = np.array([x >= 0 for x in a])  # threshold 0.5 <=> logit >= 0 (sigmoid is monotone)
    sb = np.array([x >= 0 for x in b])
    assert thr == 0.5
    return int((sa != sb).sum())


def digest(a):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    d = a.astype(np.float64)
    return {"n": int(a.size), "sum": float(d.sum()), "sq": float((d * d).sum()),
            "head": [int(x) for x in a[:16].view(np.uint32)]}


def load_cpu_order(shv, weights, **kw):
    """An fp32 model in the reference CPU engine's operation order (read at load)."""
    os.environ["SHV_HIP_F32_CPU_ORDER"] = "1"
    try:
        return shv.Model(weights, "fp32", **kw)
    finally:
        del os.environ["SHV_HIP_F32_CPU_ORDER"]


@pytest.fixture(scope="module")
def fp32_model(shv, weights):
    print("[gpu] load fp32", flush=True)
    m = shv.Model(weights, "fp32")
    yield m
    m.close()


@pytest.fixture(scope="module")
def fp32_cpu_model(shv, weights):
    print("[gpu] load fp32 in the reference CPU order", flush=True)
    m = load_cpu_order(shv, weights)
    yield m
    m.close()


@pytest.mark.parametrize("order", ["engine", "cpu"])
def test_fp32_tokens_bitwise(fp32_model, fp32_cpu_model, clips, golden_tokens, order):
    """The exact tier's CNN performs the reference CPU engine's operation order in both settings."""
    m = fp32_model if order == "engine" else fp32_cpu_model
    print(f"[gpu] fp32 ({order} order) encode clip 0", flush=True)
    toks = m.encode_frames(clips[0])
    assert toks.shape == (20, 16, 384)
    assert np.array_equal(toks[0], golden_tokens[0]), np.abs(toks[0] - golden_tokens[0]).max()
    assert np.array_equal(toks[19], golden_tokens[1])


@pytest.mark.parametrize("order", ["engine", "cpu"])
def test_fp32_logits(fp32_model, fp32_cpu_model, clips, golden_logits, golden, margin, order):
    m = fp32_model if order == "engine" else fp32_cpu_model
    print(f"[gpu] fp32 ({order} order) predict {len(clips)} clips", flush=True)
    lg = m.predict(clips)
    err = float(np.abs(lg - golden_logits).max())
    nf = flips(lg, golden_logits, golden["threshold"])
    print(f"[gpu] fp32 ({order} order) max|dlogit| = {err:.3e} over {len(clips)} clips, flips {nf}", flush=True)
    margin(f"fp32 ({order} order) max|logit - reference| over {len(clips)} clips", err, FP32_TOL)
    assert err <= FP32_TOL, f"fp32 max|dlogit| {err:.3e} > {FP32_TOL}"
    assert nf == 0, f"{nf} decision flips"


def test_fp32_stages(shv, weights, clips, golden):
    """The reference CPU order: the 17 CNN stage outputs and the tokens bitwise the reference engine's, the sequence
    stages by their sums (device libm in the gates)."""
    print("[gpu] fp32 (CPU order) stage dumps", flush=True)
    stages = golden["stages_clip0"]
    with tempfile.TemporaryDirectory() as d, load_cpu_order(shv, weights, use_graphs=0) as m:
        m.set_dump_dir(d)
        m.encode_frames(clips[0][19:20])          # golden CNN stages are frame 19's
        for name in CNN_STAGES + ["tokens"]:
            got = digest(np.fromfile(Path(d) / f"{name}.f32", np.float32))
            g = stages[name]
            assert got["n"] == g["n"] and got["head"] == g["head"] and got["sum"] == g["sum"], name
        m.predict(clips[:1])
        for name in ["h0", "after_gdn_a", "after_gdn_b", "after_sisa_last", "logit"]:
            a = np.fromfile(Path(d) / f"{name}.f32", np.float32).astype(np.float64)
            g = stages[name]
            assert a.size == g["n"], name
            rel = abs(a.sum() - g["sum"]) / max(1.0, g["abs"])
            assert rel < 1e-4, (name, rel)


SEQ_STAGES = ["h0", "after_gdn_a", "after_gdn_b", "after_sisa_last", "logit"]
# Each stage's own contribution, element by element: the stage minus its input (the residual stream before the
# block: after_gdn_a - h0 is GDN-A's output, after_gdn_b - after_gdn_a the two GDN-B blocks', after_sisa_last - the
# last row of after_gdn_b the SISA block's), as max |d| / max |oracle increment|.  The residual stream itself is
# dominated by the tokens and positions, so comparing it alone would hide a block's error below the rounding of
# its input.  Measured on clip 0: reference order 1.1e-5 / 8.5e-6 / 5.7e-7 / 8.2e-8 (GDN-A, GDN-B, SISA, logit:
# device expf / log1pf in the gates, compounded by the decay products over 321 tokens); the chunked delta rule of
# the other settings 2.2e-5 / 1.7e-5 / 1.5e-6 to 4.2e-6 / 1.6e-7 to 5.1e-6 in fp32, fp16 and bf16 alike (its order
# differs from the token-by-token recurrence; the operand parts carry fp32-level precision).  A wrong weight, gate
# or sign moves an increment by O(1).
SEQ_INC_TOL = {"fp32-cpu": 5e-5, "fp32": 1e-4, "fp16": 2e-4, "bf16": 2e-4}


@pytest.fixture(scope="module")
def seq_oracle(orc, weights, fp32_model, clips):
    """Clip 0's tokens (the exact tier's CNN: bitwise the reference's) and the oracle's sequence stages for them."""
    toks = fp32_model.encode_frames(clips[0]).reshape(20, 16, 384)
    print("[gpu] oracle sequence stages of clip 0 (CPU)", flush=True)
    o = orc.Oracle(weights)
    try:
        stages = {}
        o.classify(toks, stages)
    finally:
        o.close()
    return toks, stages


def seq_increments(st):
    f = {n: st[n].astype(np.float64) for n in SEQ_STAGES}
    return {"h0": f["h0"],
            "gdn_a": f["after_gdn_a"] - f["h0"],
            "gdn_b": f["after_gdn_b"] - f["after_gdn_a"],
            "sisa_last": f["after_sisa_last"] - f["after_gdn_b"][-f["after_sisa_last"].size:],
            "logit": f["logit"]}


@pytest.mark.parametrize("mode", ["fp32-cpu", "fp32", "fp16", "bf16"])
def test_sequence_stages_elementwise(shv, weights, seq_oracle, mode, margin):
    """Each sequence stage of one window, element by element, against the oracle's (the reference CPU engine's
    operation order, checked bitwise against its golden digests) on the same tokens: the exact tier in the reference
    order and in its own, and the half tiers.  The window input h0 is exact in every tier."""
    toks, ref = seq_oracle
    print(f"[gpu] {mode}: sequence stage dumps of clip 0", flush=True)
    with tempfile.TemporaryDirectory() as d:
        if mode == "fp32-cpu":
            m = load_cpu_order(shv, weights, use_graphs=0)
        else:
            m = shv.Model(weights, mode.split("-")[0], experimental=mode != "fp32", use_graphs=0)
        with m:
            m.set_dump_dir(d)
            lg = m.classify(toks.reshape(1, 20, 16, 384))
            got = {n: np.fromfile(Path(d) / f"{n}.f32", np.float32) for n in SEQ_STAGES}
    assert np.all(np.isfinite(lg))
    for n in SEQ_STAGES:
        assert got[n].shape == ref[n].shape, (n, got[n].shape, ref[n].shape)
    assert np.array_equal(got["h0"], ref["h0"])
    gi, ri = seq_increments(got), seq_increments(ref)
    for name in ["gdn_a", "gdn_b", "sisa_last", "logit"]:
        a, b = gi[name], ri[name]
        err = float(np.abs(a - b).max()) / max(1e-30, float(np.abs(b).max()))
        print(f"[gpu] {mode} {name}: max|d| / max|oracle| {err:.3e}", flush=True)
        margin(f"{mode} sequence stage {name} vs oracle (relative, every element)", err, SEQ_INC_TOL[mode])
        assert err <= SEQ_INC_TOL[mode], (name, err)


def test_row_independence_fp32(fp32_model, clips):
    """A clip's logit does not depend on the rest of the batch.  One clip's GEMMs run on the matrix-core kernel's
    small tiles and its delta rule on eight key groups per column, the batch of 6 on larger tiles and four groups:
    the comparison holds the tilings and splits to bitwise equal results."""
    print("[gpu] fp32 row independence", flush=True)
    batch = fp32_model.predict(clips[:6])
    rev = fp32_model.predict(clips[:6][::-1])[::-1]
    single = np.concatenate([fp32_model.predict(clips[i:i + 1]) for i in (0, 3, 5)])
    assert np.array_equal(batch, rev)
    assert np.array_equal(batch[[0, 3, 5]], single)


def test_classify_matches_predict(fp32_model, clips):
    print("[gpu] fp32 classify(tokens) == predict", flush=True)
    toks = fp32_model.encode_frames(clips[:2].reshape(-1, 180, 320, 3))
    lg = fp32_model.classify(toks.reshape(2, 20, 16, 384))
    assert np.array_equal(lg, fp32_model.predict(clips[:2]))


@pytest.mark.parametrize("mode,tol", [("fp16", FP16_TOL), ("bf16", BF16_TOL)])
def test_half_modes(shv, weights, clips, golden_logits, golden, mode, tol, margin):
    print(f"[gpu] {mode} predict 64 clips", flush=True)
    with shv.Model(weights, mode, experimental=True) as m:
        lg = m.predict(clips)
        err = float(np.abs(lg - golden_logits).max())
        nf = flips(lg, golden_logits, golden["threshold"])
        print(f"[gpu] {mode}: max|dlogit| = {err:.4e}, mean = {np.abs(lg - golden_logits).mean():.3e}, "
              f"flips = {nf}", flush=True)
        margin(f"{mode} max|logit - reference| over 64 clips", err, tol)
        assert np.all(np.isfinite(lg))
        assert err <= tol, f"{mode} max|dlogit| {err:.3e} > {tol}"
        assert nf == 0, f"{mode}: {nf} decision flips"
        # row independence in the MFMA tier
        sub = m.predict(clips[5:8])
        assert np.array_equal(sub, lg[5:8])
        one = m.predict(clips[7:8])
        assert np.array_equal(one, lg[7:8])


# Half-tier tokens against the reference engine's (exact fp32) tokens of clip 0, frames 0 and 19.  The split operands
# carry fp32-level precision into the matrix cores, but accumulation order differs from the reference's and the
# random-init encoder amplifies rounding through 15 blocks; the bound is relative to the largest token magnitude
# (tokens reach ~850 here), where a wrong channel, tap or pixel moves tokens by O(max).
HALF_TOKEN_REL_TOL = 2e-3


@pytest.mark.parametrize("mode", ["fp16", "bf16"])
def test_half_tier_tokens_near_reference(shv, weights, clips, golden_tokens, mode, margin):
    print(f"[gpu] {mode} tokens of clip 0 against the reference's", flush=True)
    with shv.Model(weights, mode, experimental=True) as m:
        toks = m.encode_frames(clips[0])
    scale = float(np.abs(golden_tokens).max())
    for f, g in ((0, golden_tokens[0]), (19, golden_tokens[1])):
        rel = float(np.abs(toks[f] - g).max()) / scale
        mean_rel = float(np.abs(toks[f] - g).mean()) / scale
        print(f"[gpu] {mode} frame {f}: max|dtoken| / max|token| = {rel:.3e} (mean {mean_rel:.3e})", flush=True)
        margin(f"{mode} frame {f} max|token - reference| / max|token|", rel, HALF_TOKEN_REL_TOL)
        assert np.all(np.isfinite(toks[f]))
        assert rel <= HALF_TOKEN_REL_TOL, f"{mode} frame {f}: {rel:.3e}"


# Config 3's own workload: classify on N(0,1) tokens (not encoder outputs), against the oracle's classify (the
# reference CPU engine's sequence stages, restated) for a few windows, in every tier.
@pytest.mark.parametrize("mode,tol", [("fp32", FP32_TOL), ("fp16", FP16_TOL), ("bf16", BF16_TOL)])
def test_classify_config3_tokens_against_oracle(shv, orc, weights, mode, tol, margin):
    n = 3
    rng = np.random.default_rng(31)
    toks = rng.standard_normal((n, 20, 16, 384)).astype(np.float32)
    print(f"[gpu] {mode} classify {n} windows of N(0,1) tokens", flush=True)
    with shv.Model(weights, mode, experimental=mode != "fp32") as m:
        lg = m.classify(toks)
    o = orc.Oracle(weights)
    try:
        ref = np.array([o.classify(toks[w].reshape(20, 16 * 384))[0] for w in range(n)], np.float32)
    finally:
        o.close()
    err = float(np.abs(lg - ref).max())
    print(f"[gpu] {mode} config-3 classify: logits {lg}, oracle {ref}, max|d| {err:.3e}", flush=True)
    margin(f"{mode} config-3 classify max|logit - oracle| ({n} windows)", err, tol)
    assert np.all(np.isfinite(lg))
    assert err <= tol, f"{mode}: {err:.3e}"


def test_async_coalescing_and_slots(shv, weights, clips):
    print("[gpu] async API", flush=True)
    with shv.Model(weights, "fp32", token_slots=64) as m:
        ref = m.predict(clips[:3])
        toks = m.encode_frames(clips[:3].reshape(-1, 180, 320, 3)).reshape(3, 20, 6144)
        # job A encodes clip 0, stores its frames into slots 0..19 and classifies window 0 from its own frames
        la = np.full(1, -7.0, np.float32)
        ja, ka = m.submit(frames=clips[0], store_slots=np.arange(20), n_windows=1,
                          window_frames=np.arange(20), logits_out=la)
        # job B: window from slots 0..19 (reads what A stored; A is earlier in FIFO order)
        lb = np.full(1, -7.0, np.float32)
        jb, kb = m.submit(n_windows=1, window_frames=np.full(20, -1), window_slots=np.arange(20), logits_out=lb)
        # job C: window from host tokens of clip 2, mixed with frames of its own request for clip 1
        lc = np.full(2, -7.0, np.float32)
        tok2 = np.ascontiguousarray(toks[2])
        ptrs = [tok2[i].ctypes.data for i in range(20)] + [0] * 20
        wf = np.concatenate([np.full(20, -1), np.arange(20)])
        seen = []
        cb = shv.CALLBACK(lambda job, status, user: seen.append(status))
        jc, kc = m.submit(frames=clips[1], n_windows=2, window_frames=wf, window_tokens=ptrs, logits_out=lc,
                          callback=cb)
        for j in (ja, jb, jc):
            assert m.job_wait(j) == 0
        rc, t = m.job_timing(jc)
        assert rc == 0 and t["batch_windows"] >= 2
        for j in (ja, jb, jc):
            m.job_free(j)
        assert seen == [1]
        assert la[0] == ref[0] and lb[0] == ref[0]
        assert lc[0] == ref[2] and lc[1] == ref[1]


def test_failed_batch_gives_nan(shv, weights, clips):
    print("[gpu] injected batch failure", flush=True)
    with shv.Model(weights, "fp32") as m:
        os.environ["SHV_HIP_TEST_FAIL_BATCH"] = "1"
        try:
            out = np.zeros(1, np.float32)
            j, keep = m.submit(frames=clips[0], n_windows=1, window_frames=np.arange(20), logits_out=out)
            assert m.job_wait(j) == -1
            assert "injected" in m.job_error(j)
            assert m.job_status(j) == -1
            m.job_free(j)
            assert np.isnan(out[0])
        finally:
            del os.environ["SHV_HIP_TEST_FAIL_BATCH"]
        assert np.all(np.isfinite(m.predict(clips[:1])))


def test_invalid_requests(shv, weights, clips):
    with shv.Model(weights, "fp32", max_frames=40, max_windows=2, token_slots=4) as m:
        out = np.zeros(3, np.float32)
        with pytest.raises(shv.ShvError, match="more frames than max_frames"):
            m.submit(frames=np.zeros((41, 180, 320, 3), np.uint8))
        with pytest.raises(shv.ShvError, match="more windows"):
            m.submit(n_windows=3, logits_out=out)
        with pytest.raises(shv.ShvError, match="store slot out of range"):
            m.submit(frames=clips[0][:2], store_slots=[0, 4])
        with pytest.raises(shv.ShvError, match="duplicate store slot"):
            m.submit(frames=clips[0][:2], store_slots=[1, 1])
        with pytest.raises(shv.ShvError, match="window frame index out of range"):
            m.submit(frames=clips[0][:2], n_windows=1, window_frames=np.full(20, 5), logits_out=out)
        with pytest.raises(shv.ShvError, match="no token source"):
            m.submit(n_windows=1, logits_out=out)
        with pytest.raises(shv.ShvError, match="empty request"):
            m.submit()
        # predict splits into GPU batches of min(max_windows, max_frames / 20) = 2 clips
        lg = m.predict(clips[:3])
        assert np.all(np.isfinite(lg))


def test_forward_device_matches_predict(shv, weights, clips):
    print("[gpu] forward_device", flush=True)
    n = 3
    hip = shv.Hip()
    with shv.Model(weights, "fp16", experimental=True, max_frames=n * 20, max_windows=n) as m:
        ref = m.predict(clips[:n])
        d_frames = hip.upload(clips[:n])
        d_logits = hip.upload(np.full(n, np.nan, np.float32))
        d_tok = hip.malloc(20 * 6144 * 4)
        stream = hip.stream()
        try:
            for _ in range(2):   # capture, then graph replay
                m.forward_device(d_frames, n, d_logits, stream)
                hip.stream_sync(stream)
                assert np.array_equal(hip.download(d_logits, n, np.float32), ref)
            m.encode_device(d_frames, 20, d_tok, stream)
            hip.stream_sync(stream)
            got = hip.download(d_tok, (20, 16, 384), np.float32)
            assert np.array_equal(got, m.encode_frames(clips[0]))
        finally:
            hip.stream_destroy(stream)
            for p in (d_frames, d_logits, d_tok):
                hip.free(p)


@pytest.mark.parametrize("mode", ["fp16", "bf16"])
def test_fused_blocks_match_layer_path(shv, weights, clips, mode):
    """The fused inverted-residual kernels against the layer-by-layer path of the same tier (SHV_HIP_NO_FUSE).
    The stem is the same kernel in both paths (bitwise equal).  Blocks 1-3 run in the strip kernel, whose expand and
    project accumulators start from the bias and whose K = 16 matrix steps round in another order than the layer
    GEMMs: accumulation rounding only, held to 1e-5 of the stage's largest magnitude.  From block 4 on the SE mean
    also sums per-tile partials in another fixed order; the random-init encoder amplifies such rounding differences
    smoothly through the late blocks (measured: 1.6e-7 relative after block 4, 9e-6 after block 12, 1.4e-4 after
    block 15), so later stages are held to 1e-3 -- a wrong weight, channel, tap or pixel moves them by O(1)."""
    print(f"[gpu] {mode} fused vs layer-by-layer stage dumps", flush=True)
    dumps = {}
    for fuse in (False, True):
        if fuse:
            os.environ.pop("SHV_HIP_NO_FUSE", None)
        else:
            os.environ["SHV_HIP_NO_FUSE"] = "1"
        try:
            with tempfile.TemporaryDirectory() as d, shv.Model(weights, mode, experimental=True, use_graphs=0) as m:
                m.set_dump_dir(d)
                toks = m.encode_frames(clips[0][19:20])
                dumps[fuse] = {n: np.fromfile(Path(d) / f"{n}.f32", np.float32) for n in CNN_STAGES + ["tokens"]}
                dumps[fuse]["out"] = toks.reshape(-1)
        finally:
            os.environ.pop("SHV_HIP_NO_FUSE", None)
    for name in CNN_STAGES + ["tokens", "out"]:
        a, b = dumps[True][name], dumps[False][name]
        assert a.shape == b.shape, name
        assert np.all(np.isfinite(a)), name
        if name == "cnn00":
            assert np.array_equal(a, b), (name, float(np.abs(a - b).max()))
        else:
            err = float(np.abs(a - b).max()) / max(1e-30, float(np.abs(b).max()))
            print(f"[gpu] {mode} {name}: max rel diff {err:.2e}", flush=True)
            assert err <= (1e-5 if name in ("cnn01", "cnn02", "cnn03") else 1e-3), (name, err)


@pytest.mark.parametrize("mode", ["fp16", "bf16"])
def test_fused_tail_matches_unfused(shv, weights, clips, mode, monkeypatch):
    """The fused last 1x1 + hardswish + 4x4 pool of the half tiers (taken when no dump directory is set) repeats the
    unfused GEMM's split products in the same K order, its epilogue and the pool kernel's bin sums: tokens are bitwise
    those of the unfused path (taken while dumping).  The stem runs unfused on both sides."""
    print(f"[gpu] {mode} fused tail vs unfused tail, frames of clip 0", flush=True)
    monkeypatch.setenv("SHV_HIP_NO_STEM_FUSE", "1")
    frames = clips[0][:8]
    with shv.Model(weights, mode, experimental=True, use_graphs=0) as m:
        fused = m.encode_frames(frames)
        with tempfile.TemporaryDirectory() as d:
            m.set_dump_dir(d)
            unfused = m.encode_frames(frames)
    assert np.all(np.isfinite(fused))
    assert np.array_equal(fused.view(np.uint32), unfused.view(np.uint32)), float(np.abs(fused - unfused).max())


@pytest.mark.parametrize("mode", ["fp16", "bf16"])
def test_fused_stem_close_to_unfused(shv, weights, clips, mode, monkeypatch):
    """The stem inside block 1's strip kernel runs on the matrix cores with split operands (fp32-level operand
    precision) instead of the fp32 stem kernel's fma chains: over whole frames (borders included) its tokens stay
    within accumulation-rounding distance of the unfused path's, and so do the logits."""
    print(f"[gpu] {mode} fused stem vs stem kernel, frames of clips 0-3", flush=True)
    frames = clips[:4].reshape(-1, 180, 320, 3)
    with shv.Model(weights, mode, experimental=True, use_graphs=0, max_frames=80, max_windows=4) as m:
        fused = m.encode_frames(frames)
        lf = m.predict(clips[:4])
        monkeypatch.setenv("SHV_HIP_NO_STEM_FUSE", "1")
        unfused = m.encode_frames(frames)
        lu = m.predict(clips[:4])
    assert np.all(np.isfinite(fused))
    scale = float(np.abs(unfused).max())
    err = float(np.abs(fused - unfused).max())
    print(f"[gpu] {mode}: token max|diff| {err:.3e} (max |token| {scale:.3e}), logit max|diff| "
          f"{float(np.abs(lf - lu).max()):.3e}", flush=True)
    assert err <= 1e-3 * scale
    assert float(np.abs(lf - lu).max()) <= 2e-3


@pytest.mark.parametrize("mode", ["fp16", "bf16"])
def test_row_independence_half(shv, weights, clips, mode):
    """A clip's logit does not depend on the rest of the batch in the half tiers either.  A batch of 8 clips puts
    the sequence GEMMs (8 x 321 rows) and the late SE projects above the small-M kernel's 2048-row limit while single
    clips stay below it, so this also holds the small-M and large-M kernels to bitwise equal results."""
    print(f"[gpu] {mode} row independence: batch of 8 vs one by one", flush=True)
    with shv.Model(weights, mode, experimental=True, max_frames=160, max_windows=8) as m:
        batch = m.predict(clips[:8])
        single = np.concatenate([m.predict(clips[i:i + 1]) for i in range(8)])
    assert np.all(np.isfinite(batch))
    assert np.array_equal(batch.view(np.uint32), single.view(np.uint32)), float(np.abs(batch - single).max())


@pytest.mark.parametrize("mode", ["fp16", "bf16"])
def test_seq_gemm_dma_matches_lds(shv, weights, clips, mode, monkeypatch):
    """The sequence GEMMs take pre-split A; above 2048 rows they run in the kernel that loads operand tiles straight
    from HBM into LDS (swizzled fragment blocks, several K steps in flight).  It performs every output's MFMA
    sequence in the register-staged LDS kernel's order (SHV_HIP_NO_GEMM_DMA=1), so 16 clips (5136 sequence rows,
    partial last row and column blocks) give bitwise the same logits either way."""
    print(f"[gpu] {mode} sequence GEMMs: direct-to-LDS kernel vs register-staged kernel, 16 clips", flush=True)
    with shv.Model(weights, mode, experimental=True, use_graphs=0, max_frames=320, max_windows=16) as m:
        monkeypatch.delenv("SHV_HIP_NO_GEMM_DMA", raising=False)
        dma = m.predict(clips[:16])
        monkeypatch.setenv("SHV_HIP_NO_GEMM_DMA", "1")
        lds = m.predict(clips[:16])
    assert np.all(np.isfinite(dma))
    assert np.array_equal(dma.view(np.uint32), lds.view(np.uint32)), float(np.abs(dma - lds).max())


@pytest.mark.parametrize("mode", ["fp16"])
def test_delta_splits_bitwise(shv, weights, clips, mode):
    """The half tiers split the delta rule by batch size: the chunked scan deals a head's 128 value columns over
    4 / 2 / 1 workgroups (up to 16 / 64 / more windows) and the token-by-token kernel (SHV_HIP_DELTA_SEQ=1) splits each
    value column's keys over 8 / 4 / 2 lane groups (up to 10 / 21 / more windows).  Every split computes each output
    with the same operations in the same order, so batches of 16, 24, 48 and 72 windows give each clip bitwise the
    logit it gets alone."""
    print(f"[gpu] {mode} delta splits: batches of 16 / 24 / 48 / 72 vs one by one", flush=True)
    batch72 = np.concatenate([clips[:64], clips[:8]])
    with shv.Model(weights, mode, experimental=True, max_frames=1440, max_windows=72) as m:
        single = np.concatenate([m.predict(clips[i:i + 1]) for i in range(64)])
        single = np.concatenate([single, single[:8]])
        for n in (16, 24, 48, 72):
            batch = m.predict(batch72[:n])
            assert np.all(np.isfinite(batch))
            assert np.array_equal(batch.view(np.uint32), single[:n].view(np.uint32)), \
                (n, float(np.abs(batch - single[:n]).max()))


@pytest.mark.parametrize("mode", ["fp16", "bf16"])
def test_delta_chunked_matches_sequential(shv, weights, clips, mode, monkeypatch):
    """The half tiers' chunked delta-rule scan (32-token chunks, split-operand matrix cores) against the
    token-by-token kernel (SHV_HIP_DELTA_SEQ=1) on the same tokens: the GDN stage outputs agree to accumulation
    rounding -- 1e-4 of the stage's largest magnitude, where a wrong decay, beta, key or chunk boundary moves them
    by O(1) -- and the logits of 8 windows within 1e-3."""
    print(f"[gpu] {mode} chunked vs token-by-token delta rule", flush=True)
    with shv.Model(weights, "fp32") as m:
        toks = m.encode_frames(clips[:8].reshape(-1, 180, 320, 3)).reshape(8, 20, 16 * 384)
    stages = ("after_gdn_a", "after_gdn_b", "after_sisa_last")
    out = {}
    for seq in (False, True):
        if seq:
            monkeypatch.setenv("SHV_HIP_DELTA_SEQ", "1")
        else:
            monkeypatch.delenv("SHV_HIP_DELTA_SEQ", raising=False)
        with shv.Model(weights, mode, experimental=True, max_frames=160, max_windows=8) as m:
            logits = m.classify(toks)
            with tempfile.TemporaryDirectory() as d:
                m.set_dump_dir(d)
                m.classify(toks[:1])
                dumps = {n: np.fromfile(Path(d) / f"{n}.f32", np.float32) for n in stages}
        out[seq] = (logits, dumps)
    for n in stages:
        a, b = out[False][1][n], out[True][1][n]
        assert np.all(np.isfinite(a)), n
        err = float(np.abs(a - b).max()) / max(1e-30, float(np.abs(b).max()))
        print(f"[gpu] {mode} {n}: max rel diff {err:.2e}", flush=True)
        assert err <= 1e-4, (n, err)
    la, lb = out[False][0], out[True][0]
    print(f"[gpu] {mode} logits max|diff| {float(np.abs(la - lb).max()):.2e}", flush=True)
    assert np.all(np.isfinite(la)) and float(np.abs(la - lb).max()) <= 1e-3


def test_async_pinned_jobs_overlap_capture_and_landing(shv, weights, clips):
    """Jobs from pinned host memory need no staging copy, so the scheduler starts (and, on first use, graph-captures)
    one lane while its completion thread waits on the other lane's events.  Graphs are captured on the engine's own
    stream, so that wait never meets a stream in capture mode.  Four full jobs of 16 clips, twice (capture, then
    replay), give bitwise the logits of predict."""
    import ctypes
    print("[gpu] fp16 async jobs from pinned memory, 4 x 16 clips", flush=True)
    n, per = 64, 16
    with shv.Model(weights, "fp16", experimental=True, max_frames=per * 20, max_windows=per) as m:
        ref = m.predict(clips[:n])
        nbytes = n * 20 * shv.FRAME_BYTES
        ptr = m.lib.shv_hip_host_alloc(nbytes)
        assert ptr
        try:
            host = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(ptr)).reshape(n, 20, shv.FRAME_BYTES)
            host[:] = clips[:n].reshape(n, 20, shv.FRAME_BYTES)
            wf = np.arange(per * 20, dtype=np.int32)
            for rep in range(2):
                out = np.full(n, np.nan, np.float32)
                jobs = [m.submit(frames=host[j:j + per], n_windows=per, window_frames=wf, logits_out=out[j:j + per])
                        for j in range(0, n, per)]
                for job, _ in jobs:
                    assert m.job_wait(job) == 0, m.job_error(job)
                    m.job_free(job)
                assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (rep, float(np.abs(out - ref).max()))
        finally:
            m.lib.shv_hip_host_free(ptr)
