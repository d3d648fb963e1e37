#!/usr/bin/env python3
"""SHIELD-V batched forward benchmark on one MI355X (the headline clips/s metric).

value: clips/s of the full SHIELD-V forward (uint8 crops -> logit) in FP16 at batch 128 clips (2560 frames),
       inputs resident in HBM, through the C-ABI device entry point (shv_hip_forward_device), timed with HIP events
       on the launching stream over exactly --steps forwards after --warmup untimed ones.
extra: batch-1 end-to-end latency through shv_hip_predict (pinned host clip, H2D included, like the reference's
       2.89 ms at README.md:117) in fp16 and in the exact fp32 tier (config 0); the batch-128 fp16 rate end to end
       through shv_hip_predict from pinned host memory (the reference's own method, bench/gpu_bench.cpp:93-117);
       encoder-only frames/s (config 1); the pointwise GEMM microbench on the literal config-2 shapes, the real
       model's 1x1 shapes and the sequence shapes (config 2); sequence-stage windows/s (config 3); bf16 1,024 clips
       through the async API with HBM and MFMA rates and fp32 parity (config 4); the reference CPU engine
       (compiled from the reference sources into oracle/_ref) timed on this host's cores; the SHIELD-A sequence
       stages at 256 windows (fp16 and fp32, device-resident and from host memory) beside the reference SHIELD-A
       engine's CPU sequence; the whole SHIELD-A model from PCM (10 s windows, 128 per batch, device-resident, every
       tier) beside the reference engine's CPU path from PCM; classify alone on 128 N(0,1) windows (fp32, bf16);
       the live-update mode over device token slots (512 participants x 4 / 20 new frames).
roofline: the dominant kernel is the profiling family (one kernel at the shapes the forward gives it) with the
       largest device time per step, from a per-kernel pass with HIP events on the launching stream (graphs off).
       Its algorithmic bytes and FLOPs per launch are recorded by the engine (maps in and out, weights; 2 M N K);
       the binding roof is HBM when its FLOP/byte intensity is below the ridge (MFMA peak / HBM peak), else MFMA.
       `traffic` (HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE, calibrated on a plain device copy)
       is read from profiles/roofline_traffic.json only when that file was measured on this library's compute
       revision and names the same kernel; else null.
Synthetic data: seeded random-init weights in the reference weight-file layout and uniform uint8 crops.
--kernel-only runs just the batch forwards (timed + profiling pass) and an optional device copy of --copy-mb MiB,
so that a rocprofv3 run over it averages exactly the launches this line reports.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E
MFMA_PEAK_TFLOPS = 2500.0       # MI355X dense fp16 / bf16 matrix cores
FP32_PEAK_TFLOPS = 157.3        # MI355X fp32 vector
REF_B128_CLIPS_PER_S = 128 / 0.191   # reference README.md:118 (RTX A6000, batch 128 FP16)
# families of the sequence stages (config 3): the role before ":" for GEMMs
SEQ_ROLES = {"window_input", "rmsnorm", "gemm_seq", "gdn_prep", "delta", "gated_norm", "sisa", "gemm_f32_small", "head"}


def load_shv():
    spec = importlib.util.spec_from_file_location("shv_hip", ROOT / "shield-sisa_amd" / "shv_hip.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["shv_hip"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(weights: Path, clips: np.ndarray, seconds: float) -> dict | None:
    """The reference CPU engine (exact FP32) on this host's cores.  A GPU box's CPU share for one GPU is 16 cores
    whatever the host shows, so the engine gets min(16, visible cores) threads."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    if not oracle.REF_SO.exists():
        return None
    visible = len(os.sched_getaffinity(0))
    threads = max(1, min(16, visible))
    ref = oracle.Reference(weights, threads=threads)
    batch = clips[: min(len(clips), 2 * threads)]
    ref.predict(batch[:1])
    n, t0 = 0, time.perf_counter()
    while True:
        ref.predict(batch)
        n += len(batch)
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    isa = ref.isa
    ref.close()
    return {"value": round(n / dt, 3), "unit": "clips/s", "cores": threads, "kind": "reference",
            "cpu": cpu_model(), "host_cpus_visible": visible,
            "sample": f"reference CPU engine exact FP32 ({isa}), shv_cpu_predict on {len(batch)}-clip batches "
                      f"repeated for {dt:.1f} s ({n} clips), {threads} threads (the box's CPU share for one GPU)"}


def measured_counters(kernel: str, revision: str) -> dict | None:
    """The dominant family's PMC figures (profiles/roofline_traffic.json), when measured on this library revision:
    HBM bytes per launch and, where recorded, the VALU / MFMA busy fractions of its SIMD cycles."""
    path = ROOT / "profiles" / "roofline_traffic.json"
    if not path.exists():
        return None
    try:
        t = json.loads(path.read_text())
    except ValueError:
        return None
    if t.get("revision") != revision or t.get("family") != kernel:
        return None
    return t


# config 2: the pointwise GEMM through the C-ABI tool (bias + hardswish), every tier, on (set, name, M, N, K):
# the literal config-2 shapes (224x224 MobileNetV3 at 2560 frames), the real model's 1x1 layers at 2560 frames of
# 180x320 (engine/cuda/model.hpp:23-29 widths, maps 90x160 .. 6x10) and the sequence GEMMs at 128 windows
# (M = 128 x 321).  The tool takes fp32 A and splits it in the kernel; the engine's sequence GEMMs read A pre-split.
GEMM_SHAPES = [
    ("config2", "b2.expand", 2560 * 28 * 28, 120, 40), ("config2", "b14.expand", 2560 * 7 * 7, 960, 160),
    ("model", "b3.expand", 2560 * 45 * 80, 72, 24), ("model", "b3.project", 2560 * 45 * 80, 24, 72),
    ("model", "b5.expand", 2560 * 23 * 40, 120, 40), ("model", "b5.project", 2560 * 23 * 40, 40, 120),
    ("model", "b7.expand", 2560 * 23 * 40, 240, 40), ("model", "b12.expand", 2560 * 12 * 20, 672, 112),
    ("model", "b12.project", 2560 * 12 * 20, 112, 672), ("model", "b14.expand", 2560 * 6 * 10, 960, 160),
    ("model", "b14.project", 2560 * 6 * 10, 160, 960), ("model", "projection", 2560 * 16, 384, 960),
    ("sequence", "gdn.in_proj", 128 * 321, 2316, 384), ("sequence", "gdn.o_proj", 128 * 321, 384, 768),
    ("sequence", "ffn.up", 128 * 321, 1920, 384), ("sequence", "ffn.down", 128 * 321, 384, 960),
    ("sequence", "sisa.in", 128 * 321, 1068, 384)]


def device_random(hip, rng, rows: int, cols: int, block_rows: int = 1 << 20) -> int:
    """rows x cols fp32 ~ 0.1 N(0,1) in device memory: one host block, repeated on the device."""
    blk = min(rows, block_rows)
    host = (rng.standard_normal((blk, cols), dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    d = hip.malloc(rows * cols * 4)
    src = hip.upload(host)
    for r0 in range(0, rows, blk):
        n = min(blk, rows - r0)
        hip.copy_d2d(d + r0 * cols * 4, src, n * cols * 4)
    hip.sync()
    hip.free(src)
    return d


def gemm_microbench(shv, hip, stream, e0, e1, iters: int = 5) -> list:
    """Per shape and tier: device time per GEMM (HIP events on the launching stream, automatic kernel choice),
    TFLOP/s against the tier's peak (matrix cores for fp16 / bf16, vector fp32 for the exact tier) and the HBM rate
    of its algorithmic bytes (fp32 A and C, W in the tier's parts, bias) against 8 TB/s."""
    rng = np.random.default_rng(3)
    out = []
    for group, name, M, N, K in GEMM_SHAPES:
        dA = device_random(hip, rng, M, K)
        W = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.1)).astype(np.float32)
        b = (rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
        dW, db, dC = hip.upload(W), hip.upload(b), hip.malloc(M * N * 4)
        for mode, wbytes, peak in (("fp16", 4, MFMA_PEAK_TFLOPS), ("bf16", 6, MFMA_PEAK_TFLOPS),
                                   ("fp32", 4, FP32_PEAK_TFLOPS)):
            with shv.PwGemm(mode, dW, N, K, stream) as g:
                g.run(dA, M, dC, db, shv.ACT_HSWISH, stream=stream)
                hip.record(e0, stream)
                for _ in range(iters):
                    g.run(dA, M, dC, db, shv.ACT_HSWISH, stream=stream)
                hip.record(e1, stream)
                ms = hip.elapsed_ms(e0, e1) / iters
            flop = 2.0 * M * N * K
            nbytes = M * K * 4.0 + N * K * wbytes + M * N * 4.0 + N * 4.0
            gbs = nbytes / (ms / 1000.0) / 1e9
            tflops = flop / (ms / 1000.0) / 1e12
            out.append({"set": group, "shape": name, "M": M, "N": N, "K": K, "mode": mode,
                        "us": round(ms * 1000.0, 1), "TFLOP/s": round(tflops, 2), "GB/s": round(gbs, 1),
                        "hbm_frac": round(gbs / HBM_PEAK_GBS, 3), "compute_frac": round(tflops / peak, 4)})
            log(f"[bench] gemm {group}/{name} {mode}: {out[-1]}")
        for p in (dA, dW, db, dC):
            hip.free(p)
    return out


def profile_forward(model, hip, stream, d_frames: int, n_clips: int, d_logits: int, steps: int) -> dict:
    """Per-family device time, bytes and FLOPs of `steps` forwards (HIP events on the launching stream, graphs
    off), summed over each family's launches."""
    model.profile_enable(True)
    for _ in range(steps):
        model.forward_device(d_frames, n_clips, d_logits, stream)
    hip.stream_sync(stream)
    stats = {f: model.profile_read(f) for f in model.profile_families()}
    model.profile_enable(False)
    return {k: v for k, v in stats.items() if v and v["launches"]}


def async_bf16(shv, hip, weights: Path, clips: np.ndarray, n_clips: int = 1024, per_job: int = 128) -> dict:
    """Config 4: n_clips clips in bf16 through the async batched API (shv_hip_submit / job_wait) from pinned host
    memory, per_job clips per request; the scheduler pipelines host copies and compute over its two lanes and
    streams.  Host-to-device copies are included.  HBM and MFMA rates: the algorithmic bytes and FLOPs per clip of a
    bf16 forward (profiling pass of the same model) at the measured clips/s; the matrix cores issue six products per
    bf16 multiply (three operand parts), so issued matrix work is six times the algorithmic FLOPs of the GEMMs.
    Parity: the first 64 clips against the exact fp32 tier."""
    import ctypes
    m = shv.Model(weights, "bf16", experimental=True, max_frames=per_job * 20, max_windows=per_job)
    lib = m.lib
    nbytes = n_clips * 20 * shv.FRAME_BYTES
    ptr = lib.shv_hip_host_alloc(nbytes)
    if not ptr:
        raise shv.ShvError("shv_hip_host_alloc failed")
    try:
        host = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(ptr)).reshape(n_clips, 20, shv.FRAME_BYTES)
        for i in range(0, n_clips, len(clips)):
            k = min(len(clips), n_clips - i)
            host[i:i + k] = clips[:k].reshape(k, 20, shv.FRAME_BYTES)
        logits = np.empty(n_clips, np.float32)
        wf = np.arange(per_job * 20, dtype=np.int32)

        def run():
            jobs = [m.submit(frames=host[j:j + per_job], n_windows=per_job, window_frames=wf,
                             logits_out=logits[j:j + per_job]) for j in range(0, n_clips, per_job)]
            for job, _ in jobs:
                if m.job_wait(job) != 0:
                    raise shv.ShvError(m.job_error(job))
                m.job_free(job)

        run()   # graphs captured
        t0 = time.perf_counter()
        run()
        dt = time.perf_counter() - t0
        npar = min(64, len(clips))
        sub = logits[:npar].copy()
        # algorithmic bytes and FLOPs of one bf16 forward of per_job clips (the scheduler is idle now)
        stream = hip.stream()
        d_frames = hip.upload(np.ascontiguousarray(host[:per_job]))
        d_logits = hip.malloc(per_job * 4)
        stats = profile_forward(m, hip, stream, d_frames, per_job, d_logits, 1)
        hip.free(d_frames)
        hip.free(d_logits)
        hip.stream_destroy(stream)
    finally:
        lib.shv_hip_host_free(ptr)
        m.close()
    with shv.Model(weights, "fp32") as ex:
        ref = ex.predict(clips[:npar])
    flips = int(np.sum((sub >= 0) != (ref >= 0)))
    cps = n_clips / dt
    bytes_clip = sum(v["bytes"] for v in stats.values()) / per_job
    flops_clip = sum(v["flops"] for v in stats.values()) / per_job
    gemm_flops_clip = sum(v["flops"] for k, v in stats.items() if ":" in k) / per_job
    mfma_issued = (gemm_flops_clip * 6.0) * cps / 1e12
    out = {"clips": n_clips, "clips_per_job": per_job, "seconds": round(dt, 4), "clips_per_s": round(cps, 1),
           "h2d_included": True, "h2d_GB_per_s": round(20 * shv.FRAME_BYTES * cps / 1e9, 1),
           "hbm_GB_per_s_algorithmic": round(bytes_clip * cps / 1e9, 1),
           "hbm_frac_algorithmic": round(bytes_clip * cps / 1e9 / HBM_PEAK_GBS, 4),
           "algorithmic_bytes_per_clip": round(bytes_clip), "algorithmic_flops_per_clip": round(flops_clip),
           "mfma_TFLOP_per_s_algorithmic": round(flops_clip * cps / 1e12, 1),
           "mfma_util_algorithmic": round(flops_clip * cps / 1e12 / MFMA_PEAK_TFLOPS, 4),
           "mfma_TFLOP_per_s_issued": round(mfma_issued, 1),
           "mfma_util_issued": round(mfma_issued / MFMA_PEAK_TFLOPS, 4),
           "parity_clips": npar, "parity_max_abs_vs_fp32": float(np.abs(sub - ref).max()), "parity_flips": flips}
    log(f"[bench] config 4 bf16 async: {out}")
    return out


def latency_b1(shv, weights: Path, clip: np.ndarray, mode: str, iters: int) -> dict:
    """Batch-1 latency through shv_hip_predict from a pinned host clip (H2D included), p50 / p95 over `iters`
    calls after 10 warm-up calls (the reference's method: README.md:117, bench/gpu_bench.cpp:93-117)."""
    with shv.Model(weights, mode, experimental=mode != "fp32") as m:
        lib = m.lib
        p = lib.shv_hip_host_alloc(20 * shv.FRAME_BYTES)
        pinned = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_uint8 * (20 * shv.FRAME_BYTES)).from_address(p))
        pinned[:] = clip.reshape(-1)
        out = np.empty(1, np.float32)
        try:
            for _ in range(10):
                if lib.shv_hip_predict(m.h, p, 1, out.ctypes.data) != 0:
                    raise shv.ShvError(shv.last_error())
            ts = []
            for _ in range(iters):
                t0 = time.perf_counter()
                lib.shv_hip_predict(m.h, p, 1, out.ctypes.data)
                ts.append((time.perf_counter() - t0) * 1000.0)
        finally:
            lib.shv_hip_host_free(p)
    r = {"mode": mode, "p50_ms": round(float(np.percentile(ts, 50)), 3), "p95_ms": round(float(np.percentile(ts, 95)), 3),
         "iters": iters, "logit": float(out[0])}
    log(f"[bench] batch-1 latency {mode}: {r}")
    return r


def predict_e2e(shv, weights: Path, clips: np.ndarray, mode: str, max_frames: int, max_windows: int,
                reps: int = 5) -> dict:
    """Batch of clips end to end through shv_hip_predict from pinned host memory (H2D and D2H included), wall
    clock per call: the reference's measurement of its 191 ms / 128 clips (bench/gpu_bench.cpp:93-117)."""
    import ctypes
    n = len(clips)
    with shv.Model(weights, mode, experimental=mode != "fp32", max_frames=max_frames, max_windows=max_windows) as m:
        lib = m.lib
        nbytes = n * 20 * shv.FRAME_BYTES
        p = lib.shv_hip_host_alloc(nbytes)
        host = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(p))
        host[:] = clips.reshape(-1)
        out = np.empty(n, np.float32)
        try:
            for _ in range(2):
                if lib.shv_hip_predict(m.h, p, n, out.ctypes.data) != 0:
                    raise shv.ShvError(shv.last_error())
            t0 = time.perf_counter()
            for _ in range(reps):
                lib.shv_hip_predict(m.h, p, n, out.ctypes.data)
            dt = (time.perf_counter() - t0) / reps
        finally:
            lib.shv_hip_host_free(p)
    per_batch = min(max_windows, max_frames // 20)
    r = {"mode": mode, "clips": n, "ms": round(dt * 1000.0, 3), "clips_per_s": round(n / dt, 1),
         "options": {"max_frames": max_frames, "max_windows": max_windows}, "clips_per_gpu_batch": per_batch,
         "h2d_included": True, "finite": bool(np.isfinite(out).all())}
    log(f"[bench] predict end to end: {r}")
    return r


def crop_bench(shv, hip, stream, model, clips_n: int, d_logits: int, iters: int = 5) -> dict:
    """Face crops on the GPU (shv_hip_native_crops_rgb): clips_n x 20 crops (a batch's worth) from 20 distinct
    1920x1080 native frames resident in HBM (INTER_AREA canvas shrink, then the 320x180 crop), rects of the
    reference's crop_geometry family (crop height 101 -> 180x101 letterbox units); wall clock per call (the entry
    point returns when the crops are written).  Then the device-only pipeline: crops straight into the model's
    input layout + the forward (frames -> logits).  Beside it, the reference CPU crop (oracle/_ref,
    shv_native_crop_rgb) on one host core over a bounded sample."""
    rng = np.random.default_rng(7)
    W, H, n = 1920, 1080, clips_n * 20
    frames = [hip.upload(rng.integers(0, 256, (H, W, 3), dtype=np.uint8)) for _ in range(20)]
    rects = [(int(rng.integers(0, 320 - 180 + 1)), int(rng.integers(0, 180 - 101 + 1)), 180, 101) for _ in range(n)]
    fr = [(frames[i % 20], W, H, 3 * W) for i in range(n)]
    d_crops = hip.malloc(n * shv.FRAME_BYTES)
    shv.native_crops_rgb(fr, rects, d_crops, stream)
    t0 = time.perf_counter()
    for _ in range(iters):
        shv.native_crops_rgb(fr, rects, d_crops, stream)
    crop_s = (time.perf_counter() - t0) / iters
    model.forward_device(d_crops, clips_n, d_logits, stream)
    hip.stream_sync(stream)
    t0 = time.perf_counter()
    for _ in range(iters):
        shv.native_crops_rgb(fr, rects, d_crops, stream)
        model.forward_device(d_crops, clips_n, d_logits, stream)
    hip.stream_sync(stream)
    pipe_s = (time.perf_counter() - t0) / iters
    out = {"crops": n, "native": f"{W}x{H}", "rect": "180x101", "ms_per_call": round(crop_s * 1000, 3),
           "crops_per_s": round(n / crop_s, 1), "pipeline_ms_per_batch": round(pipe_s * 1000, 3),
           "pipeline_clips_per_s": round(clips_n / pipe_s, 1)}
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    if oracle.PREP_SO.exists():
        ref = oracle.PrepRef()
        host = [rng.integers(0, 256, (H, W, 3), dtype=np.uint8) for _ in range(4)]
        k, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 2.0:
            ref.native_crop(host[k % 4], rects[k % n])
            k += 1
        out["cpu_reference_crops_per_s_1core"] = round(k / (time.perf_counter() - t0), 1)
    log(f"[bench] crops: {out}")
    for f in frames:
        hip.free(f)
    hip.free(d_crops)
    return out


AUDIO_WINDOWS = 256


def audio_cpu_baseline(weights: Path, tokens: np.ndarray, seconds: float) -> dict | None:
    """The reference SHIELD-A engine's sequence stages (exact mode, compiled from the reference sources into
    oracle/_ref) on this host's cores: one window per call, min(16, visible cores) calls in flight (the engine's
    workspace is per thread; the box's CPU share for one GPU is 16 cores)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from concurrent.futures import ThreadPoolExecutor
    if not oracle.AUDIO_SO.exists():
        return None
    visible = len(os.sched_getaffinity(0))
    threads = max(1, min(16, visible))
    ref = oracle.AudioReference(weights)
    ref.sequence(tokens[0])
    n, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        while time.perf_counter() - t0 < seconds:
            list(ex.map(lambda i: ref.sequence(tokens[i % len(tokens)]), range(n, n + 4 * threads)))
            n += 4 * threads
    dt = time.perf_counter() - t0
    ref.close()
    return {"value": round(n / dt, 2), "unit": "windows/s", "cores": threads, "kind": "reference",
            "cpu": cpu_model(), "host_cpus_visible": visible,
            "sample": f"reference SHIELD-A shield::sequence, exact mode, {n} windows in {dt:.1f} s on {threads} "
                      f"threads (one window per call)"}


def audio_bench(shv, hip, stream, e0, e1, steps: int, revision: str, cpu_seconds: float | None) -> dict:
    """Row f4: the SHIELD-A sequence stages (125 tokens + readout -> logit per window) at 256 windows from HBM through
    shv_hip_audio_sequence_device, fp16 and fp32; the same from pageable host memory (PCIe inclusive); the roofline
    of the dominant kernel family; the reference's CPU sequence beside it."""
    out = {"workload": f"shielda_sequence_b{AUDIO_WINDOWS}", "windows": AUDIO_WINDOWS, "tokens_per_window": 126,
           "data": "synthetic (seeded SHLDA001 sequence weights, N(0,1) tokens)"}
    with tempfile.TemporaryDirectory() as td:
        w = Path(td) / "audio.shlda"
        shv.write_audio_weights(w, 5)
        toks = shv.audio_tokens(AUDIO_WINDOWS, 17)
        d_tok = hip.upload(toks)
        d_out = hip.malloc(AUDIO_WINDOWS * 4)
        for mode in ("fp16", "fp32"):
            log(f"[bench] audio {mode}: {AUDIO_WINDOWS} windows")
            m = shv.AudioModel(w, mode, max_windows=AUDIO_WINDOWS, experimental=mode != "fp32")
            for _ in range(3):
                m.sequence_device(d_tok, AUDIO_WINDOWS, d_out, stream=stream)
            hip.stream_sync(stream)
            hip.record(e0, stream)
            for _ in range(steps):
                m.sequence_device(d_tok, AUDIO_WINDOWS, d_out, stream=stream)
            hip.record(e1, stream)
            ms = hip.elapsed_ms(e0, e1) / steps
            m.profile_enable(True)
            m.sequence_device(d_tok, AUDIO_WINDOWS, d_out, stream=stream)
            hip.stream_sync(stream)
            stats = {f: m.profile_read(f) for f in m.profile_families()}
            m.profile_enable(False)
            stats = {k: v for k, v in stats.items() if v and v["launches"]}
            fam = {k: round(v["ms"], 3) for k, v in sorted(stats.items(), key=lambda kv: -kv[1]["ms"])}
            m.sequence(toks)
            t0 = time.perf_counter()
            host_logits = m.sequence(toks)
            host_s = time.perf_counter() - t0
            out[mode] = {"windows_per_s": round(AUDIO_WINDOWS / (ms / 1000.0), 1), "ms_per_batch": round(ms, 4),
                         "host_memory_windows_per_s": round(AUDIO_WINDOWS / host_s, 1),
                         "finite": bool(np.isfinite(host_logits).all()), "family_ms": fam,
                         "roofline": roofline_of(stats, 1, mode, revision, traffic_file=False)}
            log(f"[bench] audio {mode}: {ms:.3f} ms / {AUDIO_WINDOWS} windows -> "
                f"{out[mode]['windows_per_s']} windows/s; dominant {out[mode]['roofline']['kernel']}")
            m.close()
        hip.free(d_tok)
        hip.free(d_out)
        if cpu_seconds:
            out["cpu_baseline"] = audio_cpu_baseline(w, toks, cpu_seconds)
    return out


AUDIO_PCM_WINDOWS = 128


def audio_pcm_cpu_baseline(weights: Path, pcm: np.ndarray, seconds: float) -> dict | None:
    """The reference SHIELD-A engine from PCM (frontend + sequence, exact mode, compiled from the reference sources
    into oracle/_ref) on this host's cores: one window per call, min(16, visible cores) calls in flight."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from concurrent.futures import ThreadPoolExecutor
    if not oracle.AUDIO_SO.exists():
        return None
    visible = len(os.sched_getaffinity(0))
    threads = max(1, min(16, visible))
    ref = oracle.AudioReference(weights)
    ref.predict(pcm[:1])
    n, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        while time.perf_counter() - t0 < seconds:
            list(ex.map(lambda i: ref.predict(pcm[i % len(pcm):i % len(pcm) + 1]), range(n, n + 2 * threads)))
            n += 2 * threads
    dt = time.perf_counter() - t0
    ref.close()
    return {"value": round(n / dt, 2), "unit": "windows/s", "cores": threads, "kind": "reference",
            "cpu": cpu_model(), "host_cpus_visible": visible,
            "sample": f"reference SHIELD-A PCM -> logit (frontend_cnn + sequence), exact mode, {n} windows in "
                      f"{dt:.1f} s on {threads} threads (one window per call)"}


def audio_pcm_bench(shv, hip, stream, e0, e1, steps: int, revision: str, cpu_seconds: float | None) -> dict:
    """Row f4, the whole SHIELD-A model: 10 s windows of 16 kHz PCM resident in HBM -> logits through
    shv_hip_audio_predict_device (log-mel, CNN, frequency attention, tokens, sequence stages) in every tier; HIP events
    on the launching stream; the roofline of the dominant kernel family; the reference's CPU path beside it."""
    out = {"workload": f"shielda_pcm_b{AUDIO_PCM_WINDOWS}", "windows": AUDIO_PCM_WINDOWS,
           "samples_per_window": 160000, "inputs": "device-resident (HBM)", "entry": "shv_hip_audio_predict_device",
           "data": "synthetic (seeded SHLDA001 whole-model weights, PCM N(0, 0.1^2) clipped to [-1, 1])"}
    with tempfile.TemporaryDirectory() as td:
        w = Path(td) / "audio_model.shlda"
        shv.write_audio_model_weights(w, 5)
        pcm = shv.audio_pcm(AUDIO_PCM_WINDOWS, 23)
        d_pcm = hip.upload(pcm)
        d_out = hip.malloc(AUDIO_PCM_WINDOWS * 4)
        for mode in ("fp16", "bf16", "fp32"):
            log(f"[bench] audio PCM {mode}: {AUDIO_PCM_WINDOWS} windows")
            m = shv.AudioModel(w, mode, max_windows=AUDIO_PCM_WINDOWS, experimental=mode != "fp32")
            for _ in range(2):
                m.predict_device(d_pcm, AUDIO_PCM_WINDOWS, d_out, stream=stream)
            hip.stream_sync(stream)
            hip.record(e0, stream)
            for _ in range(steps):
                m.predict_device(d_pcm, AUDIO_PCM_WINDOWS, d_out, stream=stream)
            hip.record(e1, stream)
            ms = hip.elapsed_ms(e0, e1) / steps
            logits = hip.download(d_out, AUDIO_PCM_WINDOWS, np.float32)
            m.profile_enable(True)
            m.predict_device(d_pcm, AUDIO_PCM_WINDOWS, d_out, stream=stream)
            hip.stream_sync(stream)
            stats = {f: m.profile_read(f) for f in m.profile_families()}
            m.profile_enable(False)
            stats = {k: v for k, v in stats.items() if v and v["launches"]}
            fam = {k: round(v["ms"], 3) for k, v in sorted(stats.items(), key=lambda kv: -kv[1]["ms"])}
            wps = AUDIO_PCM_WINDOWS / (ms / 1000.0)
            out[mode] = {"windows_per_s": round(wps, 1), "ms_per_batch": round(ms, 4),
                         "audio_seconds_per_s": round(wps * 10.0, 1), "finite": bool(np.isfinite(logits).all()),
                         "family_ms": fam, "roofline": roofline_of(stats, 1, mode, revision, traffic_file=False)}
            log(f"[bench] audio PCM {mode}: {ms:.3f} ms / {AUDIO_PCM_WINDOWS} windows -> {wps:.0f} windows/s; "
                f"dominant {out[mode]['roofline']['kernel']}")
            m.close()
        hip.free(d_pcm)
        hip.free(d_out)
        if cpu_seconds:
            out["cpu_baseline"] = audio_pcm_cpu_baseline(w, pcm, cpu_seconds)
    return out


def config3_classify(shv, hip, stream, e0, e1, weights: Path, steps: int, windows: int = 128) -> dict:
    """The classify-only workload: the GDN + SISA sequence stages alone on `windows` windows of N(0,1) tokens resident in
    HBM (shv_hip_classify_device, one pass of windows * 321 rows), in the exact tier (fp32 activations and
    arithmetic) and the bf16 tier; HIP events on the launching stream."""
    rng = np.random.default_rng(33)
    toks = rng.standard_normal((windows, 20, 16, 384)).astype(np.float32)
    d_tok = hip.upload(toks)
    d_lg = hip.malloc(windows * 4)
    out = {"windows": windows, "tokens_per_window": 321, "d_model": 384, "inputs": "device-resident (HBM)",
           "entry": "shv_hip_classify_device", "data": "N(0,1) tokens, seed 33"}
    try:
        for mode in ("fp32", "bf16"):
            with shv.Model(weights, mode, experimental=mode != "fp32", max_frames=20, max_windows=windows) as m:
                for _ in range(2):
                    m.classify_device(d_tok, windows, d_lg, stream)
                hip.stream_sync(stream)
                hip.record(e0, stream)
                for _ in range(steps):
                    m.classify_device(d_tok, windows, d_lg, stream)
                hip.record(e1, stream)
                ms = hip.elapsed_ms(e0, e1) / steps
                lg = hip.download(d_lg, windows, np.float32)
            out[mode] = {"ms_per_batch": round(ms, 4), "windows_per_s": round(windows / (ms / 1000.0), 1),
                         "finite": bool(np.isfinite(lg).all())}
            log(f"[bench] config 3 {mode}: {ms:.3f} ms / {windows} windows -> {out[mode]['windows_per_s']} windows/s")
    finally:
        hip.free(d_tok)
        hip.free(d_lg)
    return out


def live_update(shv, weights: Path, mode: str = "fp16", participants: int = 512, hops: int = 3,
                new_frames=(4, 20)) -> dict:
    """The reference's live mode (bench/gpu_bench.cpp:142-218; docs/PERFORMANCE.md:34-36): participant p owns
    device token slots [24 p, 24 p + 24) as a ring; a warm-up hop stores every participant's first 20 frames; then
    each hop, all participants at once (burst), submits one job per participant that encodes its `new` frames from
    pinned host memory into the next slots and classifies the window of its last 20 frames from the slots.  Latency
    per job = queue + run time (shv_hip_job_timing), the reference's measure; the model runs with the reference's
    default options and participants * 24 token slots.  Requests are built before a hop starts, so the submit
    loop is a few microseconds per job."""
    import ctypes
    distinct = 16
    res = {"mode": mode, "participants": participants, "hops": hops, "arrival": "burst",
           "entry": "shv_hip_submit (token slots)", "reference_p99_ms": {"4": 221.0, "20": 705.0},
           "reference_hardware": "RTX A6000 (docs/PERFORMANCE.md:34-36)"}
    with shv.Model(weights, mode, experimental=mode != "fp32", token_slots=participants * 24) as m:
        lib = m.lib
        nbytes = distinct * 20 * shv.FRAME_BYTES
        hp = lib.shv_hip_host_alloc(nbytes)
        src = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(hp))
        src[:] = shv.synth_clips(distinct, 2000).reshape(-1)
        logit = np.empty(participants, np.float32)
        try:
            for newf in new_frames:
                nframes = np.zeros(participants, np.int64)

                def build(pi: int, nnew: int):
                    store = np.array([pi * 24 + int((nframes[pi] + i) % 24) for i in range(nnew)], np.int32)
                    last = int(nframes[pi]) + nnew
                    wslots = np.array([pi * 24 + (last - 20 + t) % 24 for t in range(20)], np.int32)
                    f0 = int(nframes[pi]) % (distinct * 20 - nnew)
                    r = shv.Request()
                    r.frames = hp + f0 * shv.FRAME_BYTES
                    r.n_frames = nnew
                    r.store_slots = store.ctypes.data
                    r.n_windows = 1
                    r.window_slots = wslots.ctypes.data
                    r.logits_out = logit.ctypes.data + 4 * pi
                    nframes[pi] = last
                    return r, store, wslots

                def run_hop(reqs):
                    jobs = [lib.shv_hip_submit(m.h, ctypes.byref(q[0])) for q in reqs]
                    if not all(jobs):
                        raise shv.ShvError(shv.last_error())
                    out = []
                    for j in jobs:
                        if lib.shv_hip_job_wait(j) != 0:
                            raise shv.ShvError(lib.shv_hip_job_error(j).decode())
                        q, r, g = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
                        bf, bw = ctypes.c_int(), ctypes.c_int()
                        lib.shv_hip_job_timing(j, ctypes.byref(q), ctypes.byref(r), ctypes.byref(g), ctypes.byref(bf),
                                               ctypes.byref(bw))
                        out.append((q.value + r.value, q.value, g.value, bw.value))
                        lib.shv_hip_job_free(j)
                    return out

                run_hop([build(pi, 20) for pi in range(participants)])   # warm-up: 20 frames each
                rows = []
                t0 = time.perf_counter()
                for _ in range(hops):
                    rows += run_hop([build(pi, newf) for pi in range(participants)])
                wall = (time.perf_counter() - t0) * 1000.0
                lat = np.array([x[0] for x in rows])
                r = {"lat_p50_ms": round(float(np.percentile(lat, 50)), 3),
                     "lat_p95_ms": round(float(np.percentile(lat, 95)), 3),
                     "lat_p99_ms": round(float(np.percentile(lat, 99)), 3), "lat_max_ms": round(float(lat.max()), 3),
                     "queue_p50_ms": round(float(np.percentile([x[1] for x in rows], 50)), 3),
                     "batch_gpu_p50_ms": round(float(np.percentile([x[2] for x in rows], 50)), 3),
                     "mean_batch_windows": round(float(np.mean([x[3] for x in rows])), 1),
                     "wall_ms": round(wall, 1), "finite": bool(np.isfinite(logit).all())}
                res[str(newf)] = r
                log(f"[bench] live {mode}: {participants} participants x {newf} new frames: {r}")
        finally:
            lib.shv_hip_host_free(hp)
    return res


def roofline_of(stats: dict, steps: int, mode: str, revision: str, traffic_file: bool = True) -> dict:
    """The family with the most device time per step, against the roof its intensity selects."""
    dom = max(stats, key=lambda k: stats[k]["ms"])
    d = stats[dom]
    avg_ms = d["ms"] / d["launches"]
    bytes_l = d["bytes"] / d["launches"]
    flops_l = d["flops"] / d["launches"]
    gbs = bytes_l / (avg_ms / 1000.0) / 1e9
    tflops = flops_l / (avg_ms / 1000.0) / 1e12
    peak_tf = FP32_PEAK_TFLOPS if mode == "fp32" else MFMA_PEAK_TFLOPS
    ridge = peak_tf * 1e12 / (HBM_PEAK_GBS * 1e9)
    intensity = flops_l / bytes_l if bytes_l else 0.0
    counters = measured_counters(dom, revision) if traffic_file else None
    traffic = float(counters["traffic_bytes_per_launch"]) if counters else None
    if intensity < ridge:
        r = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
             "frac": round(gbs / HBM_PEAK_GBS, 4)}
    else:
        r = {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak_tf, "unit": "TFLOP/s",
             "frac": round(tflops / peak_tf, 4)}
    r.update({"traffic": None if traffic is None else round(traffic), "kernel": dom,
              "algorithmic_bytes_per_launch": round(bytes_l), "algorithmic_flops_per_launch": round(flops_l),
              "intensity_flop_per_byte": round(intensity, 1), "ridge_flop_per_byte": round(ridge, 1),
              "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "compute_frac": round(tflops / peak_tf, 4),
              "avg_launch_ms": round(avg_ms, 4), "launches_per_step": d["launches"] // steps,
              "ms_per_step": round(d["ms"] / steps, 4)})
    # what issue-bound kernels are bound by: the fraction of SIMD cycles issuing VALU / MFMA work (PMC)
    for k in ("valu_busy_frac", "mfma_busy_frac"):
        if counters and k in counters:
            r[k] = counters[k]
    return r


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=128)
    ap.add_argument("--mode", default="fp16", choices=["fp16", "bf16", "fp32"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--latency-iters", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-only", action="store_true")
    ap.add_argument("--copy-mb", type=int, default=0)
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-async", action="store_true")
    ap.add_argument("--no-crop", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--no-audio", action="store_true")
    ap.add_argument("--no-live", action="store_true")
    ap.add_argument("--gemm-only", action="store_true", help="only the GEMM microbench (config 2 and the model / "
                    "sequence shapes), for a kernel trace of its launches")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every GPU box here has one GPU, and the SHIELD-V forward has no "
              "cross-GPU step (clips are independent rows; each GPU would run its own model); run with --gpus 1",
              file=sys.stderr)
        return 2

    shv = load_shv()
    hip = shv.Hip()
    B = args.batch
    revision = shv.library().shv_hip_compute_revision().decode()
    if args.gemm_only:
        stream = hip.stream()
        e0, e1 = hip.event(), hip.event()
        print(json.dumps({"gemm_microbench": gemm_microbench(shv, hip, stream, e0, e1), "revision": revision}),
              flush=True)
        return 0
    with tempfile.TemporaryDirectory() as td:
        w = Path(td) / "bench.weights"
        shv.write_weights(w, seed=1, threshold=0.5)
        clips = shv.synth_clips(B, 1000)
        log(f"[bench] load {args.mode} model, batch {B} clips, revision {revision}")
        model = shv.Model(w, args.mode, experimental=args.mode != "fp32", max_frames=B * 20, max_windows=B)
        stream = hip.stream()
        d_frames = hip.upload(clips)
        d_logits = hip.malloc(B * 4)
        e0, e1 = hip.event(), hip.event()
        hip.sync()
        for _ in range(args.warmup):
            model.forward_device(d_frames, B, d_logits, stream)
        hip.stream_sync(stream)
        log("[bench] warmup done")
        hip.record(e0, stream)
        for _ in range(args.steps):
            model.forward_device(d_frames, B, d_logits, stream)
        hip.record(e1, stream)
        total_ms = hip.elapsed_ms(e0, e1)
        hip.sync()
        ms = total_ms / args.steps
        value = B / (ms / 1000.0)
        logits = hip.download(d_logits, B, np.float32)
        log(f"[bench] {ms:.3f} ms/step -> {value:.1f} clips/s; finite logits {np.isfinite(logits).all()}")

        # per-kernel timing with HIP events on the launching stream (graphs off while profiling)
        prof_steps = max(1, min(args.steps, 3))
        stats = profile_forward(model, hip, stream, d_frames, B, d_logits, prof_steps)
        per_step = {k: round(v["ms"] / prof_steps, 3) for k, v in sorted(stats.items(), key=lambda kv: -kv[1]["ms"])}
        log("[bench] per-step ms by kernel family: " + json.dumps(per_step))
        seq_ms = sum(v["ms"] for k, v in stats.items() if k.split(":")[0] in SEQ_ROLES) / prof_steps
        seq_wps = B / (seq_ms / 1000.0)
        log(f"[bench] sequence stages {seq_ms:.3f} ms / {B} windows -> {seq_wps:.0f} windows/s")
        roofline = roofline_of(stats, prof_steps, args.mode, revision)
        log("[bench] roofline " + json.dumps(roofline))

        copy = None
        if args.copy_mb > 0:   # plain device copy: calibrates the PMC byte counters and shows achievable HBM rate
            nbytes = args.copy_mb << 20
            src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
            hip.memset(src, 1, nbytes)
            hip.copy_d2d(dst, src, nbytes, stream)
            hip.stream_sync(stream)
            hip.record(e0, stream)
            for _ in range(5):
                hip.copy_d2d(dst, src, nbytes, stream)
            hip.record(e1, stream)
            cms = hip.elapsed_ms(e0, e1) / 5
            copy = {"bytes": nbytes, "ms": round(cms, 4), "GB/s": round(2 * nbytes / (cms / 1000.0) / 1e9, 1)}
            log(f"[bench] device copy {args.copy_mb} MiB: {cms:.3f} ms -> {copy['GB/s']} GB/s (read + write)")
            hip.free(src)
            hip.free(dst)

        crops = None if args.kernel_only or args.no_crop else crop_bench(shv, hip, stream, model, B, d_logits)

        enc_ms = None
        if not args.kernel_only:   # encoder only (config 1: 2560 frames)
            d_tok = hip.malloc(B * 20 * 6144 * 4)
            model.encode_device(d_frames, B * 20, d_tok, stream)
            hip.stream_sync(stream)
            enc_steps = max(3, args.steps // 2)
            hip.record(e0, stream)
            for _ in range(enc_steps):
                model.encode_device(d_frames, B * 20, d_tok, stream)
            hip.record(e1, stream)
            enc_ms = hip.elapsed_ms(e0, e1) / enc_steps
            log(f"[bench] encoder {enc_ms:.3f} ms / {B * 20} frames")
            hip.free(d_tok)
        model.close()
        hip.free(d_frames)
        hip.free(d_logits)
        c3 = None if args.kernel_only else config3_classify(shv, hip, stream, e0, e1, w, max(3, args.steps // 2))
        gemm = None if args.kernel_only or args.no_gemm else gemm_microbench(shv, hip, stream, e0, e1)
        audio = audio_pcm = None
        if not args.kernel_only and not args.no_audio:
            audio = audio_bench(shv, hip, stream, e0, e1, max(3, args.steps // 2), revision,
                                None if args.no_cpu else min(5.0, args.cpu_seconds))
            audio_pcm = audio_pcm_bench(shv, hip, stream, e0, e1, max(3, args.steps // 2), revision,
                                        None if args.no_cpu else min(5.0, args.cpu_seconds))
        hip.stream_destroy(stream)

        lat = lat32 = None
        if not args.kernel_only and args.latency_iters > 0:
            lat = latency_b1(shv, w, clips[0], args.mode, args.latency_iters)
            lat32 = latency_b1(shv, w, clips[0], "fp32", args.latency_iters)   # config 0: the exact tier

        e2e = None
        if not args.kernel_only and not args.no_e2e:
            # the reference's defaults split 128 clips into 4 GPU batches of 32 pipelined over 2 lanes; beside it
            # the same 128 clips as one GPU batch
            e2e = {"reference_options": predict_e2e(shv, w, clips, args.mode, 640, 512),
                   "one_gpu_batch": predict_e2e(shv, w, clips, args.mode, B * 20, B)}

        c4 = None
        if not args.kernel_only and not args.no_async:
            c4 = async_bf16(shv, hip, w, clips)

        live = None
        if not args.kernel_only and not args.no_live:
            live = live_update(shv, w, args.mode)

        cpu = None
        if not args.no_cpu and not args.kernel_only:
            cpu = cpu_baseline(w, clips, args.cpu_seconds)

    line = {
        "metric": "SHIELD-V clips/sec at batch 128 FP16 on 1 MI355X; batch-1 latency (ms)",
        "value": round(value, 2),
        "unit": "clips/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.mode,
        "data": "synthetic (seeded random-init weights in the SHLDV001 layout, uniform uint8 crops)",
        "config": {"workload": f"shieldv_forward_{args.mode}_b{B}", "clips": B, "frames_per_clip": 20,
                   "crop": "180x320x3 uint8", "tokens_per_window": 321, "d_model": 384,
                   "inputs": "device-resident (HBM)", "entry": "shv_hip_forward_device",
                   "reference_gpu_clips_per_s": round(REF_B128_CLIPS_PER_S, 1)},
        "latency_b1_ms": None if lat is None else lat["p50_ms"],
        "latency_b1_fp32_ms": None if lat32 is None else lat32["p50_ms"],
        "latency_b1": {"fp16": lat, "fp32": lat32} if lat else None,
        "predict_b128_e2e": e2e,
        "encoder_frames_per_s": None if enc_ms is None else round(B * 20 / (enc_ms / 1000.0), 1),
        "sequence_windows_per_s_in_forward": round(seq_wps, 1),
        "config3_classify": c3,
        "live_update": live,
        "async_bf16_1024": c4,
        "family_ms_per_step": per_step,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "device_copy": copy,
        "gemm_microbench": gemm,
        "face_crops": crops,
        "shielda_sequence": audio,
        "shielda_pcm": audio_pcm,
        "revision": revision,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
