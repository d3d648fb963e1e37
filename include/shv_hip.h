/*
 * shv_hip.h -- SHIELD-V video detector, MI355X (gfx950) HIP inference engine, C API (libshield_v_hip.so).
 *
 * Drop-in counterpart of the reference CUDA engine API (engine/include/shv_cuda.h:74-151): every function,
 * struct and constant below replaces the shv_cuda_* item of the same suffix, with the same argument meaning,
 * the same struct layouts and the same error behaviour.  Per-item citations name the replaced declaration.
 *
 * Function: uint8 RGB crops [20][180][320][3] -> MobileNetV3-Large features (folded BatchNorm) -> 4x4 pool ->
 * Linear 960->384 = 16 tokens per frame -> + (time + row) + col, readout -> GDN-A -> GDN-B x2 -> SISA (last row)
 * -> RMSNorm -> head -> logit.  Decision (caller side): score = sigmoid(logit) in double, alert iff
 * score >= shv_hip_threshold(m).  A NaN logit means "unavailable" (failed job or non-finite result).
 *
 * MODES: "fp32" = IEEE fp32 everywhere, same per-element operation order as the reference CPU exact engine
 * (GEMM K blocks of 64, the same reduction trees); always loadable.  "bf16" / "fp16" = every convolution and
 * all-row GEMM, and the chunked delta-rule scan, on the matrix cores in that type with fp32 accumulation: each fp32
 * operand is carried as 3 (bf16) or 2 (fp16) parts of that type, each part the rounding of what the earlier parts
 * leave, and the significant part products are issued as separate MFMAs, so operands keep fp32-level precision.
 * Activations are stored in fp32 in every mode; residual stream, norms, recurrences, SISA last row and head are
 * fp32, SISA prefix sums double.  Approximate modes load only with a passing certificate line
 *   "<weights sha256> <mode> <shv_hip_compute_revision()> PASS <cert json> <cert json sha256> threshold=<%.17g>"
 * in "<weights>.hip.cert" (first line "SHIELDV_HIP_CERT_V2") whose threshold equals the loaded one exactly.
 * SIDECAR "<weights>.json": "output_sha256" must equal the weight file's SHA-256 and "threshold" must be present,
 * finite and in (0, 1), in every mode.
 *
 * ROW INDEPENDENCE: the logit of a window and the tokens of a frame are bitwise identical whatever else is in
 * the batch (size, order, padding, coalescing), in every mode: no split-K, fixed reduction orders, no atomics.
 *
 * THREADING AND LIFETIMES: as the reference contract (engine/include/shv_cuda.h:36-59).  One worker thread per
 * model drives a copy stream and a compute stream; jobs run in FIFO order and consecutive jobs coalesce into one
 * GPU batch up to the limits; callbacks run on the worker thread; every job is freed exactly once with
 * shv_hip_job_free; shv_hip_free completes queued jobs first; errors are thread-local.
 *
 * DEVICE TOKEN SLOTS (options.token_slots > 0): a pool of 16x384 fp32 token blocks resident in HBM, written by
 * store_slots and read by window_slots, with the reference's hazard rule for coalescing.
 */
#ifndef SHV_HIP_H
#define SHV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* constants: shv_cuda.h:74-77 */
#define SHV_HIP_API_VERSION 1
#define SHV_HIP_FRAME_BYTES 172800    /* 180 x 320 x 3 uint8 RGB */
#define SHV_HIP_TOKEN_FLOATS 6144     /* 16 tokens x 384, one frame */
#define SHV_HIP_WINDOW_FRAMES 20

typedef struct shv_hip_model shv_hip_model;   /* shv_cuda.h:79 */
typedef struct shv_hip_job shv_hip_job;       /* shv_cuda.h:80 */

/* shv_cuda.h:82-89 (same fields, same defaults) */
typedef struct shv_hip_options {
    int max_frames;       /* frames per GPU batch (CNN); default 640 */
    int max_windows;      /* windows per GPU batch (sequence); default 512 */
    int max_host_tokens;  /* host-provided token blocks per GPU batch; default 2048 */
    int token_slots;      /* device token slots (0 = none); default 0 */
    int use_graphs;       /* HIP graphs per batch bucket; default 1 */
    int max_delay_us;     /* scheduler: wait up to this long for more jobs before launching; default 0 */
} shv_hip_options;

void shv_hip_default_options(shv_hip_options* opt);                                     /* shv_cuda.h:91 */
/* weights: SHLDV001 file (+ "<weights>.json").  mode: "fp32" | "bf16" | "fp16" (NULL = "fp32").
 * device: HIP device ordinal.  NULL on error. */
shv_hip_model* shv_hip_load(const char* weights, const char* mode, int device);          /* shv_cuda.h:94 */
shv_hip_model* shv_hip_load_ex(const char* weights, const char* mode, int device,
                               const shv_hip_options* opt);                              /* shv_cuda.h:95 */
void shv_hip_free(shv_hip_model* m);                                                     /* shv_cuda.h:96 */

const char* shv_hip_last_error(void);                                                    /* shv_cuda.h:98 */
const char* shv_hip_mode(const shv_hip_model* m);                                        /* shv_cuda.h:99 */
const char* shv_hip_fingerprint(const shv_hip_model* m);  /* SHA-256 hex of the weights; shv_cuda.h:100 */
double shv_hip_threshold(const shv_hip_model* m);         /* from "<weights>.json"; shv_cuda.h:101 */
const char* shv_hip_compute_revision(void);               /* "hip-<16 hex>" of the numeric sources; :102 */
int shv_hip_limits(const shv_hip_model* m, int* max_frames, int* max_windows, int* max_host_tokens,
                   int* token_slots);                                                    /* shv_cuda.h:103 */
size_t shv_hip_weight_bytes(const shv_hip_model* m);      /* device bytes of weights; shv_cuda.h:104 */
size_t shv_hip_device_bytes(const shv_hip_model* m);      /* device bytes allocated in total; :105 */

/* synchronous (split into GPU batches internally); shv_cuda.h:107-114.
 * rgb: n x 180x320x3 uint8; tokens: n x 16 x 384 fp32 (before positions).  tokens (classify): b x 20 x 16 x 384
 * fp32; clips (predict): b x 20 x 180x320x3 uint8; logits: b fp32.  On failure outputs are NaN and -1 returned. */
int shv_hip_encode_frames(shv_hip_model* m, const uint8_t* rgb, size_t n, float* tokens);   /* :112 */
int shv_hip_classify(shv_hip_model* m, const float* tokens, size_t b, float* logits);       /* :113 */
int shv_hip_predict(shv_hip_model* m, const uint8_t* clips, size_t b, float* logits);       /* :114 */

/* asynchronous; shv_cuda.h:116-147 */
typedef void (*shv_hip_callback)(shv_hip_job* job, int status /* 1 done, -1 failed */, void* user);

typedef struct shv_hip_request {      /* shv_cuda.h:118-135, same layout */
    const uint8_t* frames;            /* n_frames x 180x320x3 uint8 */
    size_t n_frames;
    float* tokens_out;                /* optional: n_frames x 6144 fp32 (host) */
    const int32_t* store_slots;       /* optional: n_frames device token slots (-1 = do not store) */
    size_t n_windows;                 /* entry e = window*20 + frame position: */
    const int32_t* window_frames;     /*   >= 0 -> frame of this request (NULL = all -1) */
    const int32_t* window_slots;      /*   else >= 0 -> device token slot */
    const float* const* window_tokens;/*   else host pointer to 6144 fp32 */
    float* logits_out;                /* n_windows fp32 (NaN for every window of a failed job) */
    shv_hip_callback callback;        /* optional */
    void* user;
} shv_hip_request;

shv_hip_job* shv_hip_submit(shv_hip_model* m, const shv_hip_request* req);               /* shv_cuda.h:139 */
int shv_hip_job_status(const shv_hip_job* job);   /* 0 pending, 1 done, -1 failed; shv_cuda.h:140 */
int shv_hip_job_wait(shv_hip_job* job);           /* blocks; 0 done, -1 failed; shv_cuda.h:141 */
const char* shv_hip_job_error(const shv_hip_job* job);                                   /* shv_cuda.h:142 */
int shv_hip_job_timing(const shv_hip_job* job, double* queue_ms, double* run_ms, double* gpu_ms,
                       int* batch_frames, int* batch_windows);                           /* shv_cuda.h:145 */
void shv_hip_job_free(shv_hip_job* job);                                                 /* shv_cuda.h:147 */

/* pinned host memory (hipHostMalloc); frames in it are DMA'd without staging; shv_cuda.h:149-151 */
void* shv_hip_host_alloc(size_t bytes);
void shv_hip_host_free(void* p);

/* ---------------------------------------------------------------------------------------------------------------
 * Engine-level entry points.  No counterpart in shv_cuda.h: the reference reaches its Engine class directly from
 * C++ tools (bench/gpu_kbench.cu:59-98, bench/gpu_dump.cu).  They serve benchmarks and parity tools that run the
 * forward on buffers already resident in HBM, without the scheduler or any host copy.
 * Device pointers only; `stream` is a hipStream_t (NULL = the model's compute stream).  Not thread-safe against
 * the model's own worker: call them only while no job is queued or running on `m`.  The calls are asynchronous and
 * share the model's activation buffers (and, in fp32, its small-GEMM workspace): calls on one model must run one
 * after another on the device -- issue them on one stream, or synchronise between streams.
 */
/* d_frames: n_clips*20 crops in device memory; d_logits: n_clips fp32 in device memory.  n_clips <= limits. */
int shv_hip_forward_device(shv_hip_model* m, const uint8_t* d_frames, int n_clips, float* d_logits, void* stream);
/* encode only: d_frames (n_frames crops) -> d_tokens (n_frames x 6144 fp32), device memory. */
int shv_hip_encode_device(shv_hip_model* m, const uint8_t* d_frames, int n_frames, float* d_tokens, void* stream);
/* classify only (the sequence stages alone): d_tokens n_windows x [20][16][384] fp32 (a window's 20
 * frames' tokens back to back, the layout of shv_hip_classify's host tokens) -> d_logits [n_windows], device memory;
 * n_windows <= limits.  One pass on `stream`. */
int shv_hip_classify_device(shv_hip_model* m, const float* d_tokens, int n_windows, float* d_logits, void* stream);
/* Per-kernel-family timing with HIP events on the launching stream (graphs are off while enabled):
 * enable(1)/disable(0); read the accumulated milliseconds, launch count, algorithmic bytes and FLOPs of family
 * `name` (-1 if unknown); list writes the family names seen since enabling, one per line, into buf (at most cap
 * bytes with the terminating NUL) and returns the full length.  A family is one kernel at the shapes the forward
 * gives it: "ir_<cin>x<cexp>x<cout>" fused blocks, "gdn_prep", ..., GEMMs as "<role>:<kernel template>". */
int shv_hip_profile_enable(shv_hip_model* m, int on);
int shv_hip_profile_read(shv_hip_model* m, const char* name, double* total_ms, long long* launches,
                         double* bytes, double* flops);
long long shv_hip_profile_list(shv_hip_model* m, char* buf, size_t cap);
/* Debug: write float32 intermediates of frame 0 / window 0 of the next synchronous call into dir (graphs off). */
int shv_hip_set_dump_dir(shv_hip_model* m, const char* dir);

/* Pointwise-conv GEMM microbench.  No counterpart in shv_cuda.h: the reference benches its GEMM from a C++ tool
 * (bench/gpu_gemm_bench.cu:27-116: engine GEMM on the model's 1x1 shapes, and a bitwise check that every kernel
 * variant gives the same outputs).  C[m][n] = act(A[m][k] . W[n][k]^T + bias[n]) in the arithmetic of `mode`
 * ("fp32": fp32 matrix cores, or the CPU engine's VALU order; "fp16" / "bf16": split-operand MFMA), fp32 A, W, bias and C in
 * device memory, row-major with leading dimensions k (A, W) and n (C).  act: the reference's codes
 * (engine/cuda/common.cuh:69): 0 none, 1 ReLU, 2 hardswish, 3 SiLU, 4 hardsigmoid.  d_bias may be NULL.
 * create repacks W on the device (synchronising `stream`); NULL + last_error on failure (fp16 / bf16 need k % 8 == 0).
 * run: variant 0 = the engine's own kernel choice; fp32: 1 GEMV, 2 tiled, 3 K blocks in parallel (1-3: the CPU
 * engine's operation order; 3 allocates its workspace of ceil(k / 64) * m * n floats and synchronises `stream`),
 * 4 the fp32 matrix cores (k % 4 == 0), 5 narrow (CPU order; the (k, n) shapes of blocks 1-6 only: 16x16, 16x64,
 * 64x24, 24x72, 72x24, 72x40, 40x120, 120x40), 6 column chunks (CPU order, k <= 1024, k % 4 == 0); fp16 / bf16:
 * 1 small-M, 2..6 direct with
 * 1..5 column tiles per wave, 7 LDS-staged, 8 streaming (n <= 160).  Returns 0, or -1 + last_error.  Asynchronous on
 * `stream` except fp32 variant 3. */
typedef struct shv_hip_gemm shv_hip_gemm;
shv_hip_gemm* shv_hip_gemm_create(const char* mode, int n, int k, const float* d_w, void* stream);
int shv_hip_gemm_run(shv_hip_gemm* g, const float* d_a, long long m, const float* d_bias, int act, float* d_c,
                     int variant, void* stream);
void shv_hip_gemm_free(shv_hip_gemm* g);

/* Face crops on the GPU: the reference's lazy native crop (engine/include/shv_prep.h:181-186, shv_native_crop_rgb;
 * engine/preprocess/canvas.cpp:66-91) for n frames at once, frames and crops in DEVICE memory.  Crop i =
 * cv2.resize(canvas_i[4y:4(y+h), 4x:4(x+w)], (320,180), INTER_AREA) with canvas_i the frame letterboxed into
 * 1280x720 (INTER_AREA when shrinking, INTER_LINEAR when enlarging, bars zero), byte-exact to the reference;
 * written to d_out + i * SHV_HIP_FRAME_BYTES, i.e. the crop layout shv_hip_forward_device reads.  Rects must lie in
 * the 320x180 letterbox with w >= 80, h >= 45 (the reference's crop_geometry gives h in [80,180], w = round(16h/9)).
 * Synchronous on `stream`; one call at a time per process.  Returns 0, or -1 + last_error. */
typedef struct {
    const uint8_t* data;   /* device pointer */
    int width, height;
    ptrdiff_t stride;      /* bytes per row */
} shv_hip_rgb_image;       /* shv_rgb_image, shv_prep.h:74-78 */
typedef struct { int x, y, w, h; } shv_hip_rect;   /* shv_rect, shv_prep.h:86 */
int shv_hip_native_crops_rgb(const shv_hip_rgb_image* frames, const shv_hip_rect* rects, int n, uint8_t* d_out,
                             void* stream);
/* The same for I420 frames (shv_native_crop_i420, shv_prep.h:186): equal to converting the frame to RGB24 as the
 * reference does (ffmpeg's unscaled yuv420p -> rgb24, BT.601 limited range; engine/preprocess/color.cpp:4-11) and
 * cropping; planes in device memory, chroma (width + 1) / 2 x (height + 1) / 2. */
typedef struct {
    const uint8_t *y, *u, *v;   /* device pointers */
    ptrdiff_t y_stride, u_stride, v_stride;
    int width, height;          /* luma size */
} shv_hip_i420_image;           /* shv_i420_image, shv_prep.h:80-84 */
int shv_hip_native_crops_i420(const shv_hip_i420_image* frames, const shv_hip_rect* rects, int n, uint8_t* d_out,
                              void* stream);

/* Gated delta rule of one tier on device buffers (the scan of config 3 on its own; no counterpart in shv_cuda.h --
 * the reference runs its delta_kernel only inside classify, engine/cuda/seq.cu:106-195).  Per window 321 rows; rows
 * = n_windows * 321: q, k [rows][384] (6 heads x 64, l2-normalised; q scaled), v, o [rows][768] (6 heads x 128),
 * decay, beta [rows][8] (head h in column h).  Per (window, head): S_0 = 0, S_t = a_t S_{t-1} + k_t u_t^T,
 * u_t = b_t (v_t - a_t S_{t-1}^T k_t), o_t = S_t^T q_t.  variant 0: the tier's own kernel (fp32: token by token
 * with each value column's keys split over lane groups, or in the reference's order when SHV_HIP_F32_CPU_ORDER=1;
 * fp16 / bf16: the chunked scan), 1: token by token (fp32: the reference's order; fp16 / bf16: key split),
 * 2: chunked (fp16 / bf16), 3: key split (every tier).  Synchronous for the chunked scan (it allocates a work buffer
 * per call).  Returns 0, or -1 + last_error. */
int shv_hip_delta_rule(const char* mode, const float* d_q, const float* d_k, const float* d_v, const float* d_decay,
                       const float* d_beta, int n_windows, float* d_o, int variant, void* stream);

/* The gated delta rule above without any allocation, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments and results as shv_hip_delta_rule (bitwise), but asynchronous on `stream` in every variant: the
 * chunked scan (variant 0 or 2, every tier) works in a static device array for at most 16 windows (30.5 MB per
 * GPU, held until the process ends) and rejects more windows (-1 + last_error); the token-by-token variants need no
 * work memory.  Every call on one GPU shares that array: calls that overlap on one GPU (other streams or
 * threads) race -- serialise them.  Returns 0, or -1 + last_error. */
int shv_hip_delta_rule_noalloc(const char* mode, const float* d_q, const float* d_k, const float* d_v,
                               const float* d_decay, const float* d_beta, int n_windows, float* d_o, int variant,
                               void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * SHIELD-A on the GPU: the whole audio model from PCM (shv_hip_audio_predict*: the frontend, engine/audio/
 * frontend.cpp -- log-mel frames, CNN, frequency attention, 125 tokens of 384 per 10 s window -- then the sequence
 * stages) in place of the reference's shield_predict / shield_predict_batch (engine/audio/include/shield.h:39-41,
 * engine/audio/api.cpp:194-216), and the sequence stages alone from tokens (shv_hip_audio_sequence*: the per-window
 * call of shield::sequence, engine/audio/core.hpp:26, sequence.cpp:349: tokens + readout -> GDN-A -> GDN-B x2 ->
 * SISA last row -> head -> logit, which the reference exports through no C entry point of its own), batched over
 * windows, with the SHIELD-V sequence kernels.
 * Modes: "fp32" (fp32 operands and arithmetic throughout; the GEMMs on the fp32 matrix cores; elementwise functions
 * are the device's, within a few ulp of glibc's) and "fp16" / "bf16" (split-operand matrix cores, fp32-level operand
 * precision); the production library loads "fp32" only, the experimental library every mode.  A handle serialises
 * its calls.  Functions return 0 (or a non-NULL handle) on success, -1 / NULL + shv_hip_last_error() on failure. */
typedef struct shv_hip_audio shv_hip_audio;

/* A SHLDA001 file (container: engine/audio/weights.cpp:16-48; sequence tensors and shapes: engine/audio/
 * sequence.cpp:290-317; frontend tensors, when present: frontend.cpp:146-160) on `device`, buffers for max_windows
 * (1..4096) windows per launch.  Files without the frontend's tensors load for the token entry points only. */
shv_hip_audio* shv_hip_audio_load(const char* weights, const char* mode, int device, int max_windows);
void shv_hip_audio_free(shv_hip_audio* a);
const char* shv_hip_audio_mode(const shv_hip_audio* a);
const char* shv_hip_audio_fingerprint(const shv_hip_audio* a);   /* SHA-256 hex of the weight file */
size_t shv_hip_audio_device_bytes(const shv_hip_audio* a);
/* n windows of host tokens (window w at tokens + w * stride floats, stride >= 48000) -> logits[n] (host);
 * synchronous, any n (batches of max_windows) */
int shv_hip_audio_sequence(shv_hip_audio* a, const float* tokens, size_t n, size_t stride, float* logits);
/* the same on device buffers, asynchronous on `stream` (NULL = the handle's own stream), n <= max_windows.  The
 * calls of one handle share its activation buffers: each call's device work starts after the previous call's has
 * ended, whatever streams they were issued on (an event of the handle orders them). */
int shv_hip_audio_sequence_device(shv_hip_audio* a, const float* d_tokens, int n, size_t stride, float* d_logits,
                                  void* stream);
/* 1 when the handle's weights carry the frontend (the PCM entry points work), else 0 */
int shv_hip_audio_has_frontend(const shv_hip_audio* a);
/* n windows of 16 kHz PCM (window w at pcm + w * stride_samples, stride_samples >= 160000; every sample finite and
 * in [-1, 1], else -1 before any work) -> logits[n] (host); synchronous, any n (batches of max_windows).  The logits
 * are NaN after a failure.  Replaces shield_predict_batch (engine/audio/api.cpp:200-216; shield_predict is n = 1). */
int shv_hip_audio_predict(shv_hip_audio* a, const float* pcm, size_t n, size_t stride_samples, float* logits);
/* the same on device buffers, asynchronous on `stream` (NULL = the handle's own stream), n <= max_windows; the PCM is
 * not range-checked.  Ordered with the handle's other calls as shv_hip_audio_sequence_device. */
int shv_hip_audio_predict_device(shv_hip_audio* a, const float* d_pcm, int n, size_t stride_samples,
                                 float* d_logits, void* stream);
/* the frontend alone (shield::frontend_cnn, engine/audio/frontend.cpp:258-280, without its stream cache): host PCM
 * as shv_hip_audio_predict -> tokens [n][125][384] (host) */
int shv_hip_audio_frontend(shv_hip_audio* a, const float* pcm, size_t n, size_t stride_samples, float* tokens);
/* per-kernel-family timing and stage dumps, as shv_hip_profile_* / shv_hip_set_dump_dir (dump names: tokens, gdn_a,
 * gdn_b, sisa_last, logit -- the reference's, sequence.cpp:324-345; from PCM also mel ([80][997]) and cnn
 * ([125][384]), frontend.cpp:272-275) */
int shv_hip_audio_profile_enable(shv_hip_audio* a, int on);
int shv_hip_audio_profile_read(shv_hip_audio* a, const char* name, double* total_ms, long long* launches,
                               double* bytes, double* flops);
long long shv_hip_audio_profile_list(shv_hip_audio* a, char* buf, size_t cap);
int shv_hip_audio_set_dump_dir(shv_hip_audio* a, const char* dir);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif
#ifdef __cplusplus
}
#endif
#endif /* SHV_HIP_H */
