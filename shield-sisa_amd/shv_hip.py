"""ctypes binding of libshield_v_hip.so (include/shv_hip.h) and of the synthetic-input library.

This is the Python-side mirror of the reference engine's C API (engine/include/shv_cuda.h): the same calls,
argument meaning and error behaviour (-1 / NULL plus a thread-local error string, NaN outputs on failure).
The product is the C-ABI library; this module only marshals numpy buffers.  It refuses to run when the HIP
library is missing -- there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_DIR = PKG / "lib"
FRAME_BYTES = 172800
TOKEN_FLOATS = 6144
WINDOW_FRAMES = 20
AUDIO_WINDOW_SAMPLES = 160000   # one SHIELD-A window: 10 s of 16 kHz PCM (engine/audio/include/shield.h:8)


class ShvError(RuntimeError):
    pass


class Options(ctypes.Structure):
    _fields_ = [("max_frames", ctypes.c_int), ("max_windows", ctypes.c_int), ("max_host_tokens", ctypes.c_int),
                ("token_slots", ctypes.c_int), ("use_graphs", ctypes.c_int), ("max_delay_us", ctypes.c_int)]


CALLBACK = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p)


class Request(ctypes.Structure):
    _fields_ = [("frames", ctypes.c_void_p), ("n_frames", ctypes.c_size_t), ("tokens_out", ctypes.c_void_p),
                ("store_slots", ctypes.c_void_p), ("n_windows", ctypes.c_size_t),
                ("window_frames", ctypes.c_void_p), ("window_slots", ctypes.c_void_p),
                ("window_tokens", ctypes.c_void_p), ("logits_out", ctypes.c_void_p), ("callback", CALLBACK),
                ("user", ctypes.c_void_p)]


_P = ctypes.c_void_p
_SIGS = {
    "shv_hip_default_options": (None, [_P]),
    "shv_hip_load": (_P, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]),
    "shv_hip_load_ex": (_P, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, _P]),
    "shv_hip_free": (None, [_P]),
    "shv_hip_last_error": (ctypes.c_char_p, []),
    "shv_hip_mode": (ctypes.c_char_p, [_P]),
    "shv_hip_fingerprint": (ctypes.c_char_p, [_P]),
    "shv_hip_threshold": (ctypes.c_double, [_P]),
    "shv_hip_compute_revision": (ctypes.c_char_p, []),
    "shv_hip_limits": (ctypes.c_int, [_P, _P, _P, _P, _P]),
    "shv_hip_weight_bytes": (ctypes.c_size_t, [_P]),
    "shv_hip_device_bytes": (ctypes.c_size_t, [_P]),
    "shv_hip_encode_frames": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _P]),
    "shv_hip_classify": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _P]),
    "shv_hip_predict": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _P]),
    "shv_hip_submit": (_P, [_P, _P]),
    "shv_hip_job_status": (ctypes.c_int, [_P]),
    "shv_hip_job_wait": (ctypes.c_int, [_P]),
    "shv_hip_job_error": (ctypes.c_char_p, [_P]),
    "shv_hip_job_timing": (ctypes.c_int, [_P, _P, _P, _P, _P, _P]),
    "shv_hip_job_free": (None, [_P]),
    "shv_hip_host_alloc": (_P, [ctypes.c_size_t]),
    "shv_hip_host_free": (None, [_P]),
    "shv_hip_forward_device": (ctypes.c_int, [_P, _P, ctypes.c_int, _P, _P]),
    "shv_hip_encode_device": (ctypes.c_int, [_P, _P, ctypes.c_int, _P, _P]),
    "shv_hip_classify_device": (ctypes.c_int, [_P, _P, ctypes.c_int, _P, _P]),
    "shv_hip_profile_enable": (ctypes.c_int, [_P, ctypes.c_int]),
    "shv_hip_profile_read": (ctypes.c_int, [_P, ctypes.c_char_p, _P, _P, _P, _P]),
    "shv_hip_profile_list": (ctypes.c_longlong, [_P, _P, ctypes.c_size_t]),
    "shv_hip_set_dump_dir": (ctypes.c_int, [_P, ctypes.c_char_p]),
    "shv_hip_gemm_create": (_P, [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, _P, _P]),
    "shv_hip_gemm_run": (ctypes.c_int, [_P, _P, ctypes.c_longlong, _P, ctypes.c_int, _P, ctypes.c_int, _P]),
    "shv_hip_gemm_free": (None, [_P]),
    "shv_hip_delta_rule": (ctypes.c_int, [ctypes.c_char_p, _P, _P, _P, _P, _P, ctypes.c_int, _P, ctypes.c_int, _P]),
    "shv_hip_delta_rule_noalloc": (ctypes.c_int, [ctypes.c_char_p, _P, _P, _P, _P, _P, ctypes.c_int, _P, ctypes.c_int,
                                                  _P]),
    "shv_hip_native_crops_rgb": (ctypes.c_int, [_P, _P, ctypes.c_int, _P, _P]),
    "shv_hip_native_crops_i420": (ctypes.c_int, [_P, _P, ctypes.c_int, _P, _P]),
    "shv_hip_audio_load": (_P, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_int]),
    "shv_hip_audio_free": (None, [_P]),
    "shv_hip_audio_mode": (ctypes.c_char_p, [_P]),
    "shv_hip_audio_fingerprint": (ctypes.c_char_p, [_P]),
    "shv_hip_audio_device_bytes": (ctypes.c_size_t, [_P]),
    "shv_hip_audio_sequence": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_size_t, _P]),
    "shv_hip_audio_sequence_device": (ctypes.c_int, [_P, _P, ctypes.c_int, ctypes.c_size_t, _P, _P]),
    "shv_hip_audio_has_frontend": (ctypes.c_int, [_P]),
    "shv_hip_audio_predict": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_size_t, _P]),
    "shv_hip_audio_predict_device": (ctypes.c_int, [_P, _P, ctypes.c_int, ctypes.c_size_t, _P, _P]),
    "shv_hip_audio_frontend": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_size_t, _P]),
    "shv_hip_audio_profile_enable": (ctypes.c_int, [_P, ctypes.c_int]),
    "shv_hip_audio_profile_read": (ctypes.c_int, [_P, ctypes.c_char_p, _P, _P, _P, _P]),
    "shv_hip_audio_set_dump_dir": (ctypes.c_int, [_P, ctypes.c_char_p]),
    "shv_hip_audio_profile_list": (ctypes.c_longlong, [_P, _P, ctypes.c_size_t]),
}

_libs: dict[str, ctypes.CDLL] = {}


def library(experimental: bool = False) -> ctypes.CDLL:
    name = "libshield_v_hip_experimental.so" if experimental else "libshield_v_hip.so"
    if name not in _libs:
        path = LIB_DIR / name
        if not path.exists():
            raise ShvError(f"{path} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(str(path))
        for fn, (res, args) in _SIGS.items():
            f = getattr(lib, fn)
            f.restype = res
            f.argtypes = args
        _libs[name] = lib
    return _libs[name]


def synth_library() -> ctypes.CDLL:
    if "synth" not in _libs:
        path = LIB_DIR / "libshv_synth.so"
        if not path.exists():
            raise ShvError(f"{path} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(str(path))
        lib.shv_synth_weights.restype = ctypes.c_int
        lib.shv_synth_weights.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_double, ctypes.c_char_p,
                                          ctypes.POINTER(ctypes.c_longlong), ctypes.POINTER(ctypes.c_int)]
        lib.shv_synth_audio_weights.restype = ctypes.c_int
        lib.shv_synth_audio_weights.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_char_p,
                                                ctypes.POINTER(ctypes.c_int)]
        lib.shv_synth_audio_model_weights.restype = ctypes.c_int
        lib.shv_synth_audio_model_weights.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_char_p,
                                                      ctypes.POINTER(ctypes.c_int)]
        lib.shv_synth_bytes.restype = None
        lib.shv_synth_bytes.argtypes = [_P, ctypes.c_size_t, ctypes.c_uint64]
        lib.shv_synth_sha256.restype = None
        lib.shv_synth_sha256.argtypes = [_P, ctypes.c_size_t, ctypes.c_char_p]
        _libs["synth"] = lib
    return _libs["synth"]


def write_audio_weights(path, seed: int = 5) -> str:
    """Seeded synthetic SHLDA001 weights of the SHIELD-A sequence stages; returns the SHA-256 hex."""
    sha = ctypes.create_string_buffer(65)
    if synth_library().shv_synth_audio_weights(str(path).encode(), seed, sha, None) != 0:
        raise ShvError(f"cannot write {path}")
    return sha.value.decode()


def write_audio_model_weights(path, seed: int = 5) -> str:
    """Seeded synthetic SHLDA001 weights of the whole SHIELD-A model (the sequence stages drawn as
    write_audio_weights draws them, then the frontend's tensors); returns the SHA-256 hex."""
    sha = ctypes.create_string_buffer(65)
    if synth_library().shv_synth_audio_model_weights(str(path).encode(), seed, sha, None) != 0:
        raise ShvError(f"cannot write {path}")
    return sha.value.decode()


def audio_pcm(n: int, seed: int = 23) -> np.ndarray:
    """n SHIELD-A windows of 16 kHz PCM (160,000 samples), float32 N(0, 0.1^2) clipped to [-1, 1], seeded."""
    x = np.random.default_rng(seed).normal(0.0, 0.1, (n, AUDIO_WINDOW_SAMPLES))
    return np.clip(x, -1.0, 1.0).astype(np.float32)


def audio_tokens(n: int, seed: int = 17) -> np.ndarray:
    """n windows of SHIELD-A sequence input: 125 tokens x 384, float32 ~ N(0,1) from a seeded generator."""
    return np.random.default_rng(seed).standard_normal((n, 125, 384)).astype(np.float32)


def write_weights(path, seed: int = 1, threshold: float = 0.5) -> str:
    """Seeded synthetic SHLDV001 weights + sidecar; returns the SHA-256 hex."""
    sha = ctypes.create_string_buffer(65)
    rc = synth_library().shv_synth_weights(str(path).encode(), seed, threshold, sha, None, None)
    if rc != 0:
        raise ShvError(f"cannot write {path}")
    return sha.value.decode()


def synth_clips(n_clips: int, seed0: int = 1000) -> np.ndarray:
    """uint8 [n, 20, 180, 320, 3]; clip i from seed seed0 + i, uniform on {0..255}."""
    out = np.empty((n_clips, WINDOW_FRAMES, 180, 320, 3), np.uint8)
    lib = synth_library()
    for i in range(n_clips):
        lib.shv_synth_bytes(out[i].ctypes.data, out[i].nbytes, seed0 + i)
    return out


def sha256_bytes(a: np.ndarray) -> str:
    buf = ctypes.create_string_buffer(65)
    a = np.ascontiguousarray(a)
    synth_library().shv_synth_sha256(a.ctypes.data, a.nbytes, buf)
    return buf.value.decode()


def last_error(experimental: bool = False) -> str:
    return library(experimental).shv_hip_last_error().decode()


def default_options() -> Options:
    o = Options()
    library().shv_hip_default_options(ctypes.byref(o))
    return o


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


class Model:
    """One loaded model (shv_hip_load_ex)."""

    def __init__(self, weights, mode: str | None = "fp32", device: int = 0, experimental: bool = False,
                 **options):
        self.lib = library(experimental)
        self.experimental = experimental
        opt = Options()
        self.lib.shv_hip_default_options(ctypes.byref(opt))
        for k, v in options.items():
            setattr(opt, k, int(v))
        self.options = opt
        self.h = self.lib.shv_hip_load_ex(str(weights).encode(), None if mode is None else mode.encode(), device,
                                          ctypes.byref(opt))
        if not self.h:
            raise ShvError(self.lib.shv_hip_last_error().decode())

    def close(self):
        if self.h:
            self.lib.shv_hip_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _err(self) -> str:
        return self.lib.shv_hip_last_error().decode()

    @property
    def mode(self) -> str:
        return self.lib.shv_hip_mode(self.h).decode()

    @property
    def fingerprint(self) -> str:
        return self.lib.shv_hip_fingerprint(self.h).decode()

    @property
    def threshold(self) -> float:
        return self.lib.shv_hip_threshold(self.h)

    def limits(self):
        v = [ctypes.c_int() for _ in range(4)]
        if self.lib.shv_hip_limits(self.h, *[ctypes.byref(x) for x in v]) != 0:
            raise ShvError(self._err())
        return tuple(x.value for x in v)

    def weight_bytes(self) -> int:
        return self.lib.shv_hip_weight_bytes(self.h)

    def device_bytes(self) -> int:
        return self.lib.shv_hip_device_bytes(self.h)

    def predict(self, clips: np.ndarray) -> np.ndarray:
        clips = np.ascontiguousarray(clips, dtype=np.uint8)
        b = clips.size // (WINDOW_FRAMES * FRAME_BYTES)
        out = np.empty(b, np.float32)
        if self.lib.shv_hip_predict(self.h, _ptr(clips), b, _ptr(out)) != 0:
            raise ShvError(self._err())
        return out

    def encode_frames(self, frames: np.ndarray) -> np.ndarray:
        frames = np.ascontiguousarray(frames, dtype=np.uint8)
        n = frames.size // FRAME_BYTES
        out = np.empty((n, 16, 384), np.float32)
        if self.lib.shv_hip_encode_frames(self.h, _ptr(frames), n, _ptr(out)) != 0:
            raise ShvError(self._err())
        return out

    def classify(self, tokens: np.ndarray) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.float32)
        b = tokens.size // (WINDOW_FRAMES * TOKEN_FLOATS)
        out = np.empty(b, np.float32)
        if self.lib.shv_hip_classify(self.h, _ptr(tokens), b, _ptr(out)) != 0:
            raise ShvError(self._err())
        return out

    def submit(self, frames=None, n_windows=0, window_frames=None, window_slots=None, window_tokens=None,
               tokens_out=None, store_slots=None, logits_out=None, callback=None):
        """Returns (job handle, keep-alive list); the caller must keep buffers alive until the job completes."""
        keep = []
        r = Request()
        if frames is not None:
            frames = np.ascontiguousarray(frames, dtype=np.uint8)
            keep.append(frames)
            r.frames = frames.ctypes.data
            r.n_frames = frames.size // FRAME_BYTES
        for name, arr, dt in (("store_slots", store_slots, np.int32), ("window_frames", window_frames, np.int32),
                              ("window_slots", window_slots, np.int32)):
            if arr is not None:
                a = np.ascontiguousarray(arr, dtype=dt)
                keep.append(a)
                setattr(r, name, a.ctypes.data)
        if window_tokens is not None:
            ptrs = (ctypes.c_void_p * len(window_tokens))(*window_tokens)
            keep.append(ptrs)
            r.window_tokens = ctypes.cast(ptrs, ctypes.c_void_p)
        if tokens_out is not None:
            r.tokens_out = tokens_out.ctypes.data
        r.n_windows = n_windows
        if logits_out is not None:
            r.logits_out = logits_out.ctypes.data
        if callback is not None:
            keep.append(callback)
            r.callback = callback
        keep.append(r)
        job = self.lib.shv_hip_submit(self.h, ctypes.byref(r))
        if not job:
            raise ShvError(self._err())
        return job, keep

    def job_wait(self, job) -> int:
        return self.lib.shv_hip_job_wait(job)

    def job_status(self, job) -> int:
        return self.lib.shv_hip_job_status(job)

    def job_error(self, job) -> str:
        return self.lib.shv_hip_job_error(job).decode()

    def job_timing(self, job):
        q, r, g = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        bf, bw = ctypes.c_int(), ctypes.c_int()
        rc = self.lib.shv_hip_job_timing(job, ctypes.byref(q), ctypes.byref(r), ctypes.byref(g), ctypes.byref(bf),
                                         ctypes.byref(bw))
        return rc, dict(queue_ms=q.value, run_ms=r.value, gpu_ms=g.value, batch_frames=bf.value,
                        batch_windows=bw.value)

    def job_free(self, job) -> None:
        self.lib.shv_hip_job_free(job)

    # engine-level (device buffers)
    def forward_device(self, d_frames: int, n_clips: int, d_logits: int, stream: int | None = None) -> None:
        if self.lib.shv_hip_forward_device(self.h, d_frames, n_clips, d_logits, stream) != 0:
            raise ShvError(self._err())

    def classify_device(self, d_tokens: int, n_windows: int, d_logits: int, stream: int | None = None) -> None:
        if self.lib.shv_hip_classify_device(self.h, d_tokens, n_windows, d_logits, stream) != 0:
            raise ShvError(self._err())

    def encode_device(self, d_frames: int, n_frames: int, d_tokens: int, stream: int | None = None) -> None:
        if self.lib.shv_hip_encode_device(self.h, d_frames, n_frames, d_tokens, stream) != 0:
            raise ShvError(self._err())

    def profile_enable(self, on: bool) -> None:
        if self.lib.shv_hip_profile_enable(self.h, 1 if on else 0) != 0:
            raise ShvError(self._err())

    def profile_read(self, family: str):
        ms, n, b, f = ctypes.c_double(), ctypes.c_longlong(), ctypes.c_double(), ctypes.c_double()
        rc = self.lib.shv_hip_profile_read(self.h, family.encode(), ctypes.byref(ms), ctypes.byref(n),
                                           ctypes.byref(b), ctypes.byref(f))
        if rc != 0:
            return None
        return dict(ms=ms.value, launches=n.value, bytes=b.value, flops=f.value)

    def profile_families(self) -> list:
        n = self.lib.shv_hip_profile_list(self.h, None, 0)
        if n < 0:
            raise ShvError(self._err())
        buf = ctypes.create_string_buffer(int(n) + 1)
        self.lib.shv_hip_profile_list(self.h, buf, len(buf))
        return [x for x in buf.value.decode().split("\n") if x]

    def set_dump_dir(self, d: str) -> None:
        if self.lib.shv_hip_set_dump_dir(self.h, d.encode()) != 0:
            raise ShvError(self._err())


AUDIO_WINDOW_FLOATS = 125 * 384


class AudioModel:
    """SHIELD-A on the GPU (shv_hip_audio_load): PCM windows -> logits through the whole model (weights with the
    frontend's tensors), or windows of 125 x 384 frontend tokens -> logits through the sequence stages."""

    def __init__(self, weights, mode: str = "fp32", device: int = 0, max_windows: int = 256,
                 experimental: bool = False):
        self.lib = library(experimental)
        self.h = self.lib.shv_hip_audio_load(str(weights).encode(), mode.encode(), device, max_windows)
        if not self.h:
            raise ShvError(self.lib.shv_hip_last_error().decode())

    def close(self):
        if self.h:
            self.lib.shv_hip_audio_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _err(self) -> str:
        return self.lib.shv_hip_last_error().decode()

    @property
    def mode(self) -> str:
        return self.lib.shv_hip_audio_mode(self.h).decode()

    @property
    def fingerprint(self) -> str:
        return self.lib.shv_hip_audio_fingerprint(self.h).decode()

    def device_bytes(self) -> int:
        return self.lib.shv_hip_audio_device_bytes(self.h)

    def sequence(self, tokens: np.ndarray, stride: int | None = None) -> np.ndarray:
        """tokens [n][125][384] (or a float32 array whose rows are `stride` floats apart) -> logits [n]"""
        tokens = np.ascontiguousarray(tokens, dtype=np.float32)
        stride = AUDIO_WINDOW_FLOATS if stride is None else stride
        n = tokens.size // stride
        out = np.empty(n, np.float32)
        if self.lib.shv_hip_audio_sequence(self.h, _ptr(tokens), n, stride, _ptr(out)) != 0:
            raise ShvError(self._err())
        return out

    def sequence_device(self, d_tokens: int, n: int, d_logits: int, stride: int = AUDIO_WINDOW_FLOATS,
                        stream: int | None = None) -> None:
        if self.lib.shv_hip_audio_sequence_device(self.h, d_tokens, n, stride, d_logits, stream) != 0:
            raise ShvError(self._err())

    @property
    def has_frontend(self) -> bool:
        return self.lib.shv_hip_audio_has_frontend(self.h) == 1

    def predict(self, pcm: np.ndarray, stride: int | None = None) -> np.ndarray:
        """PCM windows [n][160000] (or rows `stride` samples apart) -> logits [n] through the whole model"""
        pcm = np.ascontiguousarray(pcm, dtype=np.float32)
        stride = AUDIO_WINDOW_SAMPLES if stride is None else stride
        n = pcm.size // stride
        out = np.empty(n, np.float32)
        if self.lib.shv_hip_audio_predict(self.h, _ptr(pcm), n, stride, _ptr(out)) != 0:
            raise ShvError(self._err())
        return out

    def predict_device(self, d_pcm: int, n: int, d_logits: int, stride: int = AUDIO_WINDOW_SAMPLES,
                       stream: int | None = None) -> None:
        if self.lib.shv_hip_audio_predict_device(self.h, d_pcm, n, stride, d_logits, stream) != 0:
            raise ShvError(self._err())

    def frontend(self, pcm: np.ndarray, stride: int | None = None) -> np.ndarray:
        """PCM windows -> frontend tokens [n][125][384]"""
        pcm = np.ascontiguousarray(pcm, dtype=np.float32)
        stride = AUDIO_WINDOW_SAMPLES if stride is None else stride
        n = pcm.size // stride
        out = np.empty((n, 125, 384), np.float32)
        if self.lib.shv_hip_audio_frontend(self.h, _ptr(pcm), n, stride, _ptr(out)) != 0:
            raise ShvError(self._err())
        return out

    def profile_enable(self, on: bool) -> None:
        if self.lib.shv_hip_audio_profile_enable(self.h, 1 if on else 0) != 0:
            raise ShvError(self._err())

    def profile_read(self, family: str):
        ms, n, b, f = ctypes.c_double(), ctypes.c_longlong(), ctypes.c_double(), ctypes.c_double()
        rc = self.lib.shv_hip_audio_profile_read(self.h, family.encode(), ctypes.byref(ms), ctypes.byref(n),
                                                 ctypes.byref(b), ctypes.byref(f))
        if rc != 0:
            return None
        return dict(ms=ms.value, launches=n.value, bytes=b.value, flops=f.value)

    def profile_families(self) -> list:
        n = self.lib.shv_hip_audio_profile_list(self.h, None, 0)
        if n < 0:
            raise ShvError(self._err())
        buf = ctypes.create_string_buffer(int(n) + 1)
        self.lib.shv_hip_audio_profile_list(self.h, buf, len(buf))
        return [x for x in buf.value.decode().split("\n") if x]

    def set_dump_dir(self, d: str) -> None:
        if self.lib.shv_hip_audio_set_dump_dir(self.h, d.encode()) != 0:
            raise ShvError(self._err())


class Hip:
    """Minimal ctypes view of the HIP runtime that libshield_v_hip.so itself links (one runtime per process):
    device buffers, streams and events for callers of the device-pointer entry points."""

    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        library()
        rt = ctypes.CDLL("libamdhip64.so.7")
        for name, args in (("hipMalloc", [_P, ctypes.c_size_t]), ("hipFree", [_P]),
                           ("hipMemcpy", [_P, _P, ctypes.c_size_t, ctypes.c_int]),
                           ("hipDeviceSynchronize", []), ("hipStreamCreate", [_P]), ("hipStreamDestroy", [_P]),
                           ("hipStreamSynchronize", [_P]), ("hipEventCreate", [_P]), ("hipEventDestroy", [_P]),
                           ("hipEventRecord", [_P, _P]), ("hipEventSynchronize", [_P]),
                           ("hipEventElapsedTime", [_P, _P, _P]), ("hipSetDevice", [ctypes.c_int]),
                           ("hipMemset", [_P, ctypes.c_int, ctypes.c_size_t]),
                           ("hipMemcpyAsync", [_P, _P, ctypes.c_size_t, ctypes.c_int, _P])):
            f = getattr(rt, name)
            f.restype = ctypes.c_int
            f.argtypes = args
        self.rt = rt

    def check(self, rc: int, what: str) -> None:
        if rc != 0:
            raise ShvError(f"{what} failed with HIP error {rc}")

    def malloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        self.check(self.rt.hipMalloc(ctypes.byref(p), nbytes), "hipMalloc")
        return p.value

    def free(self, p: int) -> None:
        self.check(self.rt.hipFree(p), "hipFree")

    def upload(self, arr: np.ndarray) -> int:
        arr = np.ascontiguousarray(arr)
        p = self.malloc(arr.nbytes)
        self.check(self.rt.hipMemcpy(p, arr.ctypes.data, arr.nbytes, self.H2D), "hipMemcpy H2D")
        return p

    def download(self, p: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        self.check(self.rt.hipMemcpy(out.ctypes.data, p, out.nbytes, self.D2H), "hipMemcpy D2H")
        return out

    def memset(self, p: int, value: int, nbytes: int) -> None:
        self.check(self.rt.hipMemset(p, value, nbytes), "hipMemset")

    def copy_d2d(self, dst: int, src: int, nbytes: int, stream: int | None = None) -> None:
        self.check(self.rt.hipMemcpyAsync(dst, src, nbytes, self.D2D, stream), "hipMemcpyAsync D2D")

    def sync(self) -> None:
        self.check(self.rt.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream(self) -> int:
        s = ctypes.c_void_p()
        self.check(self.rt.hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        return s.value

    def stream_sync(self, s: int) -> None:
        self.check(self.rt.hipStreamSynchronize(s), "hipStreamSynchronize")

    def stream_destroy(self, s: int) -> None:
        self.check(self.rt.hipStreamDestroy(s), "hipStreamDestroy")

    def event(self) -> int:
        e = ctypes.c_void_p()
        self.check(self.rt.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, e: int, s: int) -> None:
        self.check(self.rt.hipEventRecord(e, s), "hipEventRecord")

    def elapsed_ms(self, e0: int, e1: int) -> float:
        self.check(self.rt.hipEventSynchronize(e1), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.check(self.rt.hipEventElapsedTime(ctypes.byref(ms), e0, e1), "hipEventElapsedTime")
        return ms.value

    def event_destroy(self, e: int) -> None:
        self.check(self.rt.hipEventDestroy(e), "hipEventDestroy")


ACT_NONE, ACT_RELU, ACT_HSWISH, ACT_SILU, ACT_HSIGMOID = 0, 1, 2, 3, 4   # the reference's codes (common.cuh:69)
GEMM_VARIANTS = {"fp32": [1, 2, 3, 4, 5, 6], "fp16": list(range(1, 10)), "bf16": list(range(1, 10))}
GEMM_NARROW_VARIANTS = {8}   # N <= 160 only


class PwGemm:
    """Pointwise-conv GEMM of one tier on device buffers (shv_hip_gemm_*): W [n][k] fp32 repacked at creation."""

    def __init__(self, mode: str, d_w: int, n: int, k: int, stream: int | None = None):
        self.lib = library()
        self.g = self.lib.shv_hip_gemm_create(mode.encode(), n, k, d_w, stream)
        if not self.g:
            raise ShvError(last_error())
        self.mode, self.n, self.k = mode, n, k

    def run(self, d_a: int, m: int, d_c: int, d_bias: int | None = None, act: int = ACT_NONE, variant: int = 0,
            stream: int | None = None) -> None:
        if self.lib.shv_hip_gemm_run(self.g, d_a, m, d_bias, act, d_c, variant, stream) != 0:
            raise ShvError(last_error())

    def close(self) -> None:
        if self.g:
            self.lib.shv_hip_gemm_free(self.g)
            self.g = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class RgbImage(ctypes.Structure):   # shv_hip_rgb_image (a device frame)
    _fields_ = [("data", ctypes.c_void_p), ("width", ctypes.c_int), ("height", ctypes.c_int),
                ("stride", ctypes.c_ssize_t)]


class Rect(ctypes.Structure):       # shv_hip_rect
    _fields_ = [("x", ctypes.c_int), ("y", ctypes.c_int), ("w", ctypes.c_int), ("h", ctypes.c_int)]


def native_crops_rgb(frames, rects, d_out: int, stream: int | None = None) -> None:
    """frames: [(device pointer, width, height, stride)], rects: [(x, y, w, h)] -> len(rects) crops at d_out."""
    n = len(rects)
    fa = (RgbImage * max(1, n))(*[RgbImage(*f) for f in frames])
    ra = (Rect * max(1, n))(*[Rect(*[int(v) for v in r]) for r in rects])
    lib = library()
    if lib.shv_hip_native_crops_rgb(ctypes.cast(fa, ctypes.c_void_p), ctypes.cast(ra, ctypes.c_void_p), n, d_out,
                                    stream) != 0:
        raise ShvError(last_error())


class I420Image(ctypes.Structure):   # shv_hip_i420_image (device planes)
    _fields_ = [("y", ctypes.c_void_p), ("u", ctypes.c_void_p), ("v", ctypes.c_void_p), ("y_stride", ctypes.c_ssize_t),
                ("u_stride", ctypes.c_ssize_t), ("v_stride", ctypes.c_ssize_t), ("width", ctypes.c_int),
                ("height", ctypes.c_int)]


def native_crops_i420(frames, rects, d_out: int, stream: int | None = None) -> None:
    """frames: [(y, u, v, y_stride, u_stride, v_stride, width, height)] device planes -> len(rects) crops at d_out."""
    n = len(rects)
    fa = (I420Image * max(1, n))(*[I420Image(*f) for f in frames])
    ra = (Rect * max(1, n))(*[Rect(*[int(v) for v in r]) for r in rects])
    lib = library()
    if lib.shv_hip_native_crops_i420(ctypes.cast(fa, ctypes.c_void_p), ctypes.cast(ra, ctypes.c_void_p), n, d_out,
                                     stream) != 0:
        raise ShvError(last_error())


def delta_rule(mode: str, d_q: int, d_k: int, d_v: int, d_decay: int, d_beta: int, n_windows: int, d_o: int,
               variant: int = 0, stream: int | None = None) -> None:
    """shv_hip_delta_rule on device buffers (see include/shv_hip.h for the layout)."""
    lib = library()
    if lib.shv_hip_delta_rule(mode.encode(), d_q, d_k, d_v, d_decay, d_beta, n_windows, d_o, variant, stream) != 0:
        raise ShvError(last_error())


def delta_rule_noalloc(mode: str, d_q: int, d_k: int, d_v: int, d_decay: int, d_beta: int, n_windows: int, d_o: int,
                       variant: int = 0, stream: int | None = None) -> None:
    """shv_hip_delta_rule_noalloc: the same without allocating (static work area, asynchronous on `stream`)."""
    lib = library()
    if lib.shv_hip_delta_rule_noalloc(mode.encode(), d_q, d_k, d_v, d_decay, d_beta, n_windows, d_o, variant,
                                      stream) != 0:
        raise ShvError(last_error())


def sigmoid64(logit: float) -> float:
    """Score in double precision (the decision contract: score >= threshold)."""
    import math
    x = float(logit)
    if x >= 0:
        return 1.0 / (1.0 + math.exp(-x))
    e = math.exp(x)
    return e / (1.0 + e)
