"""TEST INFRASTRUCTURE ONLY.  ctypes access to the oracle (this repo's C restatement, oracle/_build), to the
reference CPU engine compiled from /root/reference (oracle/_ref) and to the reference preprocessing's crop path
compiled from the same tree (oracle/_ref/libshield_v_prep_crop.so).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may use this module, and only as the checker / the timed CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_build" / "libshv_oracle.so"
REF_SO = HERE / "_ref" / "libshield_v_cpu.so"
PREP_SO = HERE / "_ref" / "libshield_v_prep_crop.so"
AUDIO_SO = HERE / "_ref" / "libshield_a_ref.so"
FRAME_BYTES = 172800

DUMP_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), ctypes.c_size_t)

EPI = dict(store=0, relu=1, hs=2, res=3, acc=4, acc_div2=5, swiglu=6, hsig=7, silu=8)


def build(ref: bool = False) -> None:
    """Compile the oracle (and, when /root/reference exists, the reference CPU engine)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if ref and Path("/root/reference/engine/model/runtime.cpp").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "-j4", "ref"], check=True)


class Oracle:
    def __init__(self, weights):
        if not ORACLE_SO.exists():
            build()
        lib = ctypes.CDLL(str(ORACLE_SO))
        lib.orc_load.restype = ctypes.c_void_p
        lib.orc_load.argtypes = [ctypes.c_char_p]
        lib.orc_free.argtypes = [ctypes.c_void_p]
        lib.orc_last_error.restype = ctypes.c_char_p
        lib.orc_encode_frame.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, DUMP_FN, ctypes.c_void_p]
        lib.orc_classify.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, DUMP_FN, ctypes.c_void_p]
        lib.orc_gemm.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_void_p, ctypes.c_int]
        lib.orc_exp.restype = ctypes.c_float
        lib.orc_exp.argtypes = [ctypes.c_float]
        lib.orc_silu.restype = ctypes.c_float
        lib.orc_silu.argtypes = [ctypes.c_float]
        lib.orc_hswish.restype = ctypes.c_float
        lib.orc_hswish.argtypes = [ctypes.c_float]
        lib.orc_delta_rule.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_int]
        self.lib = lib
        self.h = None
        if weights is not None:
            self.h = lib.orc_load(str(weights).encode())
            if not self.h:
                raise RuntimeError("oracle load failed: " + lib.orc_last_error().decode())

    def close(self):
        if self.h:
            self.lib.orc_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode_frame(self, rgb: np.ndarray, dumps: dict | None = None) -> np.ndarray:
        rgb = np.ascontiguousarray(rgb, dtype=np.uint8)
        out = np.empty((16, 384), np.float32)
        cb = DUMP_FN(0)
        if dumps is not None:
            def f(ctx, name, data, n):
                dumps[name.decode()] = np.ctypeslib.as_array(data, (n,)).copy()
            cb = DUMP_FN(f)
        self.lib.orc_encode_frame(self.h, rgb.ctypes.data, out.ctypes.data, cb, None)
        return out

    def classify(self, tokens20: np.ndarray, dumps: dict | None = None) -> float:
        """tokens20: [20, 16, 384] float32"""
        t = np.ascontiguousarray(tokens20, dtype=np.float32).reshape(20, 6144)
        ptrs = (ctypes.c_void_p * 20)(*[t[i].ctypes.data for i in range(20)])
        out = np.zeros(1, np.float32)
        cb = DUMP_FN(0)
        if dumps is not None:
            def f(ctx, name, data, n):
                dumps[name.decode()] = np.ctypeslib.as_array(data, (n,)).copy()
            cb = DUMP_FN(f)
        self.lib.orc_classify(self.h, ptrs, out.ctypes.data, cb, None)
        return out

    def predict(self, clip: np.ndarray, dumps: dict | None = None):
        """clip uint8 [20,180,320,3] -> (logit float32 [1], tokens [20,16,384])"""
        clip = np.ascontiguousarray(clip, dtype=np.uint8).reshape(20, FRAME_BYTES)
        toks = np.stack([self.encode_frame(clip[f], dumps if f == 0 else None) for f in range(20)])
        return self.classify(toks, dumps), toks

    def gemm(self, A, W, bias=None, epi="store", R=None, C=None):
        A = np.ascontiguousarray(A, np.float32)
        W = np.ascontiguousarray(W, np.float32)
        M, K = A.shape
        N = W.shape[0]
        ncol = N // 2 if epi == "swiglu" else N
        if C is None:
            C = np.zeros((M, ncol), np.float32)
        C = np.ascontiguousarray(C, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        Rr = None if R is None else np.ascontiguousarray(R, np.float32)
        self.lib.orc_gemm(A.ctypes.data, K, M, W.ctypes.data, None if b is None else b.ctypes.data, N, K,
                          C.ctypes.data, ncol, EPI[epi], None if Rr is None else Rr.ctypes.data,
                          0 if Rr is None else Rr.shape[1])
        return C

    def delta_rule(self, q, k, v, decay, beta):
        q, k, v = (np.ascontiguousarray(x, np.float32) for x in (q, k, v))
        decay = np.ascontiguousarray(decay, np.float32)
        beta = np.ascontiguousarray(beta, np.float32)
        T = q.shape[0]
        o = np.zeros((T, 128), np.float32)
        self.lib.orc_delta_rule(q.ctypes.data, k.ctypes.data, v.ctypes.data, decay.ctypes.data, beta.ctypes.data, T,
                                64, 128, o.ctypes.data, 128)
        return o


class Reference:
    """The reference CPU engine (engine/model, compiled by `make -C oracle ref`)."""

    def __init__(self, weights, threads: int = 1, mode: str = "exact", isa: str | None = None):
        if not REF_SO.exists():
            raise RuntimeError(f"{REF_SO} not built (make -C oracle ref needs /root/reference)")
        lib = ctypes.CDLL(str(REF_SO))
        lib.shv_cpu_load_ex.restype = ctypes.c_void_p
        lib.shv_cpu_load_ex.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p]
        lib.shv_cpu_predict.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.shv_cpu_encode_frames.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.shv_cpu_classify.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.shv_cpu_last_error.restype = ctypes.c_char_p
        lib.shv_cpu_free.argtypes = [ctypes.c_void_p]
        lib.shv_cpu_isa.restype = ctypes.c_char_p
        lib.shv_cpu_isa.argtypes = [ctypes.c_void_p]
        self.lib = lib
        self.h = lib.shv_cpu_load_ex(str(weights).encode(), mode.encode(), threads,
                                     None if isa is None else isa.encode())
        if not self.h:
            raise RuntimeError("reference load failed: " + lib.shv_cpu_last_error().decode())
        self.threads = threads

    @property
    def isa(self) -> str:
        return self.lib.shv_cpu_isa(self.h).decode()

    def predict(self, clips: np.ndarray) -> np.ndarray:
        clips = np.ascontiguousarray(clips, np.uint8)
        b = clips.size // (20 * FRAME_BYTES)
        out = np.empty(b, np.float32)
        if self.lib.shv_cpu_predict(self.h, clips.ctypes.data, b, out.ctypes.data) != 0:
            raise RuntimeError(self.lib.shv_cpu_last_error().decode())
        return out

    def encode_frames(self, frames: np.ndarray) -> np.ndarray:
        frames = np.ascontiguousarray(frames, np.uint8)
        n = frames.size // FRAME_BYTES
        out = np.empty((n, 16, 384), np.float32)
        if self.lib.shv_cpu_encode_frames(self.h, frames.ctypes.data, n, out.ctypes.data) != 0:
            raise RuntimeError(self.lib.shv_cpu_last_error().decode())
        return out

    def classify(self, tokens: np.ndarray) -> np.ndarray:
        """tokens: b windows x [20][16][384] float32 (shv_cpu_classify, engine/include/shv_cpu.h:106-107)."""
        tokens = np.ascontiguousarray(tokens, np.float32)
        b = tokens.size // (20 * 16 * 384)
        out = np.empty(b, np.float32)
        if self.lib.shv_cpu_classify(self.h, tokens.ctypes.data, b, out.ctypes.data) != 0:
            raise RuntimeError(self.lib.shv_cpu_last_error().decode())
        return out

    def close(self):
        if self.h:
            self.lib.shv_cpu_free(self.h)
            self.h = None


class AudioReference:
    """The reference SHIELD-A engine (engine/audio, compiled by `make -C oracle ref` with
    oracle/audio_ref_driver.cpp), exact mode: its sequence stages (tokens [125][384] -> logit, optional stage dumps:
    tokens, gdn_a, gdn_b, sisa_last, logit as .f32 files), its frontend (PCM -> tokens, dumps mel and cnn) and the
    two together (PCM -> logit)."""

    def __init__(self, weights):
        if not AUDIO_SO.exists():
            raise RuntimeError(f"{AUDIO_SO} not built (make -C oracle ref needs /root/reference)")
        lib = ctypes.CDLL(str(AUDIO_SO))
        lib.ora_audio_load.restype = ctypes.c_void_p
        lib.ora_audio_load.argtypes = [ctypes.c_char_p]
        lib.ora_audio_error.restype = ctypes.c_char_p
        lib.ora_audio_sequence.restype = ctypes.c_int
        lib.ora_audio_sequence.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p]
        lib.ora_audio_frontend.restype = ctypes.c_int
        lib.ora_audio_frontend.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p]
        lib.ora_audio_predict.restype = ctypes.c_int
        lib.ora_audio_predict.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.ora_audio_free.argtypes = [ctypes.c_void_p]
        self.lib = lib
        self.h = lib.ora_audio_load(str(weights).encode())
        if not self.h:
            raise RuntimeError("reference audio load failed: " + lib.ora_audio_error().decode())

    def frontend(self, pcm: np.ndarray, dump_dir: str | None = None) -> np.ndarray:
        """160,000 PCM samples -> tokens [125][384] (shield::frontend_cnn); the dump holds mel.f32 [80][997] and
        cnn.f32"""
        x = np.ascontiguousarray(pcm, dtype=np.float32).reshape(160000)
        out = np.zeros((125, 384), np.float32)
        rc = self.lib.ora_audio_frontend(self.h, x.ctypes.data, out.ctypes.data,
                                         None if dump_dir is None else str(dump_dir).encode())
        if rc != 0:
            raise RuntimeError(self.lib.ora_audio_error().decode())
        return out

    def predict(self, pcm: np.ndarray) -> np.ndarray:
        """PCM windows [n][160000] -> logits [n] (frontend, then the sequence stages)"""
        x = np.ascontiguousarray(pcm, dtype=np.float32).reshape(-1, 160000)
        out = np.zeros(len(x), np.float32)
        for i in range(len(x)):
            if self.lib.ora_audio_predict(self.h, x[i].ctypes.data, out[i:].ctypes.data) != 0:
                raise RuntimeError(self.lib.ora_audio_error().decode())
        return out

    def sequence(self, tokens: np.ndarray, dump_dir: str | None = None) -> float:
        t = np.ascontiguousarray(tokens, dtype=np.float32).reshape(125 * 384)
        out = np.zeros(1, np.float32)
        rc = self.lib.ora_audio_sequence(self.h, t.ctypes.data, out.ctypes.data,
                                         None if dump_dir is None else str(dump_dir).encode())
        if rc != 0:
            raise RuntimeError(self.lib.ora_audio_error().decode())
        return out[0]

    def close(self):
        if self.h:
            self.lib.ora_audio_free(self.h)
            self.h = None


class _RgbImage(ctypes.Structure):   # shv_rgb_image (engine/include/shv_prep.h:74-78)
    _fields_ = [("data", ctypes.c_void_p), ("width", ctypes.c_int), ("height", ctypes.c_int),
                ("stride", ctypes.c_ssize_t)]


class _Rect(ctypes.Structure):       # shv_rect (shv_prep.h:86)
    _fields_ = [("x", ctypes.c_int), ("y", ctypes.c_int), ("w", ctypes.c_int), ("h", ctypes.c_int)]


class _I420Image(ctypes.Structure):   # shv_i420_image (shv_prep.h:80-84)
    _fields_ = [("y", ctypes.c_void_p), ("u", ctypes.c_void_p), ("v", ctypes.c_void_p), ("y_stride", ctypes.c_ssize_t),
                ("u_stride", ctypes.c_ssize_t), ("v_stride", ctypes.c_ssize_t), ("width", ctypes.c_int),
                ("height", ctypes.c_int)]


class PrepRef:
    """The reference's lazy native crop, shv_native_crop_rgb (engine/preprocess/canvas.cpp:134-143), compiled from
    its own sources by `make -C oracle ref`: the checker of the GPU crops."""

    def __init__(self):
        if not PREP_SO.exists():
            raise RuntimeError(f"{PREP_SO} not built (make -C oracle ref needs /root/reference)")
        lib = ctypes.CDLL(str(PREP_SO))
        lib.shv_native_crop_rgb.restype = ctypes.c_int
        lib.shv_native_crop_rgb.argtypes = [ctypes.POINTER(_RgbImage), _Rect, ctypes.c_void_p]
        lib.shv_native_crop_i420.restype = ctypes.c_int
        lib.shv_native_crop_i420.argtypes = [ctypes.POINTER(_I420Image), _Rect, ctypes.c_void_p]
        lib.shv_canvas_info_get.restype = ctypes.c_int
        lib.shv_prep_last_error.restype = ctypes.c_char_p
        self.lib = lib

    def native_crop(self, frame: np.ndarray, rect) -> np.ndarray:
        frame = np.ascontiguousarray(frame, np.uint8)
        h, w = frame.shape[:2]
        img = _RgbImage(frame.ctypes.data, w, h, w * 3)
        out = np.empty((180, 320, 3), np.uint8)
        if self.lib.shv_native_crop_rgb(ctypes.byref(img), _Rect(*[int(v) for v in rect]), out.ctypes.data) != 0:
            raise RuntimeError(self.lib.shv_prep_last_error().decode())
        return out

    def native_crop_i420(self, y: np.ndarray, u: np.ndarray, v: np.ndarray, rect) -> np.ndarray:
        y, u, v = (np.ascontiguousarray(a, np.uint8) for a in (y, u, v))
        img = _I420Image(y.ctypes.data, u.ctypes.data, v.ctypes.data, y.shape[1], u.shape[1], v.shape[1],
                         y.shape[1], y.shape[0])
        out = np.empty((180, 320, 3), np.uint8)
        if self.lib.shv_native_crop_i420(ctypes.byref(img), _Rect(*[int(x) for x in rect]), out.ctypes.data) != 0:
            raise RuntimeError(self.lib.shv_prep_last_error().decode())
        return out
