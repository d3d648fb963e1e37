"""Seeded face-crop cases shared by the crop tests and tests/golden/make_crop_golden.py: native RGB frames of
several sizes (copy, integer and fractional shrink, enlarge, portrait with side bars, odd sizes) and crop rectangles
of the reference's crop_geometry family (h in [80, 180], w = round(16 h / 9)) plus free ones (w >= 80, h >= 45)."""
import numpy as np

SIZES = [(1280, 720), (1920, 1080), (2560, 1440), (640, 360), (1366, 768), (720, 1280), (1000, 1000),
         (3840, 2160), (853, 480), (320, 180)]


def frame(w, h, seed):
    """Half the frames uniform noise, half smooth gradients with noise (rounding ties are common there)."""
    rng = np.random.default_rng(seed)
    if seed % 2:
        return rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    y, x = np.mgrid[0:h, 0:w]
    base = np.stack([(x * 255 // max(1, w - 1)), (y * 255 // max(1, h - 1)), ((x + y) * 3) % 256], -1)
    return np.clip(base + rng.integers(-3, 4, (h, w, 3)), 0, 255).astype(np.uint8)


def rects(seed, n=6):
    rng = np.random.default_rng(10_000 + seed)
    out = []
    for i in range(n):
        if i < 4:
            ch = [80, 101, 135, 180][i]
            cw = min(320, int(np.rint(ch * 16 / 9)))
            if cw == 320:
                ch = 180
        else:
            cw, ch = int(rng.integers(80, 321)), int(rng.integers(45, 181))
        out.append((int(rng.integers(0, 320 - cw + 1)), int(rng.integers(0, 180 - ch + 1)), cw, ch))
    return out


def cases():
    """[(case id, frame size, frame seed, rect)]"""
    out = []
    for k, (w, h) in enumerate(SIZES):
        for j, r in enumerate(rects(k)):
            out.append((f"{w}x{h}#{j}", (w, h), k, r))
    return out


I420_SIZES = [(1280, 720), (1920, 1080), (853, 480), (1365, 767), (640, 360), (720, 1280)]


def i420_frame(w, h, seed):
    """Y, U, V planes (chroma (w + 1) / 2 x (h + 1) / 2), seeded; even seeds smooth, odd seeds noise."""
    rng = np.random.default_rng(50_000 + seed)
    cw, ch = (w + 1) // 2, (h + 1) // 2
    if seed % 2:
        return (rng.integers(0, 256, (h, w), dtype=np.uint8), rng.integers(0, 256, (ch, cw), dtype=np.uint8),
                rng.integers(0, 256, (ch, cw), dtype=np.uint8))
    yy, xx = np.mgrid[0:h, 0:w]
    cy, cx = np.mgrid[0:ch, 0:cw]
    Y = np.clip(16 + (xx * 219 // max(1, w - 1)) + rng.integers(-2, 3, (h, w)), 0, 255).astype(np.uint8)
    U = np.clip(128 + (cx * 100 // max(1, cw - 1)) - 50 + rng.integers(-2, 3, (ch, cw)), 0, 255).astype(np.uint8)
    V = np.clip(128 + (cy * 100 // max(1, ch - 1)) - 50 + rng.integers(-2, 3, (ch, cw)), 0, 255).astype(np.uint8)
    return Y, U, V


def i420_cases():
    out = []
    for k, (w, h) in enumerate(I420_SIZES):
        for j, r in enumerate(rects(100 + k)):
            out.append((f"i420 {w}x{h}#{j}", (w, h), k, r))
    return out
