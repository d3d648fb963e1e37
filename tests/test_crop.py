"""Face crops on the GPU (shv_hip_native_crops_rgb) against the reference preprocessing's lazy native crop
(shv_native_crop_rgb, engine/preprocess/canvas.cpp:66-91, compiled from its own sources into oracle/_ref): byte-exact
on every case of tests/crop_cases.py -- canvas copy, integer shrink (2x, 3x), fractional shrink, enlargement
(INTER_LINEAR), portrait frames with side bars, odd sizes; crops of the crop_geometry family and free rects.
tests/golden/crops_golden.json holds the reference crops' SHA-256 (tests/golden/make_crop_golden.py)."""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import crop_cases

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "crops_golden.json").read_text())


def test_reference_crops_match_golden(orc):
    if not orc.PREP_SO.exists():
        pytest.skip("reference preprocessing not built (needs /root/reference)")
    ref = orc.PrepRef()
    frames = {}
    for cid, (w, h), seed, rect in crop_cases.cases():
        if seed not in frames:
            frames[seed] = crop_cases.frame(w, h, seed)
        assert hashlib.sha256(ref.native_crop(frames[seed], rect).tobytes()).hexdigest() == GOLDEN[cid], cid
    planes = {}
    for cid, (w, h), seed, rect in crop_cases.i420_cases():
        if seed not in planes:
            planes[seed] = crop_cases.i420_frame(w, h, seed)
        assert hashlib.sha256(ref.native_crop_i420(*planes[seed], rect).tobytes()).hexdigest() == GOLDEN[cid], cid


def test_crop_entry_rejects_bad_rects(shv):
    """Validation runs before the device is touched (so it also holds without a GPU)."""
    for rect, msg in (((250, 0, 80, 45), "letterbox"), ((0, 0, 79, 45), "80x45"), ((0, 0, 80, 44), "80x45"),
                      ((-1, 0, 80, 45), "letterbox")):
        with pytest.raises(shv.ShvError) as e:
            shv.native_crops_rgb([(1, 1280, 720, 3840)], [rect], 1)
        assert msg in str(e.value), (rect, str(e.value))
    with pytest.raises(shv.ShvError) as e:
        shv.native_crops_rgb([(1, 1280, 720, 100)], [(0, 0, 80, 45)], 1)
    assert "bad frame" in str(e.value)


@pytest.mark.gpu
def test_gpu_crops_match_reference(shv, orc):
    cases = crop_cases.cases()
    print(f"[gpu] {len(cases)} crops from {len(crop_cases.SIZES)} frame sizes in one call", flush=True)
    hip = shv.Hip()
    frames, dev = {}, {}
    try:
        for cid, (w, h), seed, rect in cases:
            if seed not in frames:
                frames[seed] = crop_cases.frame(w, h, seed)
                dev[seed] = hip.upload(frames[seed])
        d_out = hip.malloc(len(cases) * shv.FRAME_BYTES)
        shv.native_crops_rgb([(dev[s], w, h, 3 * w) for _, (w, h), s, _ in cases], [r for *_, r in cases], d_out)
        got = hip.download(d_out, (len(cases), 180, 320, 3), np.uint8)
        hip.free(d_out)
        ref = orc.PrepRef() if orc.PREP_SO.exists() else None
        bad = []
        for i, (cid, (w, h), seed, rect) in enumerate(cases):
            if hashlib.sha256(got[i].tobytes()).hexdigest() != GOLDEN[cid]:
                detail = ""
                if ref is not None:
                    r = ref.native_crop(frames[seed], rect)
                    dif = np.argwhere(r != got[i])
                    detail = f" {len(dif)} bytes differ, first {dif[0].tolist()} ref {r[tuple(dif[0])]} got " \
                             f"{got[i][tuple(dif[0])]}, max |d| {int(np.abs(r.astype(int) - got[i]).max())}"
                bad.append(cid + detail)
        assert not bad, bad[:8]
    finally:
        for p in dev.values():
            hip.free(p)


@pytest.mark.gpu
def test_gpu_i420_crops_match_reference(shv, orc):
    """I420 frames (odd sizes included: chroma planes (w + 1) / 2 wide) converted per pixel on the GPU."""
    cases = crop_cases.i420_cases()
    print(f"[gpu] {len(cases)} I420 crops from {len(crop_cases.I420_SIZES)} frame sizes in one call", flush=True)
    hip = shv.Hip()
    planes, dev = {}, {}
    try:
        for cid, (w, h), seed, rect in cases:
            if seed not in planes:
                planes[seed] = crop_cases.i420_frame(w, h, seed)
                dev[seed] = [hip.upload(a) for a in planes[seed]]
        d_out = hip.malloc(len(cases) * shv.FRAME_BYTES)
        frames = [(*dev[s], w, (w + 1) // 2, (w + 1) // 2, w, h) for _, (w, h), s, _ in cases]
        shv.native_crops_i420(frames, [r for *_, r in cases], d_out)
        got = hip.download(d_out, (len(cases), 180, 320, 3), np.uint8)
        hip.free(d_out)
        ref = orc.PrepRef() if orc.PREP_SO.exists() else None
        bad = []
        for i, (cid, (w, h), seed, rect) in enumerate(cases):
            if hashlib.sha256(got[i].tobytes()).hexdigest() != GOLDEN[cid]:
                detail = ""
                if ref is not None:
                    r = ref.native_crop_i420(*planes[seed], rect)
                    dif = np.argwhere(r != got[i])
                    detail = f" {len(dif)} bytes differ, max |d| {int(np.abs(r.astype(int) - got[i]).max())}"
                bad.append(cid + detail)
        assert not bad, bad[:8]
    finally:
        for ps in dev.values():
            for p in ps:
                hip.free(p)
