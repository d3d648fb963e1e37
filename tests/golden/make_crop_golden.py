"""Write tests/golden/crops_golden.json from the reference preprocessing's crop path (shv_native_crop_rgb,
compiled from /root/reference by `make -C oracle ref`): the SHA-256 of every crop of tests/crop_cases.py (RGB frames through shv_native_crop_rgb, I420 frames through
shv_native_crop_i420).
Run here:  python tests/golden/make_crop_golden.py.  The file is data (case ids and output hashes)."""
import hashlib
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))

import crop_cases  # noqa: E402
import oracle as orc  # noqa: E402


def main():
    ref = orc.PrepRef()
    frames = {}
    out = {}
    for cid, (w, h), seed, rect in crop_cases.cases():
        if seed not in frames:
            frames[seed] = crop_cases.frame(w, h, seed)
        out[cid] = hashlib.sha256(ref.native_crop(frames[seed], rect).tobytes()).hexdigest()
    planes = {}
    for cid, (w, h), seed, rect in crop_cases.i420_cases():
        if seed not in planes:
            planes[seed] = crop_cases.i420_frame(w, h, seed)
        out[cid] = hashlib.sha256(ref.native_crop_i420(*planes[seed], rect).tobytes()).hexdigest()
    (ROOT / "tests" / "golden" / "crops_golden.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"{len(out)} crops")


if __name__ == "__main__":
    main()
