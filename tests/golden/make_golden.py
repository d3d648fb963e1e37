"""Write the golden fixtures of this repository from the reference CPU engine.

Run here (where /root/reference exists):  python tests/golden/make_golden.py
It compiles the reference CPU engine from its own sources (oracle/Makefile, target `ref`), generates the seeded
synthetic weights (seed 1, threshold 0.5) and clips (seeds 1000 + i), and records, from the reference engine in
its exact tier:
  - golden_seed1.json: weight SHA-256, clip SHA-256s, the float32 bit patterns of 64 logits, and per-stage
    digests (count, float64 sum, sum |x|, sum x^2, first 16 bit patterns) of every intermediate the reference
    dumps through SHV_CPU_DUMP_DIR (CNN stages of the clip's last frame, sequence stages of its window);
  - tokens_clip0.npy: the 16 x 384 float32 tokens of frames 0 and 19 of clip 0 ([2, 16, 384]).
The files are data (inputs' hashes, expected outputs); nothing of the reference's source is stored.
"""
from __future__ import annotations

import json
import os
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "shield-sisa_amd"))

import oracle as orc  # noqa: E402
import shv_hip  # noqa: E402

OUT = Path(__file__).resolve().parent
N_CLIPS = 64
# channels of the reference's padded NHWC dumps cnn00..cnn15 (padded to 16); cnn16 is [60][960]
CNN_CH = [16, 16, 24, 24, 40, 40, 40, 80, 80, 80, 80, 112, 112, 160, 160, 160]


def digest(a: np.ndarray) -> dict:
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    d = a.astype(np.float64)
    return {"n": int(a.size), "sum": float(d.sum()), "abs": float(np.abs(d).sum()), "sq": float((d * d).sum()),
            "head": [int(x) for x in a[:16].view(np.uint32)]}


def unpad(name: str, a: np.ndarray) -> np.ndarray:
    if name.startswith("cnn") and name != "cnn16":
        c = CNN_CH[int(name[3:])]
        cp = (c + 15) // 16 * 16
        return a.reshape(-1, cp)[:, :c].reshape(-1)
    return a


def main() -> None:
    orc.build(ref=True)
    with tempfile.TemporaryDirectory() as td:
        w = Path(td) / "w1.weights"
        sha = shv_hip.write_weights(w, seed=1, threshold=0.5)
        clips = shv_hip.synth_clips(N_CLIPS, 1000)
        ref = orc.Reference(w, threads=8)
        logits = ref.predict(clips)
        ref.close()
        dump_dir = Path(td) / "dump"
        dump_dir.mkdir()
        os.environ["SHV_CPU_DUMP_DIR"] = str(dump_dir)
        ref1 = orc.Reference(w, threads=1)
        l0 = ref1.predict(clips[:1])
        toks = ref1.encode_frames(clips[0])
        ref1.close()
        del os.environ["SHV_CPU_DUMP_DIR"]
        # encode_frames after predict rewrote the CNN dumps with the same clip's last frame (19)
        stages = {}
        for f in sorted(dump_dir.glob("*.f32")):
            stages[f.stem] = digest(unpad(f.stem, np.fromfile(f, np.float32)))
        assert l0.view(np.uint32)[0] == logits[:1].view(np.uint32)[0], "batch 1 vs batch 64 differ"
        fix = {
            "generator": "shv_synth_weights seed 1 threshold 0.5; clips shv_synth_bytes seeds 1000+i",
            "weights_sha256": sha,
            "clip_sha256": [shv_hip.sha256_bytes(clips[i]) for i in range(N_CLIPS)],
            "logits_f32_bits": [int(x) for x in logits.view(np.uint32)],
            "logits": [float(x) for x in logits],
            "threshold": 0.5,
            "stages_clip0": stages,
            "stage_frame": 19,
        }
        (OUT / "golden_seed1.json").write_text(json.dumps(fix, indent=1))
        np.save(OUT / "tokens_clip0.npy", toks[[0, 19]])
        print("logits", logits[:8], "std", logits.std(), "stages", len(stages))


if __name__ == "__main__":
    main()
