"""Write tests/golden/audio_golden.json from the reference SHIELD-A engine's sequence stages (shield::sequence in
its default exact mode, compiled from /root/reference by `make -C oracle ref` together with
oracle/audio_ref_driver.cpp) on seeded synthetic inputs: SHLDA001 sequence weights from seed 5 (the synth library)
and 8 windows of N(0, 1) tokens from numpy's default_rng(17).  Stored: the weight and token SHA-256s, every window's
logit (value and fp32 bit pattern), and for windows 0 and 5 the stage tensors the reference dumps (tokens, gdn_a,
gdn_b: every 97th value of [126][384]; sisa_last: all 384 values) with their L2 norms.
Run here:  python tests/golden/make_audio_golden.py.  The file is data (inputs named by seed, outputs)."""
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "shield-sisa_amd"))

import oracle as orc  # noqa: E402
import shv_hip  # noqa: E402

WEIGHT_SEED, TOKEN_SEED, WINDOWS, STAGE_WINDOWS, STEP = 5, 17, 8, (0, 5), 97


def main():
    out = {"weights_seed": WEIGHT_SEED, "tokens_seed": TOKEN_SEED, "windows": WINDOWS, "sample_step": STEP}
    with tempfile.TemporaryDirectory() as tmp:
        wpath = Path(tmp) / "audio.shlda"
        out["weights_sha256"] = shv_hip.write_audio_weights(wpath, WEIGHT_SEED)
        tokens = shv_hip.audio_tokens(WINDOWS, TOKEN_SEED)
        out["tokens_sha256"] = shv_hip.sha256_bytes(tokens)
        ref = orc.AudioReference(wpath)
        logits, stages = [], {}
        for w in range(WINDOWS):
            d = Path(tmp) / f"dump{w}"
            d.mkdir()
            logit = np.float32(ref.sequence(tokens[w], str(d)))
            logits.append(logit)
            if w in STAGE_WINDOWS:
                st = {}
                for name in ("tokens", "gdn_a", "gdn_b", "sisa_last"):
                    a = np.fromfile(d / f"{name}.f32", np.float32)
                    sample = a if name == "sisa_last" else a[::STEP]
                    st[name] = {"size": int(a.size), "l2": float(np.linalg.norm(a.astype(np.float64))),
                                "sample": [float(x) for x in sample]}
                stages[str(w)] = st
        ref.close()
    out["logits"] = [float(x) for x in logits]
    out["logit_bits"] = [f"{int(np.float32(x).view(np.uint32)):08x}" for x in logits]
    out["stages"] = stages
    (ROOT / "tests" / "golden" / "audio_golden.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"{WINDOWS} windows, logits {out['logits']}")


if __name__ == "__main__":
    main()
