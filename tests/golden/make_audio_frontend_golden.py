"""Write tests/golden/audio_frontend_golden.json from the reference SHIELD-A engine's frontend and whole model
(shield::frontend_cnn and frontend + shield::sequence in the default exact mode, compiled from /root/reference by
`make -C oracle ref` together with oracle/audio_ref_driver.cpp) on seeded synthetic inputs: whole-model SHLDA001
weights from seed 5 (the synth library) and 3 windows of PCM N(0, 0.1^2) clipped to [-1, 1] from numpy's
default_rng(23).  Stored: the weight and PCM SHA-256s; per window the logit (value and fp32 bit pattern), the L2
norms of the log-mel image and the tokens, every 131st log-mel value ([80][997], the reference's dump layout) and
every 73rd token value ([125][384]).
Run here:  python tests/golden/make_audio_frontend_golden.py.  The file is data (inputs named by seed, outputs)."""
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

WEIGHT_SEED, PCM_SEED, WINDOWS, MEL_STEP, TOK_STEP = 5, 23, 3, 131, 73


def main():
    out = {"weights_seed": WEIGHT_SEED, "pcm_seed": PCM_SEED, "windows": WINDOWS, "mel_step": MEL_STEP,
           "token_step": TOK_STEP}
    with tempfile.TemporaryDirectory() as tmp:
        wpath = Path(tmp) / "audio_model.shlda"
        out["weights_sha256"] = shv_hip.write_audio_model_weights(wpath, WEIGHT_SEED)
        pcm = shv_hip.audio_pcm(WINDOWS, PCM_SEED)
        out["pcm_sha256"] = shv_hip.sha256_bytes(pcm)
        ref = orc.AudioReference(wpath)
        per = []
        for w in range(WINDOWS):
            d = Path(tmp) / f"dump{w}"
            d.mkdir()
            tok = ref.frontend(pcm[w], str(d))
            mel = np.fromfile(d / "mel.f32", np.float32)
            logit = np.float32(ref.predict(pcm[w:w + 1])[0])
            per.append({"logit": float(logit), "logit_bits": f"{int(logit.view(np.uint32)):08x}",
                        "mel_l2": float(np.linalg.norm(mel.astype(np.float64))),
                        "tokens_l2": float(np.linalg.norm(tok.astype(np.float64))),
                        "mel_sample": [float(x) for x in mel[::MEL_STEP]],
                        "token_sample": [float(x) for x in tok.reshape(-1)[::TOK_STEP]]})
        ref.close()
    out["per_window"] = per
    (ROOT / "tests" / "golden" / "audio_frontend_golden.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"{WINDOWS} windows, logits {[p['logit'] for p in per]}")


if __name__ == "__main__":
    main()
