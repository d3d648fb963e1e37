#!/usr/bin/env python3
"""Quality certificates for the approximate modes (fp16, bf16) of the HIP engine: writes <weights>.hip.cert.

The reference certifies its CUDA engine's approximate modes on the real validation set against the exact fp32 logits
(bench/gpu_certify.sh:1-9; criteria bench/metrics.py:42, 131-150: AUROC / FPR / TPR limits, every sample valid).
Without labelled crops this tool certifies on clips the caller supplies (uint8 [N][20][180][320][3] in a .npy file)
or, by default, on seeded synthetic clips, against the exact fp32 tier of the same library (which reproduces the
reference CPU engine). A mode passes when
  * every logit is finite,
  * max |logit - exact logit| <= --tol, and
  * no decision differs from the exact tier's, decision = sigmoid(logit) >= threshold in double precision (the
    reference's decision contract).
The approximate mode is run through the experimental library (which skips the certificate check, like the
reference's experimental build); each passing mode then gets the line
  "<weights sha256> <mode> <revision> PASS <cert json> <cert json sha256> threshold=<repr(threshold)>"
under the header SHIELDV_HIP_CERT_V2 -- the line shv_hip_load checks (weights hash, mode, compute revision, exact
threshold). Lines for other weights, modes or revisions already in the file are kept.

  python shield-sisa_amd/certify.py --weights model.weights [--modes fp16 bf16] [--clips 64 | --clips-npy crops.npy]
"""
from __future__ import annotations

import argparse
import hashlib
import importlib.util
import json
import math
import sys
from pathlib import Path

import numpy as np

HEADER = "SHIELDV_HIP_CERT_V2"
HERE = Path(__file__).resolve().parent


def _shv():
    if "shv_hip" in sys.modules:
        return sys.modules["shv_hip"]
    spec = importlib.util.spec_from_file_location("shv_hip", HERE / "shv_hip.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["shv_hip"] = mod
    spec.loader.exec_module(mod)
    return mod


def decisions(logits: np.ndarray, threshold: float) -> np.ndarray:
    sig = _shv().sigmoid64
    return np.array([math.isfinite(float(v)) and sig(float(v)) >= threshold for v in logits], dtype=bool)


def evaluate(exact: np.ndarray, approx: np.ndarray, threshold: float, tol: float) -> dict:
    """The synthetic parity criteria of one mode against the exact tier's logits of the same clips."""
    exact = np.asarray(exact, np.float64)
    approx = np.asarray(approx, np.float64)
    if exact.shape != approx.shape or exact.ndim != 1 or exact.size == 0:
        raise ValueError("exact and approximate logits must be non-empty vectors of one length")
    finite = bool(np.isfinite(approx).all() and np.isfinite(exact).all())
    diff = np.abs(approx - exact)
    max_abs = float(diff.max()) if finite else math.inf
    flips = int((decisions(approx, threshold) != decisions(exact, threshold)).sum())
    near = float(np.min(np.abs(np.array([_shv().sigmoid64(float(v)) for v in exact]) - threshold)))
    ok = finite and max_abs <= tol and flips == 0
    return {"verdict": "PASS" if ok else "FAIL", "threshold": float(threshold), "n_clips": int(exact.size),
            "all_finite": finite, "max_abs_dlogit": max_abs, "mean_abs_dlogit": float(diff.mean()) if finite else None,
            "flips": flips, "closest_exact_score_to_threshold": near,
            "criteria": {"max_abs_dlogit": tol, "flips": 0, "all_finite": True,
                         "decision": "sigmoid(logit) >= threshold (double)", "baseline": "fp32 tier (exact)"}}


def cert_line(sha: str, mode: str, revision: str, json_path: str, json_sha: str, threshold: float) -> str:
    return f"{sha} {mode} {revision} PASS {json_path} {json_sha} threshold={float(threshold)!r}"


def merge_certificate(path: Path, sha: str, revision: str, new_lines: dict[str, str]) -> str:
    """The certificate file text: the header, the existing lines for other (weights, mode, revision), then new_lines
    (mode -> line).  A file with another header is replaced."""
    kept = []
    if path.exists():
        lines = path.read_text().splitlines()
        if lines and lines[0].strip() == HEADER:
            for ln in lines[1:]:
                f = ln.split()
                if len(f) >= 4 and f[0] == sha and f[2] == revision and f[1] in new_lines:
                    continue
                if ln.strip():
                    kept.append(ln)
    return "\n".join([HEADER] + kept + [new_lines[m] for m in sorted(new_lines)]) + "\n"


def run_logits(weights: Path, mode: str, clips: np.ndarray, batch: int, experimental: bool) -> np.ndarray:
    shv = _shv()
    out = []
    with shv.Model(weights, mode, experimental=experimental, max_frames=batch * 20, max_windows=batch) as m:
        for i in range(0, len(clips), batch):
            out.append(m.predict(clips[i:i + batch]))
    return np.concatenate(out).astype(np.float32)


def certify(weights: Path, modes: list[str], clips: np.ndarray, tol: float, batch: int, source: str) -> dict:
    shv = _shv()
    weights = Path(weights)
    revision = shv.library().shv_hip_compute_revision().decode()
    with shv.Model(weights, "fp32", max_frames=batch * 20, max_windows=batch) as m:
        sha, threshold = m.fingerprint, m.threshold
    exact = run_logits(weights, "fp32", clips, batch, experimental=False)
    results, lines = {}, {}
    for mode in modes:
        approx = run_logits(weights, mode, clips, batch, experimental=True)
        res = evaluate(exact, approx, threshold, tol)
        res.update({"mode": mode, "revision": revision, "weights_sha256": sha, "data": source})
        jpath = Path(str(weights) + f".hip.cert.{mode}.json")
        text = json.dumps(res, indent=1, sort_keys=True) + "\n"
        jpath.write_text(text)
        results[mode] = res
        if res["verdict"] == "PASS":
            lines[mode] = cert_line(sha, mode, revision, jpath.name, hashlib.sha256(text.encode()).hexdigest(),
                                    threshold)
    cert = Path(str(weights) + ".hip.cert")
    cert.write_text(merge_certificate(cert, sha, revision, lines))
    # the certified modes must now load through the checking library
    for mode in lines:
        m = shv.Model(weights, mode, max_frames=20, max_windows=1)
        m.close()
    return results


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--weights", required=True, type=Path)
    ap.add_argument("--modes", nargs="+", default=["fp16", "bf16"], choices=["fp16", "bf16"])
    ap.add_argument("--clips", type=int, default=64, help="seeded synthetic clips (ignored with --clips-npy)")
    ap.add_argument("--seed", type=int, default=1000)
    ap.add_argument("--clips-npy", type=Path, help="uint8 [N][20][180][320][3] crops to certify on")
    ap.add_argument("--tol", type=float, default=1e-2, help="largest allowed |logit - exact logit|")
    ap.add_argument("--batch", type=int, default=32)
    args = ap.parse_args()
    if args.clips_npy:
        clips = np.load(args.clips_npy)
        if clips.dtype != np.uint8 or clips.ndim != 5 or clips.shape[1:] != (20, 180, 320, 3):
            print("--clips-npy must hold uint8 [N][20][180][320][3]", file=sys.stderr)
            return 2
        source = f"caller crops {args.clips_npy.name} ({len(clips)} clips)"
    else:
        clips = _shv().synth_clips(args.clips, args.seed)
        source = f"seeded synthetic clips ({args.clips}, seed {args.seed})"
    res = certify(args.weights, args.modes, clips, args.tol, args.batch, source)
    for mode, r in res.items():
        print(f"{mode}: {r['verdict']}  max|dlogit| {r['max_abs_dlogit']:.3e}  flips {r['flips']}  "
              f"({r['n_clips']} clips, tol {args.tol:g})")
    print(Path(str(args.weights) + ".hip.cert").read_text(), end="")
    return 0 if all(r["verdict"] == "PASS" for r in res.values()) else 1


if __name__ == "__main__":
    sys.exit(main())
