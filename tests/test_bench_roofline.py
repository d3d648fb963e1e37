"""bench.py's roofline line on the CPU: the dominant family is the one with the most device time per step, its roof
is the one its intensity selects, and the PMC figures of profiles/roofline_traffic.json (HBM bytes per launch, VALU /
MFMA busy fractions) are used only for the family and library revision they were measured on."""
import importlib.util
import json
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("shv_bench", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


STATS = {   # two steps: family -> summed ms, launches, algorithmic bytes and FLOPs
    "ir_40x120x40": {"ms": 3.6, "launches": 16, "bytes": 16 * 382e6, "flops": 16 * 9.19e9},
    "gemm_seq:gemm_dma_kernel<f16,2,4,2>": {"ms": 1.9, "launches": 28, "bytes": 28 * 150e6, "flops": 28 * 23e9},
    "gdn_prep": {"ms": 0.8, "launches": 12, "bytes": 12 * 300e6, "flops": 0.0},
}


def test_dominant_family_and_hbm_roof(bench):
    r = bench.roofline_of(STATS, 2, "fp16", "hip-test", traffic_file=False)
    assert r["kernel"] == "ir_40x120x40"
    assert r["bound"] == "hbm" and r["unit"] == "GB/s"
    avg_ms = 3.6 / 16
    assert r["avg_launch_ms"] == pytest.approx(avg_ms, abs=1e-4)
    assert r["achieved"] == pytest.approx(382e6 / (avg_ms / 1e3) / 1e9, rel=1e-3)
    assert r["frac"] == pytest.approx(r["achieved"] / bench.HBM_PEAK_GBS, rel=1e-3)
    assert r["launches_per_step"] == 8 and r["traffic"] is None
    assert "valu_busy_frac" not in r


def test_mfma_roof_above_the_ridge(bench):
    stats = {"gemm": {"ms": 1.0, "launches": 10, "bytes": 10 * 1e6, "flops": 10 * 1e12}}   # 1e6 FLOP/B
    r = bench.roofline_of(stats, 1, "fp16", "hip-test", traffic_file=False)
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s"
    assert r["achieved"] == pytest.approx(1e12 / 1e-4 / 1e12, rel=1e-3)


def test_counter_file_only_for_its_revision_and_family(bench, tmp_path, monkeypatch):
    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "roofline_traffic.json").write_text(json.dumps(
        {"revision": "hip-aaaa", "family": "ir_40x120x40", "traffic_bytes_per_launch": 479000000,
         "valu_busy_frac": 0.66, "mfma_busy_frac": 0.12}))
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    r = bench.roofline_of(STATS, 2, "fp16", "hip-aaaa")
    assert r["traffic"] == 479000000 and r["valu_busy_frac"] == 0.66 and r["mfma_busy_frac"] == 0.12
    stale = bench.roofline_of(STATS, 2, "fp16", "hip-bbbb")   # another library revision
    assert stale["traffic"] is None and "valu_busy_frac" not in stale
    other = {k: v for k, v in STATS.items() if k != "ir_40x120x40"}   # another dominant family
    assert bench.roofline_of(other, 2, "fp16", "hip-aaaa")["traffic"] is None
