import importlib.util
import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


# measured parity margins, printed in the terminal summary (which shows even when test output is captured)
_MARGINS = []


@pytest.fixture
def margin():
    """margin(what, measured, bound): record a measured error next to the bound its test holds it to."""
    def record(what, measured, bound):
        _MARGINS.append((what, float(measured), float(bound)))
    return record


def pytest_terminal_summary(terminalreporter):
    if not _MARGINS:
        return
    terminalreporter.write_sep("-", "measured parity margins")
    for what, v, b in _MARGINS:
        terminalreporter.write_line(f"{what}: {v:.3e} (bound {b:.1e}, {v / b:.0%} of it)")


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def shv():
    return _load("shv_hip", ROOT / "shield-sisa_amd" / "shv_hip.py")


@pytest.fixture(scope="session")
def orc():
    import oracle
    if not oracle.ORACLE_SO.exists():
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def golden():
    return json.loads((GOLDEN / "golden_seed1.json").read_text())


@pytest.fixture(scope="session")
def golden_tokens():
    return np.load(GOLDEN / "tokens_clip0.npy")


@pytest.fixture(scope="session")
def weights(tmp_path_factory, shv, golden):
    d = tmp_path_factory.mktemp("weights")
    w = d / "seed1.weights"
    sha = shv.write_weights(w, seed=1, threshold=golden["threshold"])
    assert sha == golden["weights_sha256"], "synthetic weight generator drifted from the golden fixture"
    return w


@pytest.fixture(scope="session")
def clips(shv, golden):
    c = shv.synth_clips(len(golden["logits"]), 1000)
    assert shv.sha256_bytes(c[0]) == golden["clip_sha256"][0]
    return c


@pytest.fixture(scope="session")
def golden_logits(golden):
    return np.array(golden["logits_f32_bits"], np.uint32).view(np.float32)
