"""The kernels' hardswish / hardsigmoid divide by 6 as q = v*fp32(1/6) refined by one fma residual step, zero
returned as itself and the IEEE division only where 0 < |v| < 2.4e-38 (shield-sisa_amd/csrc/dev_common.hpp:
div6_step, div6).  This checks the identity with the IEEE quotient over all 2^32 fp32 inputs: every mismatch of the
plain step lies below the fallback bound (or is -0, which the step turns into +0), and the whole function has none
-- the exact tier's bitwise parity with the reference CPU engine (which divides) rests on it.  CPU only."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div6_formula_equals_ieee_quotient(tmp_path):
    exe = tmp_path / "div6_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe), str(HERE / "native" / "div6_check.c"),
                    "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600).stdout.split()
    mismatches, worst, fn_mismatches = int(out[0]), float(out[1]), int(out[2])
    assert mismatches > 0            # the plain formula is not exact for subnormal quotients ...
    assert worst < 2.4e-38           # ... and all of those lie below the kernels' fallback bound
    assert fn_mismatches == 0        # the function with its zero rule and fallback is the IEEE quotient
