"""The FP8 quantizer divides with Markstein's correction step instead of IEEE
divisions (fp8_quant.hip: markstein(), row_div, quant_rows_smooth_kernel).
This pins that the two give the same E4M3 codes: bitwise-equal quotients for
|x| >= 2^-102 when the quotient is a normal number, and values with the sign
of x far below the smallest E4M3 step otherwise (modes 0 and 1); and that the
SmoothQuant route, which also divides by the smoothing factors that way and
keeps a row only when its largest quotient passes a range check, returns the
reference pipeline's codes and row scales for every row it keeps (mode 2).
The check is a C program (tests/csrc/markstein_check.c) built with gcc,
because numpy has no fused multiply-add.  KC_SLOW=1 adds the complete code
check of the row-scale route (mode 3: every scale significand against every
E4M3 rounding boundary, 1.9e10 quotients), every scale significand against
random x (mode 4) and exhaustive sweeps over all 2^32 x for twelve scales
(mode 1); a record of one such run is tests/golden/markstein_sweep.txt."""
import os
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "csrc" / "markstein_check.c"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("markstein") / "markstein_check"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
                    str(SRC), "-o", str(exe), "-lm"], check=True)
    return exe


def _run(checker, *args):
    r = subprocess.run([str(checker), *map(str, args)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
    assert r.stdout.strip() == "mismatches 0"


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_markstein_matches_ieee_division_random(checker, seed):
    _run(checker, 0, 256, seed)


@pytest.mark.parametrize("seed", [1, 2])
def test_smoothquant_route_matches_two_step_reference(checker, seed):
    _run(checker, 2, 20000, seed)


def test_markstein_all_scale_significands_quick(checker):
    """Every one of the 2^23 scale significands against 4 random x each."""
    _run(checker, 4, 4, 3)


@pytest.mark.skipif(os.environ.get("KC_SLOW") != "1", reason="exhaustive sweep: set KC_SLOW=1")
@pytest.mark.parametrize("which", range(12))
def test_markstein_matches_ieee_division_exhaustive(checker, which):
    _run(checker, 1, which)


@pytest.mark.skipif(os.environ.get("KC_SLOW") != "1", reason="exhaustive sweep: set KC_SLOW=1")
def test_row_scale_codes_at_every_e4m3_boundary(checker):
    _run(checker, 3, 0)


@pytest.mark.skipif(os.environ.get("KC_SLOW") != "1", reason="exhaustive sweep: set KC_SLOW=1")
def test_markstein_all_scale_significands(checker):
    _run(checker, 4, 256, 7)
