"""The FP8 quantizer divides with Markstein's correction step instead of IEEE
divisions (fp8_quant.hip: markstein(), row_div, quant_rows_smooth_kernel).
This pins that the two give the same E4M3 codes: bitwise-equal quotients for
|x| >= 2^-102 when the quotient is a normal number, and values with the sign
of x far below the smallest E4M3 step otherwise (modes 0 and 1); and that the
SmoothQuant route, which also divides by the smoothing factors that way and
keeps a row only when its largest quotient passes a range check, returns the
reference pipeline's codes and row scales for every row it keeps (mode 2).
The check is a C program (tests/csrc/markstein_check.c) built with gcc,
because numpy has no fused multiply-add.  KC_SLOW=1 adds exhaustive sweeps
over all 2^32 x for eight scales (about a minute each)."""
import os
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "csrc" / "markstein_check.c"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("markstein") / "markstein_check"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", str(SRC),
                    "-o", str(exe), "-lm"], check=True)
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


@pytest.mark.skipif(os.environ.get("KC_SLOW") != "1", reason="exhaustive sweep: set KC_SLOW=1")
@pytest.mark.parametrize("which", [0, 2, 3, 5, 6, 7, 8, 11])
def test_markstein_matches_ieee_division_exhaustive(checker, which):
    _run(checker, 1, which)
