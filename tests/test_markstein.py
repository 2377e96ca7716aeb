"""The FP8 quantizer divides by the row scale with Markstein's correction step
instead of an IEEE division (fp8_quant.hip, row_div).  This pins that the two
give the same E4M3 codes: bitwise-equal quotients for |x| >= 2^-103 when
the quotient is a normal number, and same-sign values far below the smallest
E4M3 step otherwise.  The check is a
C program (tests/csrc/markstein_check.c) built with gcc, because numpy has no
fused multiply-add.  KC_SLOW=1 adds exhaustive sweeps over all 2^32 x for six
scales (about a minute each)."""
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


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_markstein_matches_ieee_division_random(checker, seed):
    r = subprocess.run([str(checker), "0", "256", str(seed)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
    assert r.stdout.strip() == "mismatches 0"


@pytest.mark.skipif(os.environ.get("KC_SLOW") != "1", reason="exhaustive sweep: set KC_SLOW=1")
@pytest.mark.parametrize("which", [0, 1, 3, 5, 6, 10])
def test_markstein_matches_ieee_division_exhaustive(checker, which):
    r = subprocess.run([str(checker), "1", str(which)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
