"""The activation quantizers divide by the row scale through its reciprocal (`quant1_recip`,
csrc/lse_common.h) wherever that is exact. This pins the claim by exhaustion on the CPU: every
bf16 row maximum in the reciprocal path's range and every bf16 value of such a row quantize to
the same int8 as with an IEEE division (`tests/quant_recip_check.c`). The plain product by the
reciprocal, without its correction step, must fail the same check."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).with_name("quant_recip_check.c")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    exe = tmp_path_factory.mktemp("quant_recip") / "check"
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", str(SRC),
                    "-o", str(exe), "-lm"], check=True)
    return exe


def _run(exe, *args):
    out = subprocess.run([str(exe), *args], check=True, capture_output=True, text=True,
                         env={"OMP_NUM_THREADS": "8"}).stdout.split()
    return dict(zip(out[0::2], map(int, out[1::2])))


def test_reciprocal_quantizer_matches_division_for_every_bf16_row(checker):
    r = _run(checker)
    assert r["rows"] == 28290 and r["pairs"] == 523237695
    assert r["mismatches"] == 0


def test_the_check_catches_a_dropped_correction(checker):
    assert _run(checker, "uncorrected")["mismatches"] > 0
