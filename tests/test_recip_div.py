"""The int8 KV writes divide by a reciprocal with one fused correction (div_recip in
kv_write.hip) instead of the IEEE division, for rows whose |x| stay below 2^100. This checks, on
the host with the same operations (gcc, fma from libm, no contraction), that the int8 values and
scales cannot differ from the IEEE ones: exhaustively for bf16 inputs against every calibration
the writes produce and against every bf16 row maximum, and on samples of 10^8 random pairs for K
rows after the calibration division and for arbitrary calibrations
(tests/divcheck/recip_div_check.c states the domains)."""

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "divcheck" / "recip_div_check.c"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = tmp_path_factory.mktemp("divcheck") / "recip_div_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", str(SRC), "-o", str(exe),
                    "-lm"], check=True)
    return exe


@pytest.mark.parametrize("mode,n", [("cal", None), ("vrow", None), ("krow", 100_000_000),
                                    ("calr", 100_000_000)])
def test_reciprocal_division_matches_ieee(checker, mode, n):
    args = [str(checker), mode] + ([str(n)] if n else [])
    r = subprocess.run(args, capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0 and " 0 mismatches" in r.stdout, r.stdout


def test_planted_mistake_is_caught(checker, tmp_path):
    """The checker fails where the identity does not hold: outside the domain it states (the
    overflow region past 2^100 that the kernels send to the IEEE division)."""
    src = SRC.read_text().replace("XMAX_BF16 = 0x7180", "XMAX_BF16 = 0x7f80")
    bad = tmp_path / "bad.c"
    bad.write_text(src)
    exe = tmp_path / "bad"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", str(bad), "-o", str(exe),
                    "-lm"], check=True)
    r = subprocess.run([str(exe), "cal"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 1 and "mismatch" in r.stdout
