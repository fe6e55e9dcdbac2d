"""The fast packer's division-free arithmetic against IEEE float32, on the CPU.

``csrc/pack.hip`` computes the group scale with a Markstein step on the constant RN(1/qmax),
the codes with a Markstein-corrected reciprocal, and -- for groups whose scale is not clamped
above -- the code as the low byte of ``q + 2^23`` (round half to even by the add), Value words
by adding the shifted magic codes minus a constant.  ``pack_arith_check.c`` runs those steps in
the same order with C float32 and ``fmaf`` beside the reference's IEEE formula (layout.py:12-18)
over ranges of every magnitude, exact ties, repeated values and ranges around the 1e5 qmax
boundary.  The GPU tests check the kernel itself against the oracle and the golden data."""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).with_name("pack_arith_check.c")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_and_magic_codes_match_ieee(tmp_path):
    exe = tmp_path / "pack_arith_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(SRC), "-lm"], check=True)
    out = subprocess.run([str(exe), "200000"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "differences 0" in out.stdout
    counts = out.stdout.split("magic ")[1]
    assert int(counts.split(",")[0]) > 0 and int(counts.split("clamped ")[1].split(")")[0]) > 0


def test_reciprocal_row_division_is_exact():
    """The compress kernel's Key-word and fp16-tier loops take row = i / k as
    trunc((i + 0.5) * rcp(k)) with the hardware reciprocal (1 ulp): for every k and i they use
    (k <= 512, i < 512; k <= 128, i < 128 k) any float within 2 ulps of 1 / k gives the exact
    quotient.  Brute force over every case."""
    import numpy as np

    def near(r):
        out = [r]
        lo = hi = r
        for _ in range(2):
            lo = np.nextafter(lo, np.float32(0))
            hi = np.nextafter(hi, np.float32(2))
            out += [lo, hi]
        return out

    for kmax, n_of in ((512, lambda k: 512), (128, lambda k: 128 * k)):
        for k in range(1, kmax + 1):
            n = n_of(k)
            t = np.arange(n, dtype=np.float32) + np.float32(0.5)
            want = np.arange(n) // k
            for r in near(np.float32(1.0) / np.float32(k)):
                got = (t * np.float32(r)).astype(np.float32).astype(np.int64)
                assert np.array_equal(got, want), (k, float(r))
