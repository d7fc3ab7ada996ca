"""The device powf (birdnet-neon-engine_amd/csrc/bnh_powf.h, a restatement of glibc's powf, used by GEM_A's final
power) compiled for the host and compared with the C library's powf (tests/native/powf_check.c, 8 threads): every
13th float in [2^-130, 2^8) against y = 1/p for eleven values of p, 2 million random pairs over all finite x and
|y| <= 64, and the special cases (zeros, infinities, NaNs, negative x with odd, even and non-integer y). A correctly
rounded powf fails this: glibc's differs from correct rounding on about 7 in 10^4 of GEM_A's arguments."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.timeout(300)
def test_powf_matches_c_library(tmp_path):
    exe = str(tmp_path / "powf_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", os.path.join(ROOT, "birdnet-neon-engine_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "powf_check.c"), "-o", exe, "-lm", "-lpthread"], check=True)
    r = subprocess.run([exe, "2000000", str(min(8, os.cpu_count() or 1)), "13"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
