"""The device expf (birdnet-neon-engine_amd/csrc/bnh_expf.h, a restatement of
glibc's expf) compiled for the host and compared with the C library's expf on
every one of the 2^32 float bit patterns (tests/native/expf_check.c, 8
threads, about 15 s). A correctly rounded expf would fail this: glibc's result
differs from correct rounding on a few arguments in 10^5."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.timeout(300)
def test_expf_matches_c_library_on_every_float(tmp_path):
    exe = str(tmp_path / "expf_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", os.path.join(ROOT, "birdnet-neon-engine_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "expf_check.c"), "-o", exe, "-lm", "-lpthread"], check=True)
    r = subprocess.run([exe, "1", str(min(8, os.cpu_count() or 1))], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
