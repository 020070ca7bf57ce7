"""The device Q8 quantizer rounds half away from zero as
trunc(y + copysign(0.5 - 2^-25, y)) (pi_gemv.h, q8_round_clamp); this checks
that identity against roundf for every float |y| < 2^22 (quant_int.rs:49
multiplies by 1/d with |x| <= amax, so |y| <= 127.00003 in the kernels).
The ties themselves are also checked on the device by
tests/test_gpu_kernels.py::test_q8_quantize_every_tie."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_round_half_away_identity_exhaustive(tmp_path):
    exe = tmp_path / "q8_round_identity"
    subprocess.run(["gcc", "-O2", "-fno-fast-math", "-ffp-contract=off", str(HERE / "q8_round_identity.c"),
                    "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "checked 2499805184 floats, 0 differ" in r.stdout
