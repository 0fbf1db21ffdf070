"""Exhaustive checks of the two division-free steps in the Q8_1 quantizers (q8_1_scale and q8_1_rcp in
tinystrata_amd/csrc/tsx_device.hpp), whose codes must equal the reference's IEEE-division codes bit for bit:
amax / 127 as a corrected product (every non-negative finite float, on the host) and 1 / d as the hardware reciprocal
with one Newton step (every float in [2^-100, 2^100], on the GPU)."""
import ctypes as C
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div127_corrected_product_is_the_ieee_quotient(tmp_path):
    exe = tmp_path / "div127_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", str(ROOT / "tests" / "numerics" / "div127_check.c"),
                    "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600).stdout
    assert out.strip() == "mismatches 0", out


@pytest.mark.gpu
def test_rcp_newton_is_the_ieee_reciprocal():
    import torch  # noqa: F401  (the GPU runtime is up, as in the other GPU tests)

    lib = C.CDLL(str(ROOT / "tinystrata_amd" / "libtsx_numerics_check.so"))
    lib.tsx_check_rcp_newton.argtypes = [C.POINTER(C.c_ulonglong)]
    bad = C.c_ulonglong(123)
    assert lib.tsx_check_rcp_newton(C.byref(bad)) == 0
    assert bad.value == 0
