"""The quantizers' short division sequences (csrc/common.hpp div127_rn and
rcp_rn, which form each row's scale s = max(rowmax / 127, 1e-30) and 1 / s)
against IEEE division on the device, over every float of their ranges:
tests/c_abi/rounding_check.hip, built with the library."""

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "rounding_check")


def test_division_sequences_equal_ieee_division_everywhere():
    assert os.path.exists(BIN), "tests/c_abi/rounding_check is not built (run build())"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "div127_rn mismatches: 0 of 2139095041" in r.stdout
    assert "rcp_rn mismatches: 0 of " in r.stdout
