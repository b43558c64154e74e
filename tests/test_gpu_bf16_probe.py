"""The kernels round fp32 to bf16 with gfx950's v_cvt_pk_bf16_f32 only if it
matches the reference's rounding (src/tensor/dtype.h:39-46) on every fp32
bit pattern; build/bf16_cvt_probe checks all 2^32 of them on the device."""

import os
import subprocess

import pytest

from conftest import PKG_DIR

pytestmark = pytest.mark.gpu


def test_hardware_bf16_rounding_matches_reference_on_all_patterns():
    r = subprocess.run([os.path.join(PKG_DIR, "build", "bf16_cvt_probe")], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout)
    if r.returncode == 77:
        pytest.skip("no HIP device")
    assert r.returncode == 0, r.stdout + r.stderr
