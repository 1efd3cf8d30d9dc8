"""The rope kernels' sin/cos (sharplight_amd/csrc/rope_math.hpp, f64 reduction + f32 series) against f64
libm narrowed to f32, the CPU provider's RopeOp arithmetic (src/Sharplight.Cpu/RopeOp.cs:123-183:
(float)Math.Cos/Sin of an f64 angle): within 1 f32 ulp on 8.3M angles. Compiled as host code with hipcc."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_sincos_within_one_ulp_of_libm(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = tmp_path / "rope_math_check"
    subprocess.run([hipcc, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950", "-o", str(exe),
                    os.path.join(ROOT, "tests", "rope_math_check.cpp")], check=True, capture_output=True, timeout=300)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=120).stdout.split()
    n, exact, worst = int(out[1]), int(out[3]), int(out[5])
    assert n > 8_000_000
    assert worst <= 1, out
    assert exact > 0.6 * n
