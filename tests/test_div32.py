"""Host check of the kernels' index division (mq::Div32, a multiply and a
shift) against integer division, compiled from the library's own header."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIP_INCLUDE = "/opt/rocm/include"


@pytest.mark.skipif(shutil.which("g++") is None or not os.path.isdir(HIP_INCLUDE),
                    reason="needs g++ and the HIP headers")
def test_div32_matches_integer_division(tmp_path):
    exe = tmp_path / "div32_check"
    cmd = ["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{HIP_INCLUDE}",
           f"-I{os.path.join(ROOT, 'metal-native_amd', 'csrc')}",
           os.path.join(ROOT, "tests", "native", "div32_check.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "bad 0" in out.stdout
