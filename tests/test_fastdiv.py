"""Host check of the multiply-high index division used by the HBM kernels
(ringmaster_amd/csrc/rmx_fastdiv.h): the header is compiled for the host and
compared with exact integer division on edge and random operands."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not Path(HIPCC).exists() and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_fastdiv_matches_integer_division(tmp_path):
    exe = tmp_path / "fastdiv_check"
    src = ROOT / "tests" / "native" / "fastdiv_check.cpp"
    subprocess.run([HIPCC, "-x", "c++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__",
                    "-I", "/opt/rocm/include",
                    "-I", str(ROOT / "ringmaster_amd" / "csrc"), str(src), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "0 mismatches" in res.stdout
