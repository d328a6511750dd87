"""Word boxes from malformed GPU component records on the CPU (tests/cpp/test_geometry_records.cpp)
under AddressSanitizer + UndefinedBehaviorSanitizer: every record a faulty labelling could hand
over is refused with an error or boxed, never read outside its buffers."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "wgpu-ocr_amd", "csrc")
SRC = os.path.join(ROOT, "tests", "cpp", "test_geometry_records.cpp")
ROCM_INC = "/opt/rocm/include"


def test_geometry_records_asan_ubsan(tmp_path):
    if shutil.which("g++") is None or not os.path.isdir(ROCM_INC):
        pytest.skip("g++ or the HIP headers are not available")
    exe = str(tmp_path / "geometry_records")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-D__HIP_PLATFORM_AMD__", "-I", CSRC, "-I", ROCM_INC, SRC, os.path.join(CSRC, "geometry.cpp"), "-o", exe,
           "-pthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
