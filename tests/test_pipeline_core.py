"""The page pipeline's schedule (csrc/pipeline_core.h) on the CPU, with hooks that fail on purpose
(tests/cpp/test_pipeline_core.cpp): a failing stage, detection, layout, recognition or decode
fails exactly the pages it covers and every other page finishes, as the reference reports errors
per page (src/bin/ocr-bench.rs:277-281, 303-307). Built with g++ under AddressSanitizer +
UndefinedBehaviorSanitizer, and under ThreadSanitizer. The bounded host wait (csrc/wait.h) is
forced past its deadline there: a stalled detection group fails its own pages with an error
naming it, and the other pages finish."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "wgpu-ocr_amd", "csrc")
SRC = os.path.join(ROOT, "tests", "cpp", "test_pipeline_core.cpp")


def _build_and_run(tmp_path, sanitize):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path / f"core_{sanitize.replace(',', '_')}")
    cmd = ["g++", "-std=c++17", "-O1", "-g", f"-fsanitize={sanitize}", "-fno-omit-frame-pointer", "-I", CSRC,
           SRC, "-o", exe, "-pthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               TSAN_OPTIONS="halt_on_error=1", OCR_WAIT_TIMEOUT_MS="25")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout


def test_schedule_faults_asan_ubsan(tmp_path):
    _build_and_run(tmp_path, "address,undefined")


def test_schedule_faults_tsan(tmp_path):
    _build_and_run(tmp_path, "thread")
