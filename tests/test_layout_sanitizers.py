"""CPU: the layout planner (csrc/layout.cpp) built with AddressSanitizer and
UndefinedBehaviorSanitizer by g++ (host code only) and driven through every
planner entry point over seeded random shapes, dtypes, strides and dim
orders (tests/native/layout_sanitize.cpp): no sanitizer report, every
nest inside its tensors."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_layout_planner_under_sanitizers(tmp_path):
    exe = tmp_path / "layout_sanitize"
    build = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             "-I", os.path.join(ROOT, "torch_spyre_amd", "csrc"),
             os.path.join(ROOT, "tests", "native", "layout_sanitize.cpp"),
             os.path.join(ROOT, "torch_spyre_amd", "csrc", "layout.cpp"), "-o", str(exe)]
    r = subprocess.run(build, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    assert "failures 0" in r.stdout
