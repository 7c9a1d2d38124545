"""The C++ wrapper (include/reef_hip/attention.hpp) compiles against the C ABI
and maps statuses to the engine's exceptions (std::invalid_argument,
std::length_error) with the engine's messages. Host-only: every call fails
validation before any launch."""
import os
import shutil
import subprocess

import pytest

import reef_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_wrapper_maps_statuses_to_engine_exceptions(tmp_path):
    reef_amd.lib()  # the library must be built
    exe = tmp_path / "wrapper_check"
    libdir = os.path.dirname(reef_amd.LIB_PATH)
    cmd = ["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include",
           os.path.join(ROOT, "tests", "cxx", "wrapper_check.cpp"),
           "-L", libdir, "-lreef_hip", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
