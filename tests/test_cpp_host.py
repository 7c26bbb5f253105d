"""Host logic of the evk core and evk::ai C++ layer (evk_amd/csrc/evk_runtime.cpp,
evk_amd/csrc/evk_ai.cpp) without a GPU: tests/cpp/host_tests.cpp built with
g++ against a host-memory HIP mock and a recording stub of the C ABI, under
the address and undefined-behaviour sanitizers."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_cpp_host_layer(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None or not os.path.exists("/opt/rocm/include/hip/hip_runtime_api.h"):
        pytest.skip("needs g++ and the ROCm headers")
    exe = tmp_path / "host_tests"
    srcs = ["evk_amd/csrc/evk_runtime.cpp", "evk_amd/csrc/evk_ai.cpp", "tests/cpp/hip_mock.cpp",
            "tests/cpp/evkhip_stub.cpp", "tests/cpp/host_tests.cpp"]
    cmd = [gxx, "-std=c++20", "-g", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "tests", "cpp")]
    cmd += [os.path.join(ROOT, s) for s in srcs] + ["-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout, r.stdout[-3000:] + r.stderr[-3000:]
