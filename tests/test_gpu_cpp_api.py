"""GPU run of the evk / evk::ai C++ API tests (tests/cpp/api_tests.cpp):
the reference's example/tests.h known answers through include/evk_ai.h,
plus host-fp64 parity of matmul, flash forward (with LSE), the backward
through the saved LSE (finite differences) and single-query attention."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_cpp_api_suite():
    exe = os.path.join(ROOT, "evk_amd", "bin", "api_tests")
    assert os.path.exists(exe), "evk_amd/bin/api_tests is not built: run `python -m evk_amd.build`"
    print("running", exe, flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=110)
    sys.stdout.write(r.stdout[-4000:])
    assert r.returncode == 0 and "ALL PASSED" in r.stdout, r.stdout[-3000:] + r.stderr[-2000:]
