"""Runs the C++ API test program (tests/cpp/test_gpu_api.cpp) on the GPU: the reference's GPU test cases
through veckern::gpu::PQSearcher, checked bit-exactly against the oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build", "test_gpu_api")


def test_cpp_api_program():
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} not built: run `make -C tests/cpp`")
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
