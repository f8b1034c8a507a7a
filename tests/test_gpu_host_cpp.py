"""The C++ host mirror (HipBackend / HipVerifier, xwfes_amd/host/) on the GPU:
runs tests/cpp/test_hip_backend, which checks IBackend::matmul,
run_expert_chunk, the reference's greedy-acceptance known answer, and a
2-layer chain / tree verify plus greedy / ratio acceptance against the
oracle (tests/cpp/test_hip_backend.cpp)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_hip_backend")


@pytest.mark.gpu
def test_cpp_host_mirror():
    assert os.path.exists(BIN), "build the package first (tests/cpp/test_hip_backend missing)"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert "all" in r.stdout and "checks passed" in r.stdout
