"""GPU test of the C++ host layer (neutron-star_amd/host/ffn_path.hpp): the
compiled tests/cpp/ffn_path_test drives FfnPath like the reference engine's FFN
block (decode + lm-head, prefill in both modes) and checks each output against
the CPU oracle, then the std::runtime_error convention."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(__file__), "cpp", "_build", "ffn_path_test")


def test_cpp_ffn_path():
    assert os.path.exists(BIN), "build the test binary with __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED" in r.stdout
