"""The C++ host API (include/tmsample_amd.hpp) on the GPU: the check program
tests/cpp/host_api_check (built by __graft_entry__.build()) drives
Sampler::sample / sample_token with std::mt19937 generators and compares
tokens and generator states with the C oracle."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build", "host_api_check")


def test_cpp_host_api_matches_oracle():
    assert os.path.exists(BIN), f"{BIN} not built: run __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=100)
    print(r.stdout[-3000:], r.stderr[-2000:])
    assert r.returncode == 0, r.stdout[-3000:]
    assert "0 failures" in r.stdout
