"""Builds the C++ host-API check program (tests/cpp/_build/host_api_check)
against the in-tree libtmsample_hip.so and the oracle's libtms_oracle.so.
Test infrastructure; called by __graft_entry__.build() after both libraries.

    python tests/cpp/build.py
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "_build", "host_api_check")


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cmd = [os.path.join(rocm, "bin", "hipcc"), "--offload-arch=gfx950", "-std=c++17", "-O2", "-Wall",
           "-I", os.path.join(ROOT, "include"),
           "-o", OUT + ".tmp", os.path.join(HERE, "host_api_check.cpp"),
           "-L", os.path.join(ROOT, "tensormark_amd"), "-ltmsample_hip",
           "-L", os.path.join(ROOT, "oracle", "_build"), "-ltms_oracle",
           "-Wl,-rpath,$ORIGIN/../../../tensormark_amd",
           "-Wl,-rpath,$ORIGIN/../../../oracle/_build"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building tests/cpp/host_api_check")
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
