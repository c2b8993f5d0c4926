"""Builds libtmsample_hip.so in-tree for gfx950 with hipcc.

Usage: python -m tensormark_amd.build   (or tensormark_amd.build.build())
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libtmsample_hip.so")
SOURCES = ["tms_sample.hip", "tms_topk.hip", "tms_dense.hip", "tms_spec.hip", "tms_debug.hip", "tms_history.cpp", "tms_grammar.cpp"]

# -ffp-contract=off keeps every a*b+c as two rounded operations, so the
# device arithmetic matches the host checker bit for bit.  Packed-FP32 ops
# are disabled for every HIP translation unit.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]

# Per-file flags.  The top-k kernel takes its row ticket as soon as its
# stream is in and uses the result only after publishing; the atomic
# optimizer would rewrite that single-lane atomic into a wave-wide one whose
# result is broadcast at once, waiting out the round trip there.
FILE_FLAGS = {
    "tms_topk.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}

BUILD_DIR = os.path.join(HERE, "_build")


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _run(cmd: list, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libtmsample_hip.so: " + " ".join(cmd))


def build(verbose: bool = False) -> str:
    """Compiles every source to an object (in parallel), then links the library."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include")]
    jobs = []
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        jobs.append((obj, [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src, []), *inc, "-c", "-o", obj,
                           os.path.join(CSRC, src)]))
    workers = min(len(jobs), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(lambda j: _run(j[1], verbose), jobs))
    _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB + ".tmp", *[j[0] for j in jobs]], verbose)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
