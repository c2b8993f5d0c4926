"""Builds libtmsample_hip.so in-tree for gfx950 with hipcc.

Usage: python -m tensormark_amd.build   (or tensormark_amd.build.build())
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libtmsample_hip.so")
SOURCES = ["tms_sample.hip", "tms_wide.hip", "tms_sparse.hip", "tms_rows.hip", "tms_hist.hip", "tms_chain.hip", "tms_spec.hip", "tms_debug.hip", "tms_history.cpp", "tms_grammar.cpp", "tms_filter.cpp"]

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

# Per-file flags.  The wide top-k kernel takes its row ticket as soon as
# the stream is in and uses the result only after publishing; the atomic
# optimizer would rewrite that single-lane atomic into a wave-wide one whose
# result is broadcast at once, waiting out the round trip there.
FILE_FLAGS = {
    "tms_wide.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}

BUILD_DIR = os.path.join(HERE, "_build")


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _run(cmd: list, verbose: bool) -> str:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libtmsample_hip.so: " + " ".join(cmd))
    return r.stderr


# Files whose kernels must not use scratch memory.  The wide kernel runs at
# two 1024-thread workgroups per CU (64 VGPRs), and a build of it that
# spilled to scratch under that limit sampled wrong tokens on the GPU; the
# verify kernels hold whole rows in registers, where a spill would turn the
# one read of the row into scratch traffic; the general kernel launched its
# workgroups measurably slower with any scratch (B = 1024, V = 256000 bf16:
# 243.5 against 232.3 us with 32 bytes a lane).
NO_SCRATCH = ("tms_wide.hip", "tms_spec.hip", "tms_sample.hip", "tms_sparse.hip", "tms_rows.hip")


def _check_no_scratch(src: str, remarks: str) -> None:
    sizes = re.findall(r"ScratchSize \[bytes/lane\]: (\d+)", remarks)
    if not sizes:
        raise RuntimeError(f"{src}: no kernel resource report from hipcc")
    if any(int(x) for x in sizes):
        raise RuntimeError(f"{src}: a kernel uses scratch memory ({sizes}); it must fit its register limit")


# Largest LDS a kernel of the file may take.  Four general-kernel
# workgroups share a CU's 160 KiB of LDS; a few hundred bytes more (a
# runtime helper's LDS word, say) would leave three and add a round of
# residency to a 1,280-workgroup grid.
LDS_MAX = {"tms_sample.hip": 40960}


def _check_lds(src: str, remarks: str) -> None:
    sizes = [int(x) for x in re.findall(r"LDS Size \[bytes/block\]: (\d+)", remarks)]
    if not sizes:
        raise RuntimeError(f"{src}: no kernel resource report from hipcc")
    if max(sizes) > LDS_MAX[src]:
        raise RuntimeError(f"{src}: a kernel takes {max(sizes)} bytes of LDS, above {LDS_MAX[src]}")


def build(verbose: bool = False) -> str:
    """Compiles every source to an object (in parallel), then links the library."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include")]
    jobs = []
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        extra = ["-Rpass-analysis=kernel-resource-usage"] if src in NO_SCRATCH else []
        jobs.append((src, obj, [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src, []), *inc, *extra, "-c", "-o",
                                obj, os.path.join(CSRC, src)]))
    workers = min(len(jobs), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        remarks = list(ex.map(lambda j: _run(j[2], verbose), jobs))
    for (src, _, _), rem in zip(jobs, remarks):
        if src in NO_SCRATCH:
            _check_no_scratch(src, rem)
        if src in LDS_MAX:
            _check_lds(src, rem)
    _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB + ".tmp", *[j[1] for j in jobs]], verbose)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
