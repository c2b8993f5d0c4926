"""Writes tests/golden/tie_golden.npz: rows with exact ties, sampled by the
reference's compiled tmsample::sample (oracle/_ref) under this container's
libstdc++.

The reference's order among equal values is whatever std::nth_element and
std::sort leave (unspecified); the library's contract is lowest id first.
For each row the reference's top-k order is read back from the unmodified
sample() by drawing once at the middle of every probability bucket (the
draw's words are chosen through a crafted std::mt19937), so the fixture
records, per row, the ids the reference puts at each rank, next to a few
draws at random uniforms.  Run where oracle/_ref is built:

    python tests/golden/make_tie_golden.py
"""
from __future__ import annotations

import ctypes as C
import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tie_golden.npz")
REF = os.path.join(ROOT, "oracle", "_ref", "libtmsample_ref.so")


def words_for(u: float):
    w = min(int(u * 2.0 ** 64), 2 ** 64 - 1)
    return w & 0xFFFFFFFF, w >> 32


def buckets(vals_desc, T, p):
    """The reference's pr, keep and discrete_distribution cumulative table
    for top-k values in descending order (ties do not change them)."""
    lg = [np.float32(v) / np.float32(T) for v in vals_desc]
    mx = float(lg[0])
    pr = [math.exp(float(x) - mx) for x in lg]
    z = 0.0
    for q in pr:
        z += q
    cum, keep = 0.0, len(pr)
    for k, q in enumerate(pr):
        cum += q / z
        if cum >= p:
            keep = k + 1
            break
    s = 0.0
    for q in pr[:keep]:
        s += q
    cp, acc = [], 0.0
    for q in pr[:keep]:
        acc += q / s
        cp.append(acc)
    cp[-1] = 1.0
    return keep, cp


def main():
    if not os.path.exists(REF):
        raise SystemExit("oracle/_ref not built: make -C oracle")
    lib = C.CDLL(REF)
    lib.ref_sample_words.argtypes = [C.c_void_p, C.c_int, C.c_float, C.c_int, C.c_float, C.c_int,
                                     C.c_uint32, C.c_uint32]
    rng = np.random.default_rng(20261202)
    rows = []
    # (V, distinct levels, k, top_p, T)
    specs = [(7, 4, 3, 1.0, 1.0), (16, 3, 5, 1.0, 1.0), (64, 6, 10, 1.0, 0.8), (64, 4, 40, 0.9, 1.0),
             (300, 8, 40, 0.95, 0.7), (2000, 12, 100, 0.98, 1.2), (1000, 5, 1, 1.0, 1.0),
             (128, 2, 64, 1.0, 1.0)]
    for V, levels, k, p, T in specs:
        for rep in range(6):
            lv = np.sort(rng.normal(0.0, 1.5, levels)).astype(np.float32)
            x = lv[rng.integers(0, levels, V)].astype(np.float32)
            order = sorted(range(V), key=lambda i: (-float(x[i]), i))
            vals = [float(x[i]) for i in order[:k]]
            keep, cp = buckets(vals, T, p)
            ref = []
            for j in range(keep):
                lo = cp[j - 1] if j else 0.0
                w0, w1 = words_for((lo + cp[j]) / 2.0)
                t = lib.ref_sample_words(x.ctypes.data, V, T, k, p, 0, w0, w1)
                assert t >= 0
                ref.append(t)
            draws = []
            for _ in range(8):
                w0, w1 = int(rng.integers(0, 2 ** 32)), int(rng.integers(0, 2 ** 32))
                draws.append((w0, w1, lib.ref_sample_words(x.ctypes.data, V, T, k, p, 0, w0, w1)))
            rows.append(dict(x=x, T=T, k=k, p=p, keep=keep, ref=np.array(ref, np.int32),
                             draws=np.array(draws, np.int64)))
    arrays = {}
    for i, r in enumerate(rows):
        arrays[f"x{i}"] = r["x"]
        arrays[f"ref{i}"] = r["ref"]
        arrays[f"draws{i}"] = r["draws"]
    arrays["meta"] = np.array([(r["T"], r["k"], r["p"], r["keep"]) for r in rows],
                              dtype=[("T", "<f4"), ("k", "<i4"), ("p", "<f4"), ("keep", "<i4")])
    np.savez_compressed(OUT, **arrays)
    lowest = sum(1 for r in rows
                 if list(r["ref"]) != sorted(range(len(r["x"])), key=lambda i: (-float(r["x"][i]), i))[:r["keep"]])
    print(f"wrote {len(rows)} rows to {OUT} ({os.path.getsize(OUT)} bytes); "
          f"{lowest} differ from lowest-id-first")


if __name__ == "__main__":
    main()
