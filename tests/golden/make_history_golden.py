"""Writes tests/golden/history_golden.npz from the reference's compiled
tmsample.h: input/output rows of apply_no_repeat_ngram (tmsample.h:81-114)
and apply_dry (tmsample.h:148-170) on seeded histories built to repeat.

Run where oracle/_ref/libtmsample_ref.so is built (make -C oracle):

    python tests/golden/make_history_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "history_golden.npz")


def history(rng, n, V, motif_len, repeats):
    """A history that repeats a motif, with noise and a few out-of-range ids."""
    motif = rng.integers(0, V, size=motif_len)
    h = []
    while len(h) < n:
        if rng.random() < repeats:
            h.extend(motif.tolist())
        else:
            h.extend(rng.integers(0, V, size=rng.integers(1, 4)).tolist())
    h = np.array(h[:n], np.int32)
    if rng.random() < 0.3:
        h[rng.integers(0, n)] = V + 5      # out of range: skipped by both transforms
    return h


def main():
    ref = oracle.reference()
    if ref is None:
        raise SystemExit("oracle/_ref not built: make -C oracle")
    rng = np.random.default_rng(20261202)
    d = {}
    meta = []
    i = 0
    for V in (50, 300, 4096):
        for _ in range(10):
            n = int(rng.integers(3, 200))
            h = history(rng, n, V, int(rng.integers(1, 6)), 0.6)
            x = rng.normal(0, 2, size=V).astype(np.float32)
            if rng.random() < 0.2:
                x[rng.random(V) < 0.5] = -np.inf
            kind = i % 2
            if kind == 0:
                ng = int(rng.integers(2, 5))
                y = ref.no_repeat_ngram(x, h, ng)
                meta.append((0, ng, 0.0, 0.0, 0, 0, 0))
            else:
                mult = float(rng.choice([0.5, 0.8, 2.0]))
                base = float(rng.choice([1.75, 1.5, 2.0]))
                allowed = int(rng.integers(1, 4))
                last_n = int(rng.choice([16, 64, 256]))
                brk = None
                if rng.random() < 0.5:
                    brk = (rng.random(V + 8) < 0.05).astype(np.uint8)
                    d[f"brk{i}"] = brk
                y = ref.dry(x, h, mult, base, allowed, last_n, brk)
                meta.append((1, 0, mult, base, allowed, last_n, int(brk is not None)))
            d[f"x{i}"], d[f"h{i}"], d[f"y{i}"] = x, h, y
            i += 1
    # The restore rule: every finite id banned -> the bans are undone.
    V = 8
    h = np.array([3, 5, 3, 5, 3], np.int32)
    x = np.full(V, -np.inf, np.float32)
    x[5] = 1.5
    d[f"x{i}"], d[f"h{i}"], d[f"y{i}"] = x, h, ref.no_repeat_ngram(x, h, 2)
    meta.append((0, 2, 0.0, 0.0, 0, 0, 0))
    d["meta"] = np.array(meta, dtype=[("kind", "i4"), ("ngram", "i4"), ("mult", "f4"),
                                      ("base", "f4"), ("allowed", "i4"), ("last_n", "i4"),
                                      ("brk", "i4")])
    np.savez_compressed(OUT, **d)
    print(f"{len(meta)} cases -> {OUT}")


if __name__ == "__main__":
    main()
