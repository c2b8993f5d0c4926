"""The host history transforms of the C ABI (tms_host_*) against the
reference's compiled tmsample.h, through committed golden vectors
(tests/golden/history_golden.npz, written by make_history_golden.py), plus
closed-form checks.  CPU only: these are host functions."""
from __future__ import annotations

import os

import numpy as np
import pytest

from tensormark_amd import sampler

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "history_golden.npz")


@pytest.fixture(scope="module")
def hist_golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_history_transforms_match_reference_golden(hist_golden):
    g = hist_golden
    changed = 0
    for i, m in enumerate(g["meta"]):
        x, h, want = g[f"x{i}"].copy(), g[f"h{i}"], g[f"y{i}"]
        row = x.copy()
        if m["kind"] == 0:
            sampler.apply_no_repeat_ngram(row, h, int(m["ngram"]))
        else:
            brk = g[f"brk{i}"] if m["brk"] else None
            sampler.apply_dry(row, h, float(m["mult"]), float(m["base"]), int(m["allowed"]),
                              int(m["last_n"]), brk)
        assert np.array_equal(row.view(np.uint32), want.view(np.uint32)), i
        changed += int(not np.array_equal(x, want))
    # The histories repeat by construction: most cases move some logit.
    assert changed >= len(g["meta"]) // 2


def test_ngram_ban_closed_form():
    # history a b a: context (a) was followed by b before -> b is banned
    row = np.arange(6, dtype=np.float32)
    sampler.apply_no_repeat_ngram(row, np.array([2, 4, 2], np.int32), 2)
    assert row[4] == -np.inf and np.isfinite(np.delete(row, 4)).all()
    # too short a history: no-op
    row = np.ones(6, np.float32)
    sampler.apply_no_repeat_ngram(row, np.array([1, 2], np.int32), 3)
    assert (row == 1).all()


def test_dry_closed_form():
    # history x y x y x: the tail (x) agrees with positions 0 and 2 for L=1, and
    # with position 2 for L=3 (x y x); allowed_length 1 -> penalties on y
    # (what followed): mult * base^(1-1) from i=0 and mult * base^(3-1) from i=2.
    x_id, y_id = 1, 3
    h = np.array([x_id, y_id, x_id, y_id, x_id], np.int32)
    row = np.zeros(5, np.float32)
    sampler.apply_dry(row, h, 0.5, 2.0, 1, 256)
    want = np.float32(0) - np.float32(0.5) * np.float32(1.0) - np.float32(0.5) * np.float32(4.0)
    assert row[y_id] == want
    assert (np.delete(row, y_id) == 0).all()


def test_repeat_penalty_host_closed_form():
    row = np.array([2.0, -2.0, 3.0], np.float32)
    sampler.apply_repeat_penalty(row, np.array([0, 1, 0, 7], np.int32), 64, 2.0)
    assert row.tolist() == [0.5, -4.0, 3.0]
