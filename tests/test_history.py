"""The host history transforms of the C ABI (tms_host_*) against the
reference's compiled tmsample.h, through committed golden vectors
(tests/golden/history_golden.npz, written by make_history_golden.py), plus
closed-form checks.  CPU only: these are host functions."""
from __future__ import annotations

import os

import numpy as np
import pytest

from tensormark_amd import sampler
from tensormark_amd.sampler import make_history

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


# ---- the oracle's restatement (the GPU tests' checker) against the same
#      reference outputs, and the DRY scale the device and host compute.

def test_oracle_history_matches_reference_golden(hist_golden, orc):
    g = hist_golden
    for i, m in enumerate(g["meta"]):
        x, h, want = g[f"x{i}"], g[f"h{i}"], g[f"y{i}"]
        if m["kind"] == 0:
            got = orc.no_repeat_ngram(x, h, int(m["ngram"]))
        else:
            brk = g[f"brk{i}"] if m["brk"] else None
            got = orc.dry(x, h, float(m["mult"]), float(m["base"]), int(m["allowed"]),
                          int(m["last_n"]), brk)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i


def _histories(rng, n_cases):
    """Histories that repeat: a short alphabet, periodic stretches, breakers."""
    for c in range(n_cases):
        n = int(rng.integers(2, 300))
        alpha = int(rng.integers(2, 12))
        if c % 3 == 0:
            period = int(rng.integers(1, 6))
            base = rng.integers(0, alpha, period)
            h = np.resize(base, n)
            flips = rng.random(n) < 0.05
            h = np.where(flips, rng.integers(0, alpha, n), h)
        else:
            h = rng.integers(0, alpha, n)
        if c % 7 == 0:
            h[rng.integers(0, n)] = -3          # out-of-range ids are skipped
        yield c, h.astype(np.int32)


def test_oracle_ngram_matches_compiled_reference(orc, ref):
    rng = np.random.default_rng(5)
    for c, h in _histories(rng, 300):
        V = 16
        x = rng.normal(0, 2, V).astype(np.float32)
        if c % 5 == 0:
            x[rng.random(V) < 0.8] = -np.inf      # few left: the restore rule
        ng = int(rng.integers(2, 6))
        assert np.array_equal(orc.no_repeat_ngram(x, h, ng).view(np.uint32),
                              ref.no_repeat_ngram(x, h, ng).view(np.uint32)), c


def test_oracle_dry_matches_compiled_reference(orc, ref):
    rng = np.random.default_rng(6)
    for c, h in _histories(rng, 300):
        V = 16
        x = rng.normal(0, 2, V).astype(np.float32)
        brk = (rng.random(V) < 0.2).astype(np.uint8) if c % 2 else None
        args = (float(rng.choice([0.5, 0.8, 2.0])), float(rng.choice([1.75, 1.5, 2.0, 1.1])),
                int(rng.integers(1, 4)), int(rng.choice([8, 64, 256])))
        got = orc.dry(x, h, *args, brk)
        want = ref.dry(x, h, *args, brk)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), c


def _scale_by_host(base, k, allowed=2):
    """base^k as tms_host_dry computes it: a history whose only DRY match has
    L = k + allowed, multiplier 1, on a zero row -> row[y] = -scale."""
    L = k + allowed
    t = np.arange(10, 10 + L, dtype=np.int32)
    h = np.concatenate([[1], t, [2], t]).astype(np.int32)   # ... x t y t: one match, y follows
    row = np.zeros(10 + L, np.float32)
    sampler.apply_dry(row, h, 1.0, base, allowed, 10 * L + 10)
    hit = np.nonzero(row)[0]
    assert hit.tolist() == [2], hit
    return -row[2]


def _scale_by_reference(ref, base, k, allowed=2):
    """The same history through the compiled reference's apply_dry."""
    L = k + allowed
    t = np.arange(10, 10 + L, dtype=np.int32)
    h = np.concatenate([[1], t, [2], t]).astype(np.int32)
    row = ref.dry(np.zeros(10 + L, np.float32), h, 1.0, base, allowed, 10 * L + 10)
    return -row[2]


def _round_f32(q):
    """A positive Fraction rounded to the nearest float32 (ties to even)."""
    from fractions import Fraction

    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    m = q / ulp
    lo = m.numerator // m.denominator
    r = m - lo
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and lo % 2):
        lo += 1
    return np.float32(float(lo * ulp)) if lo * ulp < Fraction(2) ** 128 else np.float32(np.inf)


def test_correctly_rounded_power_differs_from_glibc_powf_where_expected():
    """The pairs below are where glibc's powf (the reference's std::pow,
    tmsample.h:168) is one ulp off the correctly rounded base^k (exact
    rationals), and every other pair sampled agrees: the device pre-pass's
    own power (tms_history.h, used when a call brings no table) is the
    correctly rounded one, so these are the pairs the table exists for
    (the GPU side: test_gpu_history.py)."""
    from fractions import Fraction

    differ = []
    for b in (1.75, 1.5, 1.25, 2.0, 1.1):
        t = sampler.dry_scale_table(make_history(1, dry_multiplier=1.0, dry_base=b,
                                                 dry_penalty_last_n=300))[0]
        bf = Fraction(float(np.float32(b)))
        for k in range(300):
            if t[k] != _round_f32(bf ** k):
                differ.append((b, k))
    assert differ == [(1.75, 83), (1.1, 56), (1.1, 294)], differ


def test_dry_scale_table_and_host_dry_are_the_reference_powf(ref):
    """tms_dry_scale_table and tms_host_dry give the compiled reference's
    apply_dry scale bit for bit (oracle/_ref), at the pairs where glibc's
    powf is not correctly rounded and around them."""
    for b, ks in ((1.75, range(78, 90)), (1.1, list(range(50, 62)) + [294]), (1.5, range(0, 12))):
        t = sampler.dry_scale_table(make_history(1, dry_multiplier=1.0, dry_base=b,
                                                 dry_penalty_last_n=300))[0]
        for k in ks:
            want = _scale_by_reference(ref, np.float32(b), k)
            assert t[k] == want, (b, k)
            assert _scale_by_host(np.float32(b), k) == want, (b, k)
