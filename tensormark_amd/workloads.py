"""Seeded synthetic inputs for the five benchmark shapes of the sampling path.

Each generator returns numpy arrays (host) so the same inputs feed the HIP
library and the CPU checker.  Shapes and distributions:

  cfg1  B=1,    V=32000,  fp32 N(0, 2.5^2) + 5 spikes of +12; T 0.8, k 40, p 0.95;
        repetition 1.1 over a 64-id window.
  cfg2  B=64,   V=128256, fp32 N(0, 3^2) + per-row offset U[-4, 4]; repetition 1.1,
        frequency 0.2, presence 0.1 over 256-id windows; T 0.7, k 40, p 0.95,
        min-p 0.05; optional grammar mask (about 90 % of ids allowed).
  cfg3  B=128,  V=151936, fp16 N(0, 2^2); mask with 0.3 % of ids set in runs of
        1-8 (at least one per row); T 1.0, top-p 0.9, no top-k.
  cfg4  B=32,   k=8, V=32000, fp32 target N(0, 2.5^2) [B, k+1, V]; draft = target
        + N(0, 0.5^2) [B, k, V]; draft tokens drawn from the draft softmax.
  cfg5  B=1024, V=256000, bf16 Student-t (nu 3) * 2; 50 % greedy rows by a
        seeded flag; sampled rows T 1.2, k 100, p 0.98; repetition 1.05 over
        512-id windows.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from .sampler import make_params, Opts


def mask_dense(rng, B, V, p_allowed=0.9):
    """Bits set independently with probability p_allowed; id 0 always set."""
    W = (V + 31) // 32
    bits = rng.random((B, W * 32)) < p_allowed
    bits[:, V:] = False
    bits[:, 0] = True
    return pack_bits(bits)


def mask_runs(rng, B, V, density=0.003, max_run=8):
    """About density * V ids per row, in runs of 1..max_run; >= 1 per row."""
    W = (V + 31) // 32
    bits = np.zeros((B, W * 32), dtype=bool)
    mean_run = (1 + max_run) / 2
    nruns = max(1, int(round(density * V / mean_run)))
    for b in range(B):
        starts = rng.integers(0, V, size=nruns)
        lens = rng.integers(1, max_run + 1, size=nruns)
        for s, l in zip(starts, lens):
            bits[b, s:min(s + l, V)] = True
        if not bits[b, :V].any():
            bits[b, rng.integers(0, V)] = True
    return pack_bits(bits)


def pack_bits(bits: np.ndarray) -> np.ndarray:
    """[B, 32*W] bool -> [B, W] uint32, bit (id & 31) of word id >> 5."""
    B, n = bits.shape
    b = bits.reshape(B, n // 32, 32).astype(np.uint64)
    w = (b << np.arange(32, dtype=np.uint64)).sum(axis=2)
    return w.astype(np.uint32)


def unpack_bits(words: np.ndarray, V: int) -> np.ndarray:
    B, W = words.shape
    sh = np.arange(32, dtype=np.uint32)
    return ((words[:, :, None] >> sh) & 1).reshape(B, W * 32)[:, :V].astype(bool)


def cfg1(seed=1):
    rng = np.random.default_rng(seed)
    V = 32000
    x = rng.normal(0.0, 2.5, size=(1, V)).astype(np.float32)
    x[0, rng.choice(V, 5, replace=False)] += 12.0
    recent = rng.integers(0, V, size=(1, 64)).astype(np.int32)
    params = make_params(1, Opts(0.8, 40, 0.95), repeat_penalty=1.1, repeat_last_n=64,
                         seed=seed)
    return dict(logits=x, recent=recent, params=params, mask=None)


def cfg2(seed=2, B=64, V=128256, with_mask=False):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
    x += rng.uniform(-4, 4, size=(B, 1)).astype(np.float32)
    recent = rng.integers(0, V, size=(B, 256)).astype(np.int32)
    params = make_params(B, Opts(0.7, 40, 0.95), min_p=0.05, repeat_penalty=1.1,
                         repeat_last_n=256, frequency_penalty=0.2, presence_penalty=0.1,
                         seed=np.arange(B, dtype=np.uint64) + 1000 * seed)
    mask = mask_dense(rng, B, V) if with_mask else None
    return dict(logits=x, recent=recent, params=params, mask=mask)


def cfg3(seed=3, B=128, V=151936):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 2.0, size=(B, V)).astype(np.float16)
    mask = mask_runs(rng, B, V)
    params = make_params(B, Opts(1.0, 0, 0.9), seed=np.arange(B, dtype=np.uint64) + 7)
    return dict(logits=x, recent=None, params=params, mask=mask)


def _blocks(n, size):
    return [(i, min(i + size, n)) for i in range(0, n, size)]


def _pool():
    return ThreadPoolExecutor(max_workers=max(1, min(16, os.cpu_count() or 1)))


def cfg5(seed=5, B=1024, V=256000):
    """Student-t (nu 3) * 2 as z / sqrt(g / 1.5), z ~ N(0, 1), g ~ Gamma(1.5)
    (chi-square with 3 degrees is 2 * Gamma(1.5)), drawn in float32 per block
    of 64 rows from the block's own child seed on a thread pool: the values
    depend on the seed and the block, not on the number of threads."""
    ss = np.random.SeedSequence(seed)
    main, blocks = ss.spawn(2)
    rng = np.random.default_rng(main)
    spans = _blocks(B, 64)
    seeds = blocks.spawn(len(spans))
    x = np.empty((B, V), np.float32)

    def fill(i):
        lo, hi = spans[i]
        r = np.random.default_rng(seeds[i])
        z = r.standard_normal((hi - lo, V), dtype=np.float32)
        g = r.standard_gamma(1.5, (hi - lo, V), dtype=np.float32)
        g /= np.float32(1.5)
        np.sqrt(g, out=g)
        z /= g
        z *= np.float32(2.0)
        x[lo:hi] = z

    with _pool() as ex:
        list(ex.map(fill, range(len(spans))))
    recent = rng.integers(0, V, size=(B, 512)).astype(np.int32)
    greedy = rng.random(B) < 0.5
    params = make_params(B, Opts(1.2, 100, 0.98), repeat_penalty=1.05, repeat_last_n=512,
                         greedy=greedy, seed=np.arange(B, dtype=np.uint64) + 55)
    return dict(logits=x, recent=recent, params=params, mask=None)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) as uint16 bits; a NaN stays a NaN
    (quiet bit set).  32-bit arithmetic, 64 rows a block on a thread pool."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    out = np.empty(u.shape, np.uint16)
    flat_u = u.reshape(-1, u.shape[-1]) if u.ndim > 1 else u.reshape(1, -1)
    flat_o = out.reshape(flat_u.shape)

    def conv(span):
        lo, hi = span
        w = flat_u[lo:hi]
        r = w + np.uint32(0x7FFF)      # no wrap: only NaN patterns exceed 0xFFFF8000
        r += (w >> 16) & np.uint32(1)
        r >>= 16
        nan = (w & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
        r[nan] = (w[nan] >> 16) | np.uint32(0x40)
        flat_o[lo:hi] = r.astype(np.uint16)

    with _pool() as ex:
        list(ex.map(conv, _blocks(flat_u.shape[0], 64)))
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def softmax_draws(rng, logits: np.ndarray) -> np.ndarray:
    """One draw per row from softmax(logits) (float64), for draft tokens."""
    z = logits.astype(np.float64)
    z = z - z.max(axis=-1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=-1, keepdims=True)
    c = p.cumsum(axis=-1)
    u = rng.random(c.shape[:-1] + (1,))
    return np.minimum((c < u).sum(axis=-1), logits.shape[-1] - 1).astype(np.int32)


def cfg4(seed=4, B=32, k=8, V=32000):
    rng = np.random.default_rng(seed)
    target = rng.normal(0.0, 2.5, size=(B, k + 1, V)).astype(np.float32)
    draft = (target[:, :k, :] + rng.normal(0.0, 0.5, size=(B, k, V))).astype(np.float32)
    tokens = softmax_draws(rng, draft)
    params = make_params(B, Opts(1.0, 0, 1.0), seed=np.arange(B, dtype=np.uint64) + 99)
    return dict(target=target, draft=draft, tokens=tokens, params=params)
