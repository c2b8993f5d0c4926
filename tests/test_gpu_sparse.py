"""GPU parity of the sparse-mask kernel (row_kinds = TMS_ROWS_SPARSE_MASK):
only the allowed logits are read, so every answer must equal the oracle's
over the whole row, and the general kernel's for the same call.  Rows with
more allowed ids than the kernel holds (2048), top-p rows past the list
capacity and draws past the held entries are sampled whole by the same
workgroup; they are covered here too."""
from __future__ import annotations

import zlib

import numpy as np
import pytest

from tensormark_amd import workloads
from tests.helpers import params_array
from tests.test_gpu_sample import EDGE, _dev, _edge_case, check

pytestmark = pytest.mark.gpu


def run(sampler, logits, params, *, mask, recent=None, n_recent=None, topk_cap=0, dtype="f32",
        sparse=True):
    import torch

    from tensormark_amd.sampler import ROWS_ANY, ROWS_SPARSE_MASK

    if dtype == "f32":
        x = _dev(logits.astype(np.float32), torch)
    elif dtype == "f16":
        x = _dev(logits.astype(np.float16), torch)
    else:
        x = _dev(logits, torch, torch.bfloat16)   # uint16 bf16 bits
    out = sampler.sample(
        x, params,
        recent=None if recent is None else _dev(recent.astype(np.int32), torch),
        n_recent=None if n_recent is None else _dev(n_recent.astype(np.int32), torch),
        mask=_dev(mask.astype(np.uint32).view(np.int32), torch),
        topk_cap=topk_cap, row_kinds=ROWS_SPARSE_MASK if sparse else ROWS_ANY)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


def sparse_mask(rng, B, V, counts, runs=True):
    """Row b allows about counts[b] ids (in runs of 1..8 when `runs`)."""
    bits = np.zeros((B, ((V + 31) // 32) * 32), bool)
    for b in range(B):
        c = int(counts[b])
        if runs:
            while bits[b, :V].sum() < c:
                s = int(rng.integers(0, V))
                bits[b, s:min(s + int(rng.integers(1, 9)), V)] = True
        else:
            bits[b, rng.choice(V, size=c, replace=False)] = True
    return workloads.pack_bits(bits)


@pytest.mark.parametrize("cap", [64, 0])
def test_cfg3_full_size_sparse_vs_oracle(sampler, orc, cap):
    """Config 3 (B = 128, V = 151936 fp16, 0.3% allowed, top-p 0.9) through
    the sparse-mask kernel: every row equals the oracle; cap 64 asks for the
    per-entry probabilities (the sequential top-p tail)."""
    w = workloads.cfg3()
    want = orc.sample_batch(w["logits"].astype(np.float32), w["params"], mask=w["mask"], topk_cap=cap)
    g = run(sampler, w["logits"], w["params"], mask=w["mask"], topk_cap=cap, dtype="f16")
    assert (g["status"] == 0).all()
    check(g, want, cap)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_sparse_rows_vs_oracle(sampler, orc, dtype):
    """Greedy, top-k (1, 40, 128, 200), top-p and min-p rows over sparse
    masks, with history penalties (repeats, masked and out-of-range ids in
    the window), fewer finite ids than K, an allowed -inf logit, a NaN that
    the mask hides, and rows at and past the kernel's 2048 allowed ids."""
    rng = np.random.default_rng({"f32": 1, "f16": 2, "bf16": 3}[dtype])
    B, V = 16, 50000
    x32 = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    counts = [300, 40, 10, 3, 500, 800, 150, 60, 2047, 2048, 2049, 5000, 200, 100, 30, 1]
    mask = sparse_mask(rng, B, V, counts, runs=True)
    bits = np.unpackbits(mask.view(np.uint8), bitorder="little").reshape(B, -1)[:, :V].astype(bool)
    # a NaN the mask hides, an allowed -inf
    hid = np.flatnonzero(~bits[0])[5]
    x32[0, hid] = np.nan
    ok = np.flatnonzero(bits[1])
    x32[1, ok[0]] = -np.inf
    if dtype == "f32":
        xs, xw = x32, x32
    elif dtype == "f16":
        xs = x32.astype(np.float16)
        xw = xs.astype(np.float32)
    else:
        xs = workloads.to_bf16_bits(x32)
        xw = workloads.bf16_bits_to_f32(xs)
    recent = np.empty((B, 400), np.int32)
    for b in range(B):
        allowed = np.flatnonzero(bits[b])
        recent[b] = rng.choice(allowed, 400) if b % 3 else rng.integers(-5, V + 5, 400)
    recent[:, ::7] = recent[:, :1]   # repeats
    p = params_array(B, temperature=0.8, top_k=40, top_p=0.95, seed=np.arange(B) + 900)
    p["greedy"][[2, 9]] = 1
    p["top_k"] = [0, 40, 40, 40, 128, 1, 200, 0, 40, 0, 40, 0, 128, 0, 100, 40]
    p["top_p"][[7, 13]] = [0.3, 1.0]
    p["min_p"][[4, 12]] = [0.05, 0.2]
    p["temperature"][[5, 6]] = [1.7, 0.5]
    p["repeat_penalty"] = 1.2
    p["repeat_last_n"] = rng.choice([0, 64, 400], size=B)
    p["frequency_penalty"][::2] = 0.1
    p["presence_penalty"][1::2] = 0.2
    for cap in (24, 0):
        want = orc.sample_batch(xw, p, recent=recent, mask=mask, topk_cap=cap)
        g = run(sampler, xs, p, mask=mask, recent=recent, topk_cap=cap, dtype=dtype)
        check(g, want, cap)


def test_sparse_equals_general_kernel(sampler, orc):
    """The same call through both kernels: bit-identical tokens, keep
    counts, statuses, id lists and probabilities."""
    rng = np.random.default_rng(11)
    B, V = 64, 128256
    x = rng.normal(0.0, 3.0, (B, V)).astype(np.float32)
    mask = sparse_mask(rng, B, V, rng.integers(1, 1500, B), runs=False)
    recent = rng.integers(0, V, (B, 256)).astype(np.int32)
    p = params_array(B, temperature=0.7, top_k=40, top_p=0.95, seed=np.arange(B) + 77)
    p["top_k"] = rng.choice([0, 1, 40, 128, 500], size=B)
    p["greedy"] = rng.random(B) < 0.2
    p["min_p"] = rng.choice([0.0, 0.05], size=B)
    p["repeat_penalty"] = 1.1
    p["repeat_last_n"] = 256
    p["frequency_penalty"] = 0.2
    p["presence_penalty"] = 0.1
    a = run(sampler, x, p, mask=mask, recent=recent, topk_cap=16)
    b = run(sampler, x, p, mask=mask, recent=recent, topk_cap=16, sparse=False)
    for k in ("tokens", "keep", "status", "topk_ids", "topk_probs"):
        assert np.array_equal(a[k], b[k]), k
    want = orc.sample_batch(x, p, recent=recent, mask=mask, topk_cap=16)
    check(a, want, 16)


@pytest.mark.parametrize("name", list(EDGE))
def test_sparse_edge_cases(sampler, orc, name):
    """The general kernel's edge cases through the sparse-mask kernel; a row
    without a mask gets an all-ones one (20000 allowed ids: the whole-row
    path of the same workgroup)."""
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x, p, recent, mask = _edge_case(name, rng)
    V = x.shape[1]
    if mask is None:
        mask = workloads.pack_bits(np.pad(np.ones(x.shape, bool), ((0, 0), (0, (-V) % 32))))
    for cap in (40, 0):
        want = orc.sample_batch(x, p, recent=recent, mask=mask, topk_cap=cap)
        g = run(sampler, x, p, mask=mask, recent=recent, topk_cap=cap)
        check(g, want, cap)


def test_sparse_hint_past_the_vocabulary_limit(orc):
    """A vocabulary wider than the sparse-mask kernel's 262,144 ids: the
    call takes the general kernel under the same hint and still equals the
    oracle."""
    from tensormark_amd import Sampler

    rng = np.random.default_rng(91)
    B, V = 4, 262144 + 96
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    mask = sparse_mask(rng, B, V, [50, 400, 7, 1000], runs=True)
    bits = np.unpackbits(mask.view(np.uint8), bitorder="little").reshape(B, -1)
    bits[:, V - 20:V] = True   # allowed ids past the kernel's limit
    mask = workloads.pack_bits(bits)
    p = params_array(B, temperature=1.0, top_k=0, top_p=0.9, seed=np.arange(B) + 31)
    p["top_k"][1] = 40
    s = Sampler(max_batch=B, max_vocab=V)
    try:
        want = orc.sample_batch(x, p, mask=mask, topk_cap=16)
        g = run(s, x, p, mask=mask, topk_cap=16)
        check(g, want, 16)
    finally:
        s.close()
