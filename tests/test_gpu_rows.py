"""GPU parity of the row-stream kernel (row_kinds = TMS_ROWS_TOPK with a row
for every CU: one workgroup a row, the row streamed in passes): every row
equals the oracle, and the general kernel's answer for the same call.  Rows
outside the top-k promise and rows whose candidates overflow the kernel's
buffer (massive ties) are sampled whole by the same workgroup."""
from __future__ import annotations

import numpy as np
import pytest

from tensormark_amd import workloads
from tests.helpers import params_array
from tests.test_gpu_sample import _dev, check

pytestmark = pytest.mark.gpu

B = 300   # at least one row per CU (256 on MI355X) takes the row-stream kernel


def run(sampler, xs, p, *, dtype, recent=None, n_recent=None, mask=None, topk_cap=0, general=False):
    import torch

    from tensormark_amd.sampler import ROWS_ANY, ROWS_TOPK

    if dtype == "bf16":
        x = _dev(xs, torch, torch.bfloat16)
    else:
        x = _dev(xs, torch)
    out = sampler.sample(
        x, p,
        recent=None if recent is None else _dev(recent.astype(np.int32), torch),
        n_recent=None if n_recent is None else _dev(n_recent.astype(np.int32), torch),
        mask=None if mask is None else _dev(mask.astype(np.uint32).view(np.int32), torch),
        topk_cap=topk_cap, row_kinds=ROWS_ANY if general else ROWS_TOPK)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


def rows_case(dtype, seed, V=40000):
    rng = np.random.default_rng(seed)
    x32 = (rng.standard_t(3, (B, V)) * 2.0).astype(np.float32)
    x32[:, ::101] += 3.0
    # massive ties: every entry equal (the candidates overflow the buffer)
    x32[7] = 1.25
    x32[8, ::2] = 1.25
    x32[8, 1::2] = 1.0
    # NaN and +inf rows, an all -inf row
    x32[9, 777] = np.nan
    x32[10, 31] = np.inf
    x32[11] = -np.inf
    if dtype == "f32":
        xs, xw = x32, x32
    elif dtype == "f16":
        xs = x32.astype(np.float16)
        xw = xs.astype(np.float32)
    else:
        xs = workloads.to_bf16_bits(x32)
        xw = workloads.bf16_bits_to_f32(xs)
    bits = rng.random((B, ((V + 31) // 32) * 32)) < 0.85
    bits[:, V:] = False
    bits[9, 777] = bits[10, 31] = True   # the NaN and +inf are allowed
    bits[12] = False            # all masked
    bits[13, :] = False
    bits[13, [5, V // 4, V - 1]] = True   # fewer finite ids than K
    mask = workloads.pack_bits(bits)
    recent = rng.integers(0, V, (B, 512)).astype(np.int32)
    recent[:, ::9] = rng.integers(0, 4096, (B, (512 + 8) // 9))   # window ids in pass 0 too
    recent[:, 1::50] = V + 7    # outside the vocabulary
    recent[:, 2::3] = recent[:, :1]   # repeats
    n_recent = rng.integers(0, 513, B).astype(np.int32)
    p = params_array(B, temperature=1.2, top_k=100, top_p=0.98, seed=np.arange(B) + 4000)
    p["greedy"] = rng.random(B) < 0.4
    p["top_k"] = rng.choice([1, 7, 40, 100, 128], size=B)
    p["top_p"] = rng.choice([0.5, 0.9, 0.98, 1.0], size=B)
    p["min_p"] = rng.choice([0.0, 0.0, 0.05], size=B)
    p["temperature"] = rng.choice([0.3, 1.0, 1.2, 2.5], size=B)
    p["repeat_penalty"] = rng.choice([1.0, 1.05, 1.3], size=B)
    p["repeat_last_n"] = rng.choice([0, 64, 512], size=B)
    p["frequency_penalty"] = rng.choice([0.0, 0.1], size=B)
    p["presence_penalty"] = rng.choice([0.0, 0.2], size=B)
    p["greedy"][[7, 9, 11, 12]] = 0
    p["top_k"][[7, 8]] = [100, 40]
    p["greedy"][[8]] = 1
    # outside the promise: the whole-row path of the same workgroup
    p["greedy"][[14, 15]] = 0
    p["top_k"][[14, 15]] = [0, 500]
    p["temperature"][16] = 0.0   # bad parameters
    p["greedy"][16] = 0
    return xs, xw, p, mask, recent, n_recent


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_rows_kernel_vs_oracle_and_general(sampler, orc, dtype):
    xs, xw, p, mask, recent, n_recent = rows_case(dtype, {"f32": 51, "f16": 52, "bf16": 53}[dtype])
    for cap in (0, 24):
        want = orc.sample_batch(xw, p, recent=recent, n_recent=n_recent, mask=mask, topk_cap=cap)
        g = run(sampler, xs, p, dtype=dtype, recent=recent, n_recent=n_recent, mask=mask, topk_cap=cap)
        assert list(g["status"][9:13]) == [3, 3, 2, 2]
        assert g["status"][16] == 1
        check(g, want, cap)
    h = run(sampler, xs, p, dtype=dtype, recent=recent, n_recent=n_recent, mask=mask, topk_cap=24, general=True)
    for k in ("tokens", "keep", "status", "topk_ids", "topk_probs"):
        assert np.array_equal(g[k], h[k]), k


def test_rows_kernel_no_mask_no_window(sampler, orc):
    """The all-ones mask row and no history: greedy rows keep each thread's
    best entry (no candidates), top-k rows stream with the pass-0 bound."""
    rng = np.random.default_rng(60)
    V = 65536
    x = rng.normal(0.0, 3.0, (B, V)).astype(np.float32)
    p = params_array(B, temperature=0.7, top_k=40, top_p=0.95, seed=np.arange(B) + 1)
    p["greedy"] = rng.random(B) < 0.5
    p["top_k"] = rng.choice([1, 2, 40, 128], size=B)
    want = orc.sample_batch(x, p)
    g = run(sampler, x, p, dtype="f32")
    check(g, want)


@pytest.mark.parametrize("dtype,V", [("f32", 50020), ("f16", 50024), ("bf16", 33032)])
def test_rows_kernel_ragged_vocab(sampler, orc, dtype, V):
    """Vocabularies that end inside a mask word and inside a pass (33032 ids
    of bf16 are five passes of 6144 and part of a sixth): the last pass's
    mask fold and the ids past V."""
    xs, xw, p, mask, recent, n_recent = rows_case(dtype, 70 + V % 97, V=V)
    want = orc.sample_batch(xw, p, recent=recent, n_recent=n_recent, mask=mask, topk_cap=16)
    g = run(sampler, xs, p, dtype=dtype, recent=recent, n_recent=n_recent, mask=mask, topk_cap=16)
    check(g, want, 16)


def test_rows_hint_past_the_window_limit(sampler, orc):
    """A history window wider than the row-stream kernel's 512 positions:
    the call takes the general kernel under the same hint and still equals
    the oracle."""
    rng = np.random.default_rng(81)
    V, W = 20000, 600
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    recent = rng.integers(0, V, (B, W)).astype(np.int32)
    recent[:, ::5] = recent[:, :1]
    n_recent = rng.integers(0, W + 1, B).astype(np.int32)
    p = params_array(B, temperature=0.9, top_k=40, top_p=0.95, seed=np.arange(B) + 5100)
    p["greedy"] = rng.random(B) < 0.3
    p["repeat_penalty"] = 1.2
    p["repeat_last_n"] = W
    p["frequency_penalty"] = 0.1
    want = orc.sample_batch(x, p, recent=recent, n_recent=n_recent, topk_cap=8)
    g = run(sampler, x, p, dtype="f32", recent=recent, n_recent=n_recent, topk_cap=8)
    check(g, want, 8)


@pytest.mark.parametrize("V", [100, 1000, 3076])
def test_rows_kernel_short_rows(sampler, orc, V):
    """Batches too large for the wide kernel's residency with rows shorter
    than one pass (3,072 fp32 ids) or just past it: most threads hold no id,
    and K can exceed the finite ids."""
    rng = np.random.default_rng(V)
    Bs = 600
    x = rng.normal(0.0, 2.0, (Bs, V)).astype(np.float32)
    x[0] = 0.5   # all ties
    bits = rng.random((Bs, ((V + 31) // 32) * 32)) < 0.7
    bits[:, V:] = False
    bits[1] = False
    bits[2, :] = False
    bits[2, [0, V - 1]] = True
    mask = workloads.pack_bits(bits)
    W = 64
    recent = rng.integers(-3, V + 3, (Bs, W)).astype(np.int32)
    p = params_array(Bs, temperature=0.8, top_k=40, top_p=0.9, seed=np.arange(Bs) + 700)
    p["greedy"] = rng.random(Bs) < 0.3
    p["top_k"] = rng.choice([1, 5, 40, 128], size=Bs)
    p["repeat_penalty"] = 1.3
    p["repeat_last_n"] = W
    p["presence_penalty"] = 0.2
    want = orc.sample_batch(x, p, recent=recent, mask=mask, topk_cap=8)
    g = run(sampler, x, p, dtype="f32", recent=recent, mask=mask, topk_cap=8)
    assert g["status"][1] == 2
    check(g, want, 8)
