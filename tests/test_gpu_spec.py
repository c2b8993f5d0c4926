"""GPU parity of the speculative verify (tms_spec_verify, through the C ABI)
against the CPU oracle's tmo_spec_verify_seq: accepted counts, tokens and
statuses bit-exact.  The stochastic rule has no reference counterpart; its
greedy limit is spec_generate_greedy's argmax match (llama.h:5127-5131)."""
from __future__ import annotations

import numpy as np
import pytest

from tensormark_amd import workloads
from tests.helpers import params_array

pytestmark = pytest.mark.gpu


def _dev(a, torch, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to("cuda:0")


def run_spec(sampler, target, draft, tokens, params, draws=None, dtype="f32"):
    import torch

    if dtype == "f32":
        tg, dr = _dev(target.astype(np.float32), torch), _dev(draft.astype(np.float32), torch)
    elif dtype == "f16":
        tg, dr = _dev(target.astype(np.float16), torch), _dev(draft.astype(np.float16), torch)
    else:
        tg = _dev(workloads.to_bf16_bits(target), torch, torch.bfloat16)
        dr = _dev(workloads.to_bf16_bits(draft), torch, torch.bfloat16)
    out = sampler.spec_verify(
        tg, dr, _dev(tokens.astype(np.int32), torch), params,
        draws=None if draws is None else _dev(draws.astype(np.uint32).view(np.int32), torch))
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


def widen(x, dtype):
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return workloads.bf16_bits_to_f32(workloads.to_bf16_bits(x))
    return x.astype(np.float32)


def philox_words(orc, params, k):
    B = len(params)
    w = np.zeros((B, k + 1, 2), np.uint32)
    for b in range(B):
        for i in range(k + 1):
            w[b, i] = orc.row_words(int(params["seed"][b]), int(params["offset"][b]), i)
    return w


def check_spec(orc, gpu, target, draft, tokens, params, words, dtype="f32"):
    tg, dr = widen(target, dtype), widen(draft, dtype)
    for b in range(len(params)):
        st, acc, tok = orc.spec_verify_seq(tg[b], dr[b], tokens[b],
                                           float(params["temperature"][b]), words[b])
        got = (int(gpu["status"][b]), int(gpu["accepted"][b]), int(gpu["token"][b]))
        assert got == (st, acc, tok), (b, got, (st, acc, tok))


def test_spec_cfg4_full_size(orc, sampler):
    c = workloads.cfg4()
    gpu = run_spec(sampler, c["target"], c["draft"], c["tokens"], c["params"])
    words = philox_words(orc, c["params"], c["draft"].shape[1])
    check_spec(orc, gpu, c["target"], c["draft"], c["tokens"], c["params"], words)
    acc = gpu["accepted"]
    assert (gpu["status"] == 0).all()
    # The draft is the target plus noise: most drafts pass, not all.
    assert 0 < acc.mean() < 8


def test_spec_caller_draws_and_dtypes(orc, sampler):
    rng = np.random.default_rng(41)
    # 16-byte aligned rows (V a multiple of 4 for f32, 8 for f16/bf16) take the
    # chunked statistics (4096 ids a chunk, the last one ragged); the others
    # the per-row kernel.
    for dtype, V, k in [("f32", 1000, 3), ("f16", 4096, 5), ("bf16", 777, 16), ("f32", 5, 1),
                        ("f32", 50000, 2), ("bf16", 10000, 4), ("f16", 12296, 3)]:
        B = 6
        target = rng.normal(0, 2.0, size=(B, k + 1, V)).astype(np.float32)
        draft = (target[:, :k] + rng.normal(0, 1.0, size=(B, k, V))).astype(np.float32)
        tokens = workloads.softmax_draws(rng, draft)
        params = params_array(B, temperature=0.8)
        words = rng.integers(0, 2**32, size=(B, k + 1, 2), dtype=np.uint64).astype(np.uint32)
        gpu = run_spec(sampler, target, draft, tokens, params, draws=words, dtype=dtype)
        check_spec(orc, gpu, target, draft, tokens, params, words, dtype)


def test_spec_greedy_limit(orc, sampler):
    """One-hot target and draft: accept iff the draft token is the target argmax;
    the emitted token is the target argmax (llama.h:5127-5131)."""
    rng = np.random.default_rng(42)
    B, k, V = 16, 4, 300
    target = np.full((B, k + 1, V), -np.inf, np.float32)
    draft = np.full((B, k, V), -np.inf, np.float32)
    am = rng.integers(0, V, size=(B, k + 1))
    da = np.where(rng.random((B, k)) < 0.7, am[:, :k], rng.integers(0, V, size=(B, k)))
    for b in range(B):
        for i in range(k + 1):
            target[b, i, am[b, i]] = 1.0
        for i in range(k):
            draft[b, i, da[b, i]] = 1.0
    params = params_array(B, temperature=1.0)
    gpu = run_spec(sampler, target, draft, da.astype(np.int32), params)
    for b in range(B):
        j = 0
        while j < k and da[b, j] == am[b, j]:
            j += 1
        assert gpu["status"][b] == 0
        assert gpu["accepted"][b] == j
        assert gpu["token"][b] == am[b, j]


def test_spec_equal_distributions_accept_all(orc, sampler):
    rng = np.random.default_rng(43)
    B, k, V = 8, 6, 2000
    target = rng.normal(0, 2.0, size=(B, k + 1, V)).astype(np.float32)
    draft = target[:, :k].copy()
    tokens = workloads.softmax_draws(rng, draft)
    params = params_array(B, temperature=0.9, seed=np.arange(B, dtype=np.uint64) + 5)
    gpu = run_spec(sampler, target, draft, tokens, params)
    assert (gpu["accepted"] == k).all()
    words = philox_words(orc, params, k)
    check_spec(orc, gpu, target, draft, tokens, params, words)


def test_spec_error_rows(orc, sampler):
    rng = np.random.default_rng(44)
    B, k, V = 6, 3, 640
    target = rng.normal(0, 1.0, size=(B, k + 1, V)).astype(np.float32)
    draft = target[:, :k].copy()   # equal: every draft is accepted
    tokens = workloads.softmax_draws(rng, draft)
    params = params_array(B, temperature=1.0)
    params["temperature"][0] = 0.0              # bad temperature
    target[1, 2, 17] = np.nan                   # NaN in a row the tests reach
    draft[2, 0, :] = -np.inf                    # all-masked draft row
    tokens[3, 1] = V + 3                        # draft token out of range
    target[4, k, 5] = np.inf                    # +inf in the bonus row
    gpu = run_spec(sampler, target, draft, tokens, params)
    words = philox_words(orc, params, k)
    check_spec(orc, gpu, target, draft, tokens, params, words)
    assert list(gpu["status"]) == [1, 3, 2, 1, 3, 0]
    assert (gpu["token"][:5] == -1).all()


def test_spec_repeated_calls(orc, sampler):
    """Tickets and published sums return to zero: back-to-back calls agree."""
    c = workloads.cfg4(seed=9, B=8, k=4, V=32000)
    a = run_spec(sampler, c["target"], c["draft"], c["tokens"], c["params"])
    b = run_spec(sampler, c["target"], c["draft"], c["tokens"], c["params"])
    for key in a:
        assert np.array_equal(a[key], b[key]), key
    words = philox_words(orc, c["params"], 4)
    check_spec(orc, a, c["target"], c["draft"], c["tokens"], c["params"], words)


def test_spec_back_to_back_different_batches(orc, sampler):
    """Full-size calls on different batches, back to back: each call's chunk
    statistics are written by workgroups on all XCDs and read by the next
    kernel, so a stale record from the previous call would change an accept
    count or a token."""
    for seed in (21, 22, 23):
        c = workloads.cfg4(seed=seed)
        gpu = run_spec(sampler, c["target"], c["draft"], c["tokens"], c["params"])
        words = philox_words(orc, c["params"], c["draft"].shape[1])
        check_spec(orc, gpu, c["target"], c["draft"], c["tokens"], c["params"], words)


@pytest.mark.parametrize("B,V", [(24, 140000), (4, 262144)])
def test_spec_resolve_ticket_form(orc, sampler, B, V):
    """Resolve grids that are not resident at once (24 sequences x 64 parts)
    and part runs past 16 ids a thread (V = 262144: 4,096 ids a part) take
    the ticket form, whose last arriver recomputes the threshold's part;
    config 4 itself takes the waiting form.  Rows this long also take the
    two-pass statistics kernel."""
    rng = np.random.default_rng(B)
    k = 2
    target = rng.normal(0.0, 2.0, (B, k + 1, V)).astype(np.float32)
    draft = (target[:, :k] + rng.normal(0.0, 0.5, (B, k, V))).astype(np.float32)
    tokens = workloads.softmax_draws(rng, draft)
    params = params_array(B, temperature=1.0, top_k=0, top_p=1.0, seed=np.arange(B) + 3)
    params["temperature"] = rng.choice([0.8, 1.0], size=B)
    gpu = run_spec(sampler, target, draft, tokens, params)
    words = philox_words(orc, params, k)
    check_spec(orc, gpu, target, draft, tokens, params, words)
    assert (gpu["status"] == 0).all()


def test_spec_bonus_row_statistics_in_the_resolve(orc, sampler):
    """The resolve forms the bonus row's statistics itself (every part's
    maximum exchanged between the sequence's workgroups; V = 6000: three
    parts): an all-masked bonus row after every draft is accepted, a NaN
    in a bonus row that a rejection leaves unused, a NaN in the last part of
    an accepted sequence's bonus row, and plain accepted sequences."""
    rng = np.random.default_rng(47)
    B, k, V = 6, 3, 6000
    target = rng.normal(0, 1.5, size=(B, k + 1, V)).astype(np.float32)
    draft = target[:, :k].copy()                 # equal: every draft is accepted
    draft[1] = (draft[1] + rng.normal(0, 4.0, size=(k, V))).astype(np.float32)
    tokens = workloads.softmax_draws(rng, draft)
    params = params_array(B, temperature=1.0, seed=np.arange(B, dtype=np.uint64) + 9)
    params["temperature"][3] = 0.7
    target[0, k, :] = -np.inf                    # all-masked bonus row
    target[1, k, 100] = np.nan                   # unused when a draft is rejected
    target[2, k, V - 7] = np.nan                 # last part of the bonus row
    gpu = run_spec(sampler, target, draft, tokens, params)
    words = philox_words(orc, params, k)
    check_spec(orc, gpu, target, draft, tokens, params, words)
    assert gpu["status"][0] == 2 and gpu["status"][2] == 3
    assert (gpu["status"][3:] == 0).all() and (gpu["accepted"][3:] == k).all()
