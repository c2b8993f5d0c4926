"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle and
the golden vectors of the compiled reference.  Token ids, keep counts and
top-k id lists must be bit-exact; top-k probabilities within 1e-6 relative."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tensormark_amd import workloads
from tests.helpers import golden_cases, params_array

pytestmark = pytest.mark.gpu


def _dev(a, torch, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to("cuda:0")


def run_gpu(sampler, logits, params, recent=None, n_recent=None, mask=None, draws=None,
            topk_cap=0, dtype="f32"):
    import torch

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
        mask=None if mask is None else _dev(mask.astype(np.uint32).view(np.int32), torch),
        draws=None if draws is None else _dev(draws.astype(np.uint32).view(np.int32), torch),
        topk_cap=topk_cap)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


def check(gpu, want, topk_cap=0, rows=None):
    rows = np.arange(len(want["tokens"])) if rows is None else rows
    for b in rows:
        assert gpu["status"][b] == want["status"][b], (b, gpu["status"][b], want["status"][b])
        assert gpu["tokens"][b] == want["tokens"][b], (b, gpu["tokens"][b], want["tokens"][b])
        assert gpu["keep"][b] == want["keep"][b], (b, gpu["keep"][b], want["keep"][b])
        if topk_cap:
            gi, wi = gpu["topk_ids"][b], want["topk_ids"][b]
            assert np.array_equal(gi, wi), (b, gi[:8], wi[:8])
            gp, wp = gpu["topk_probs"][b], want["topk_probs"][b]
            assert np.allclose(gp, wp, rtol=1e-6, atol=0), b


def test_philox_device_matches_oracle(orc):
    import torch

    from tensormark_amd.sampler import debug_philox

    rng = np.random.default_rng(0)
    ins = [list(c) + list(k) for c, k, _ in [((0, 0, 0, 0), (0, 0), 0),
                                               ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, 0)]]
    ins += [list(int(v) for v in rng.integers(0, 2**32, 6)) for _ in range(4096)]
    a = np.array(ins, np.uint32)
    out = debug_philox(_dev(a.view(np.int32), torch)).cpu().numpy().view(np.uint32)
    for i in range(len(a)):
        assert list(out[i]) == orc.philox(a[i, :4], a[i, 4:]), i


def test_exp64_device_bitwise_equals_oracle(orc):
    import torch

    from tensormark_amd.sampler import debug_exp

    rng = np.random.default_rng(1)
    xs = np.concatenate([-rng.random(50000) * 60, -rng.random(5000) * 745, [0.0, -746.5]])
    y = debug_exp(torch.from_numpy(xs).to("cuda:0"), 1).cpu().numpy()
    want = np.array([orc.exp64(float(v)) for v in xs])
    assert np.array_equal(y.view(np.uint64), want.view(np.uint64))


def test_reciprocal_division_is_correctly_rounded():
    """The verify residual divides by a row's Z through its reciprocal and
    two fma corrections; the quotients equal IEEE division (numpy's a / b)
    bit for bit: the residual's operands (whole numbers up to 2^44 over Z in
    [2^44, 2^61)), divisors next to powers of two, and general doubles."""
    import torch

    from tensormark_amd.sampler import debug_exp

    rng = np.random.default_rng(5)
    n = 1 << 20
    a = np.floor(rng.random(n) * 2.0 ** rng.integers(0, 45, n))
    b = np.floor(2.0 ** rng.uniform(44, 61, n))
    near = rng.random(n) < 0.25
    b[near] = 2.0 ** rng.integers(45, 61, int(near.sum())) - rng.integers(1, 1000, int(near.sum())) * 2.0 ** 8
    g = rng.random(n) < 0.25
    a[g] = np.exp(rng.uniform(-300, 300, int(g.sum())))
    b[g] = np.exp(rng.uniform(-300, 300, int(g.sum())))
    x = np.empty(2 * n)
    x[0::2], x[1::2] = a, b
    y = debug_exp(torch.from_numpy(x).to("cuda:0"), 3).cpu().numpy()[:n]
    assert np.array_equal(y, a / b)


def test_q44_weight_fast_path_bitwise_equals_oracle(orc):
    """The verify weight q44(exp64(x)) for x <= 0 through the device's folded
    form equals the oracle's two-step form bit for bit, including the -40
    cut-off, where the weight reaches 0, and the grid's rounding midpoints."""
    import torch

    from tensormark_amd.sampler import debug_exp

    rng = np.random.default_rng(2)
    xs = np.concatenate([-rng.random(100000) * 45, -rng.random(2000) * 800, -rng.random(2000) * 1e-6,
                         [0.0, -0.0, -40.0, np.nextafter(-40.0, 0), np.nextafter(-40.0, -50), -31.0,
                          -30.49, -745.0, -np.inf]])
    y = debug_exp(torch.from_numpy(xs).to("cuda:0"), 2).cpu().numpy()
    want = np.array([float(orc.lib.tmo_q44(orc.exp64(float(v)))) for v in xs])
    assert np.array_equal(y, want)
    assert (want[xs < -40] == 0).all() and want[xs == 0.0].max() == 2.0 ** 44


def test_device_libm_exp_vs_glibc_report():
    """The sampler's fp64 softmax uses the HIP math library's exp where the
    reference uses glibc's.  Report how often they differ (at most 1 ulp)."""
    import math

    import torch

    from tensormark_amd.sampler import debug_exp

    rng = np.random.default_rng(2)
    xs = -rng.random(200000) * 40
    y = debug_exp(torch.from_numpy(xs).to("cuda:0"), 0).cpu().numpy()
    g = np.exp(xs)   # numpy uses the platform libm (glibc)
    diff = y != g
    ulps = np.abs(y[diff] - g[diff]) / np.array([math.ulp(v) for v in g[diff]])
    print(f"\nlibm exp: {diff.sum()} of {len(xs)} differ from glibc; max {ulps.max() if len(ulps) else 0} ulp")
    assert len(ulps) == 0 or ulps.max() <= 1.0


def test_golden_vectors_gpu(sampler, golden):
    for i, x, p, recent, mask, w0, w1, m in golden_cases(golden):
        g = run_gpu(sampler, x[None], p, recent=None if recent is None else recent[None],
                    mask=None if mask is None else mask[None],
                    draws=np.array([[w0, w1]], np.uint32))
        assert g["status"][0] == 0, i
        assert g["tokens"][0] == m["tok"], (i, g["tokens"][0], m["tok"])
        if not m["g"]:
            assert (g["keep"][0] >= 2) == (m["used"] == 2), i


def test_cfg1_vs_oracle(sampler, orc):
    w = workloads.cfg1()
    for off in range(20):
        p = w["params"].copy()
        p["offset"] = off
        want = orc.sample_batch(w["logits"], p, recent=w["recent"], topk_cap=40)
        g = run_gpu(sampler, w["logits"], p, recent=w["recent"], topk_cap=40)
        check(g, want, 40)


@pytest.mark.parametrize("with_mask", [False, True])
def test_cfg2_full_size_vs_oracle(sampler, orc, with_mask):
    w = workloads.cfg2(with_mask=with_mask)
    want = orc.sample_batch(w["logits"], w["params"], recent=w["recent"], mask=w["mask"],
                            topk_cap=40)
    g = run_gpu(sampler, w["logits"], w["params"], recent=w["recent"], mask=w["mask"],
                topk_cap=40)
    check(g, want, 40)


def test_benched_cfg2_path_vs_oracle(sampler, orc):
    """The exact call bench.py times: config 2 with its mask, the TOPK row-kind
    hint, no per-entry outputs (topk_cap 0: the tail decides the top-p cut and
    the draw from tree sums within a margin), Philox draws from the row
    parameters.  20 Philox offsets, so 1280 draws go through that tail at the
    benchmark's shape; tokens, keep counts and status of every row."""
    import torch

    from tensormark_amd.sampler import ROWS_TOPK, row_kinds_of

    w = workloads.cfg2(with_mask=True)
    assert row_kinds_of(w["params"]) == ROWS_TOPK
    x = _dev(w["logits"], torch)
    rec = _dev(w["recent"].astype(np.int32), torch)
    mask = _dev(w["mask"].view(np.int32), torch)
    for off in range(20):
        p = w["params"].copy()
        p["offset"] = p["offset"] + off
        want = orc.sample_batch(w["logits"], p, recent=w["recent"], mask=w["mask"])
        out = sampler.sample(x, p, recent=rec, mask=mask, row_kinds=ROWS_TOPK)
        torch.cuda.synchronize()
        g = {k: v.cpu().numpy() for k, v in out.items()}
        assert (want["status"] == 0).all()
        check(g, want)


@pytest.mark.parametrize("cap", [64, 0])
def test_cfg3_full_size_fp16_vs_oracle(sampler, orc, cap):
    """cap 64 returns per-entry probabilities (the sequential top-p tail);
    cap 0 returns tokens and keep counts only (the prefix-sum top-p tail)."""
    w = workloads.cfg3()
    x32 = w["logits"].astype(np.float32)
    want = orc.sample_batch(x32, w["params"], mask=w["mask"], topk_cap=cap)
    g = run_gpu(sampler, w["logits"], w["params"], mask=w["mask"], topk_cap=cap, dtype="f16")
    check(g, want, cap)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_packed_stream_rows_vs_oracle(sampler, orc, dtype):
    """2-byte rows without a history window take the general kernel's packed
    stream (20480 ids a chunk: V = 100000 in 5 chunks, not 7): greedy,
    top-k (40, 128 and 300) and top-p rows, with a mask, a NaN row and an
    all-masked row, equal the oracle over the widened values."""
    rng = np.random.default_rng(7 if dtype == "f16" else 8)
    B, V = 12, 100000
    x32 = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    x32[:, ::97] += 6.0
    if dtype == "f16":
        xs = x32.astype(np.float16)
        xw = xs.astype(np.float32)
    else:
        xs = workloads.to_bf16_bits(x32)
        xw = workloads.bf16_bits_to_f32(xs)
    xw = xw.copy()
    if dtype == "f16":
        xs[9, 5000] = np.nan
    else:
        xs[9, 5000] = 0x7FC0
    xw[9, 5000] = np.nan
    bits = rng.random((B, V)) < 0.6
    bits[9, 5000] = True
    bits[10] = False
    mask = workloads.pack_bits(bits)
    p = params_array(B, temperature=0.9, top_k=40, top_p=0.95, seed=np.arange(B) + 31)
    p["greedy"][0] = 1
    p["top_k"] = [40, 40, 128, 300, 0, 0, 40, 0, 50, 40, 40, 0]
    p["top_p"][7] = 0.3
    p["min_p"][6] = 0.02
    want = orc.sample_batch(xw, p, mask=mask, topk_cap=24)
    g = run_gpu(sampler, xs, p, mask=mask, topk_cap=24, dtype=dtype)
    assert list(g["status"][9:11]) == [3, 2]
    check(g, want, 24)


@pytest.mark.parametrize("V", [32776, 40960, 40968, 61448, 122880])
def test_packed_stream_chunk_edges(sampler, orc, V):
    """The packed stream's chunks (20480 ids) against vocabularies at and
    just past their multiples, where the last chunk holds one vector or
    the packed form saves a chunk (fp16, no window): greedy, top-k, top-p
    and min-p rows with a mask; every row equals the oracle."""
    rng = np.random.default_rng(V)
    B = 6
    x32 = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    x32[:, -8:] += 9.0   # the best ids in the last vector
    x32[2, :8] += 12.0   # or the first
    xs = x32.astype(np.float16)
    xw = xs.astype(np.float32)
    bits = rng.random((B, V)) < 0.7
    bits[:, -8:] = True
    mask = workloads.pack_bits(np.pad(bits, ((0, 0), (0, (-V) % 32))))
    p = params_array(B, temperature=0.9, top_k=40, top_p=0.9, seed=np.arange(B) + 700)
    p["greedy"][0] = 1
    p["top_k"] = [40, 1, 40, 128, 0, 0]
    p["top_p"][5] = 0.2
    p["min_p"][3] = 0.1
    want = orc.sample_batch(xw, p, mask=mask, topk_cap=12)
    g = run_gpu(sampler, xs, p, mask=mask, topk_cap=12, dtype="f16")
    check(g, want, 12)


@pytest.mark.parametrize("n_allowed", [70, 700, 1000])
def test_topp_rows_many_entries(sampler, orc, n_allowed):
    """Top-p rows (top_k = 0) holding up to 1000 entries within 40 of the
    maximum, spread over the row's chunks: the whole-list merge ranks them by
    value buckets (2 or 8 keys a thread), and the tail sums thread blocks of
    up to 5 entries; top-p, min-p and temperature varied per row, no
    per-entry outputs."""
    rng = np.random.default_rng(n_allowed)
    B, V = 64, 60000   # 4 chunks: a chunk holds at most 512 candidates
    x = rng.normal(0.0, 1.5, (B, V)).astype(np.float32)
    bits = np.zeros((B, ((V + 31) // 32) * 32), bool)
    for b in range(B):
        bits[b, rng.choice(V, size=n_allowed, replace=False)] = True
    mask = workloads.pack_bits(bits)
    p = params_array(B, temperature=1.0, top_k=0, top_p=0.9, seed=np.arange(B) + 5)
    p["top_p"] = rng.choice([0.3, 0.8, 0.95, 0.999, 1.0], size=B)
    p["min_p"] = rng.choice([0.0, 0.0, 0.01, 0.2], size=B)
    p["temperature"] = rng.choice([0.6, 1.0, 1.7], size=B)
    want = orc.sample_batch(x, p, mask=mask)
    g = run_gpu(sampler, x, p, mask=mask)
    check(g, want)


@pytest.mark.parametrize("grid", [0.5, 0.0])
def test_topp_rows_bucket_ties(sampler, orc, grid):
    """Top-p rows whose values sit on a coarse grid (many exact ties, so many
    keys share a bucket and rank by lowest id within it), and rows where
    every allowed value is equal (grid 0: one bucket holds every key)."""
    rng = np.random.default_rng(31)
    B, V = 24, 40000
    x = rng.normal(0.0, 1.5, (B, V)).astype(np.float32)
    x = np.round(x / grid) * grid if grid else np.full((B, V), 0.25, np.float32)
    x = x.astype(np.float32)
    bits = np.zeros((B, ((V + 31) // 32) * 32), bool)
    for b in range(B):
        bits[b, rng.choice(V, size=int(rng.integers(200, 900)), replace=False)] = True
    mask = workloads.pack_bits(bits)
    p = params_array(B, temperature=1.0, top_k=0, top_p=0.9, seed=np.arange(B) + 11)
    p["top_p"] = rng.choice([0.5, 0.9, 1.0], size=B)
    p["temperature"] = rng.choice([0.7, 1.0], size=B)
    want = orc.sample_batch(x, p, mask=mask)
    g = run_gpu(sampler, x, p, mask=mask)
    check(g, want)


def test_topk_128_tie_heavy_rows(sampler, orc):
    """top_k = 128 rows built to stress the wide kernel's chunk paths: values
    on a coarse grid (more than 128 candidates a chunk: the chunk ranks and
    publishes its top K), all-equal rows (more than 1024: the exact radix
    select), and rows with a few peaks; V = 200000 fp32 is seven chunks of
    the 8-slot form.  The top-k ids come back in rank order."""
    rng = np.random.default_rng(53)
    B, V = 24, 200000
    x = rng.normal(0.0, 1.0, (B, V)).astype(np.float32)
    kind = np.arange(B) % 3
    for b in range(B):
        if kind[b] == 0:
            x[b] = np.round(x[b] * 2.0) / 2.0
        elif kind[b] == 1:
            x[b] = 0.5
        else:
            x[b, rng.choice(V, 40, replace=False)] += 6.0
    p = params_array(B, temperature=1.0, top_k=128, top_p=1.0, seed=np.arange(B) + 17)
    p["temperature"] = rng.choice([0.7, 1.0, 1.3], size=B)
    p["top_p"] = rng.choice([0.5, 0.95, 1.0], size=B)
    p["greedy"] = (np.arange(B) % 8 == 7).astype(np.int32)
    want = orc.sample_batch(x, p, topk_cap=128)
    g = run_gpu(sampler, x, p, topk_cap=128)
    check(g, want, 128)


def test_cfg5_rows_bf16_vs_oracle(sampler, orc):
    w = workloads.cfg5(B=48)
    bits = workloads.to_bf16_bits(w["logits"])
    x32 = workloads.bf16_bits_to_f32(bits)
    want = orc.sample_batch(x32, w["params"], recent=w["recent"], topk_cap=100)
    g = run_gpu(sampler, bits, w["params"], recent=w["recent"], topk_cap=100, dtype="bf16")
    check(g, want, 100)


@pytest.fixture(scope="module")
def cfg5_full(orc):
    """Config 5 at its benchmark size (B = 1024, V = 256000 bf16) and the
    oracle's answer for every row, made once for both kernel choices."""
    w = workloads.cfg5()
    bits = workloads.to_bf16_bits(w["logits"])
    del w["logits"]
    x32 = workloads.bf16_bits_to_f32(bits)
    want = orc.sample_batch(x32, w["params"], recent=w["recent"], topk_cap=100)
    del x32
    return bits, w, want


def test_cfg5_full_workload_vs_oracle(sampler, cfg5_full):
    """Every row of the benchmark workload: tokens, keep counts and the
    top-100 ids and probabilities of the sampled half, the argmax of the
    greedy half (16,384 workgroups, many rounds of residency)."""
    bits, w, want = cfg5_full
    g = run_gpu(sampler, bits, w["params"], recent=w["recent"], topk_cap=100, dtype="bf16")
    assert (want["status"] == 0).all()
    check(g, want, 100)


def test_cfg5_full_workload_benched_path(sampler, cfg5_full):
    """Config 5 as bench.py runs it: no per-entry outputs (topk_cap 0, the
    tree-sum tail) and the row-kind hint from the parameters; tokens, keep
    counts and status of all 1024 rows against the oracle."""
    bits, w, want = cfg5_full
    g = run_gpu(sampler, bits, w["params"], recent=w["recent"], topk_cap=0, dtype="bf16")
    check(g, want)


def test_many_draws_same_row(sampler, orc):
    """One row, 256 batch copies with different uniforms: every draw matches."""
    rng = np.random.default_rng(3)
    V = 5000
    x = np.repeat(rng.normal(0, 1.0, (1, V)).astype(np.float32), 256, axis=0)
    p = params_array(256, temperature=1.3, top_k=100, top_p=0.97, seed=np.arange(256))
    want = orc.sample_batch(x, p, topk_cap=100)
    g = run_gpu(sampler, x, p, topk_cap=100)
    check(g, want, 100)


EDGE = {
    "all_masked": dict(),
    "nan": dict(),
    "posinf": dict(),
    "bad_temp": dict(),
    "ties_all_equal": dict(),
    "few_allowed": dict(),
    "topk1": dict(),
    "topk_gt_V": dict(),
    "tiny_temp": dict(),
    "big_window": dict(),
    "owned_window": dict(),
    "unaligned_V": dict(),
    "small_V": dict(),
    "top_p_one": dict(),
    "greedy_ties": dict(),
    "quantized_ties": dict(),
}


def _edge_case(name, rng):
    V = 20000
    x = rng.normal(0, 2, (4, V)).astype(np.float32)
    p = params_array(4, temperature=0.9, top_k=40, top_p=0.9, seed=np.arange(4))
    recent = mask = None
    if name == "all_masked":
        mask = np.zeros((4, (V + 31) // 32), np.uint32)
        mask[1:, :] = 0xFFFFFFFF
    elif name == "nan":
        x[0, 123] = np.nan
        x[2, 19999] = np.nan
    elif name == "posinf":
        x[1, 7] = np.inf
    elif name == "bad_temp":
        p["temperature"] = [0.0, -1.0, np.inf, 0.5]
    elif name == "ties_all_equal":
        x[:] = 1.0
        x[3, ::7] = 2.0
    elif name == "few_allowed":
        bits = np.zeros((4, ((V + 31) // 32) * 32), bool)
        for b in range(4):
            bits[b, rng.choice(V, size=[3, 10, 39, 45][b], replace=False)] = True
        mask = workloads.pack_bits(bits)
    elif name == "topk1":
        p["top_k"] = 1
    elif name == "topk_gt_V":
        V = 300
        x = x[:, :V].copy()
        p["top_k"] = [V + 5, V, 0, -3]
        p["top_p"] = 0.99
    elif name == "tiny_temp":
        p["temperature"] = [1e-3, 1e-6, 3.0, 100.0]
    elif name == "big_window":
        recent = rng.integers(0, 50, (4, 2000)).astype(np.int32)
        recent[:, ::3] = 7
        x[:, :50] += 8.0
        p["repeat_penalty"] = 1.3
        p["repeat_last_n"] = [2000, 1500, 10, 0]
        p["frequency_penalty"] = 0.05
        p["presence_penalty"] = 0.3
    elif name == "owned_window":
        # <= 1024 history ids: penalties through the id owners; heavy
        # repeats, penalised ids the mask hides, ids past V
        recent = rng.integers(0, 60, (4, 1000)).astype(np.int32)
        recent[:, ::5] = 19999
        recent[:, 1::97] = V + 3
        x[:, :60] += 7.0
        bits = np.ones((4, ((V + 31) // 32) * 32), bool)
        bits[:, 10:20] = False
        mask = workloads.pack_bits(bits)
        p["repeat_penalty"] = [1.3, 1.05, 2.0, 1.0]
        p["repeat_last_n"] = [1000, 400, 1, 64]
        p["frequency_penalty"] = [0.05, 0.0, -0.5, 0.2]
        p["presence_penalty"] = [0.3, 0.0, 0.1, 0.1]
        p["greedy"] = [0, 0, 1, 0]
    elif name == "unaligned_V":
        V = 20001
        x = rng.normal(0, 2, (4, V)).astype(np.float32)
    elif name == "small_V":
        V = 37
        x = rng.normal(0, 2, (4, V)).astype(np.float32)
        p["top_k"] = [40, 5, 37, 1]
    elif name == "top_p_one":
        p["top_p"] = [1.0, 1.0, 0.0, 2.0]
        p["top_k"] = [40, 128, 40, 100]
    elif name == "greedy_ties":
        x[:] = 0.5
        x[1, 5000] = 0.75
        x[2, 19999] = 0.75
        x[2, 15000] = 0.75
        p["greedy"] = 1
    elif name == "quantized_ties":
        x = np.round(x * 2) / 2
        p["top_k"] = [40, 100, 7, 128]
    return x, p, recent, mask


@pytest.mark.parametrize("cap", [40, 0])
@pytest.mark.parametrize("name", list(EDGE))
def test_edge_cases(sampler, orc, name, cap):
    """cap 40 asks for the per-entry probabilities (the sequential fp64
    tail); cap 0 takes the tail that decides from tree sums."""
    rng = np.random.default_rng(abs(hash(name)) % 2**32)
    x, p, recent, mask = _edge_case(name, rng)
    want = orc.sample_batch(x, p, recent=recent, mask=mask, topk_cap=cap)
    g = run_gpu(sampler, x, p, recent=recent, mask=mask, topk_cap=cap)
    check(g, want, cap)


@pytest.mark.parametrize("top_k", [40, 0])
def test_decisions_on_exact_boundaries(sampler, orc, top_k):
    """Equal logits over 4 or 8 allowed ids make every prefix sum exact, so
    the top-p cut can land exactly on top_p and the uniform exactly on a
    partial sum: the tree-sum tails (top-k rows, and top_k = 0 rows through
    the top-p tail) must defer those decisions to the sequential sums and
    agree with the reference's lower_bound."""
    V = 1000
    u_words = {0.0: (0, 0), 0.25: (0, 0x40000000), 0.5: (0, 0x80000000),
               0.75: (0, 0xC0000000), 0.375: (0, 0x60000000),
               0.5 - 2.0**-53: (0xFFFFF800, 0x7FFFFFFF)}
    rows = []
    for n_allowed in (4, 8):
        for top_p in (0.5, 0.75, 0.25, 0.9, 1.0):
            for u in u_words:
                rows.append((n_allowed, top_p, u))
    B = len(rows)
    x = np.full((B, V), 2.5, np.float32)
    bits = np.zeros((B, ((V + 31) // 32) * 32), bool)
    draws = np.zeros((B, 2), np.uint32)
    p = params_array(B, temperature=1.0, top_k=top_k, top_p=0.9, seed=np.arange(B))
    rng = np.random.default_rng(11)
    for b, (na, tp, u) in enumerate(rows):
        bits[b, rng.choice(V, size=na, replace=False)] = True
        draws[b] = u_words[u]
        p["top_p"][b] = tp
        assert orc.canonical(int(draws[b, 0]), int(draws[b, 1])) == u
    mask = workloads.pack_bits(bits)
    # With 4 or 8 finite entries an 8-slot id list of a top_k = 0 row runs
    # into the masked ids (-inf, in id order): the whole-row path lists them.
    for cap in (0, 8):
        want = orc.sample_batch(x, p, mask=mask, draws=draws, topk_cap=cap)
        g = run_gpu(sampler, x, p, mask=mask, draws=draws, topk_cap=cap)
        check(g, want, cap)


@pytest.mark.parametrize("B,V", [(1, 128256), (7, 70000), (13, 128256), (37, 70000), (150, 40000)])
def test_batch_sizes_off_the_xcd_grouping(sampler, orc, B, V):
    """Workgroups map to (row, chunk) so that rows of the first 8 * (B // 8)
    stay whole on one XCD and the rest follow in order: batches that are not
    a multiple of 8 mix both parts (4 and 3 chunks of the 8-slot form here).
    B = 150, V = 40000 is too many workgroups for one per CU and fits two:
    fp32 in the 4-slot form (3 chunks).  Half the rows greedy, the rest
    top-k 40 with the history penalties and a mask."""
    w = workloads.cfg2(B=B, V=V, seed=40 + B, with_mask=True)
    p = w["params"].copy()
    p["greedy"] = (np.arange(B) % 2).astype(np.int32)
    want = orc.sample_batch(w["logits"], p, recent=w["recent"], mask=w["mask"], topk_cap=40)
    g = run_gpu(sampler, w["logits"], p, recent=w["recent"], mask=w["mask"], topk_cap=40)
    check(g, want, 40)


def test_repeated_calls_reuse_workspace(sampler, orc):
    """Back-to-back launches on one context: the arrival counters reset."""
    w = workloads.cfg2(B=16, V=40000, seed=9)
    want = orc.sample_batch(w["logits"], w["params"], recent=w["recent"], topk_cap=40)
    for _ in range(5):
        g = run_gpu(sampler, w["logits"], w["params"], recent=w["recent"], topk_cap=40)
        check(g, want, 40)


def test_dense_row_without_topk(sampler, orc):
    """top_k = 0 over a row whose every entry lies within 40 of the maximum:
    the whole-row path (full sort) samples it."""
    rng = np.random.default_rng(12)
    x = rng.normal(0, 2, (2, 20000)).astype(np.float32)
    p = params_array(2, temperature=1.0, top_k=0, top_p=0.9, seed=np.arange(2))
    want = orc.sample_batch(x, p, topk_cap=16)
    g = run_gpu(sampler, x, p, topk_cap=16)
    check(g, want, 16)


def _large_k_rows(kind, K, B, V, rng):
    """Rows for 128 < top_k < V.  "dense": every entry within 40 of the
    maximum (n > K).  "spiked": 50 ids 60 above the rest, so the entries that
    move the sums are fewer than K and the rest of the top K lies past them.
    "masked": K // 2 allowed ids, so fewer than K finite entries."""
    x = rng.normal(0.0, 1.5, (B, V)).astype(np.float32)
    mask = None
    if kind == "spiked":
        for b in range(B):
            x[b, rng.choice(V, 50, replace=False)] += 60.0
    elif kind == "masked":
        bits = np.zeros((B, ((V + 31) // 32) * 32), bool)
        for b in range(B):
            bits[b, rng.choice(V, K // 2, replace=False)] = True
        mask = workloads.pack_bits(bits)
    p = params_array(B, temperature=1.0, top_k=K, top_p=0.95, seed=np.arange(B) + 3 * K)
    p["top_p"] = rng.choice([0.5, 0.9, 0.999, 1.0], size=B)
    p["min_p"] = rng.choice([0.0, 0.0, 1e-3], size=B)
    p["temperature"] = rng.choice([0.7, 1.0, 1.6], size=B)
    return x, p, mask


@pytest.mark.parametrize("cap", [0, 16])
@pytest.mark.parametrize("kind", ["dense", "spiked", "masked"])
@pytest.mark.parametrize("K", [129, 200, 1000])
def test_large_top_k_rows(sampler, orc, K, kind, cap):
    """128 < top_k < V: tmsample::sample normalises and draws over the top K
    only (tmsample.h:180-199), with the survivors both above and below K."""
    rng = np.random.default_rng(1000 * K + len(kind))
    x, p, mask = _large_k_rows(kind, K, 16, 60000, rng)
    want = orc.sample_batch(x, p, mask=mask, topk_cap=cap)
    g = run_gpu(sampler, x, p, mask=mask, topk_cap=cap)
    check(g, want, cap)


@pytest.mark.parametrize("cap", [0, 64, 2000])
def test_dense_rows_whole_row_path(sampler, orc, cap):
    """Rows only the whole-row path can finish: top_k = 0 over flat rows
    (tens of thousands of entries within 40 of the maximum) at V = 128256,
    with penalties and a mask; a row whose draw lands past the entries that
    move the sums (u just below 1 with top_p = 1); a min-p threshold below
    e^-40; id lists longer than the held entries."""
    rng = np.random.default_rng(77 + cap)
    B, V = 8, 128256
    x = rng.normal(0.0, 1.0, (B, V)).astype(np.float32)
    x[4:6, :40] += 60.0           # rows 4, 5: 40 entries move the sums
    recent = rng.integers(0, V, (B, 256)).astype(np.int32)
    p = params_array(B, temperature=1.0, top_k=0, top_p=0.9, seed=np.arange(B) + 11,
                     repeat_penalty=1.1, repeat_last_n=256, frequency_penalty=0.2,
                     presence_penalty=0.1)
    p["top_k"] = [0, 0, 50000, 0, 1000, 0, 0, 300]
    p["top_p"] = [0.9, 0.5, 0.95, 1.0, 1.0, 1.0, 0.99, 0.8]
    p["temperature"] = [1.0, 0.6, 1.3, 1.0, 1.0, 1.0, 2.0, 1.0]
    p["min_p"] = [0.0, 0.0, 0.0, 0.0, 0.0, 1e-30, 0.01, 0.0]
    draws = rng.integers(0, 2**32, (B, 2), dtype=np.uint64).astype(np.uint32)
    draws[3] = draws[4] = [0xFFFFFFFF, 0xFFFFFFFF]   # u = 1 - 2^-53
    bits = np.ones((B, ((V + 31) // 32) * 32), bool)
    bits[1, ::3] = False
    mask = workloads.pack_bits(bits)
    want = orc.sample_batch(x, p, recent=recent, mask=mask, draws=draws, topk_cap=cap)
    g = run_gpu(sampler, x, p, recent=recent, mask=mask, draws=draws, topk_cap=cap)
    check(g, want, cap)


def test_wide_kernel_error_rows(sampler, orc):
    """Rows the wide top-k kernel must reject like the general kernel:
    temperature 0 (BAD_PARAMS, on a row of ties), an all-masked row
    (ALL_MASKED), NaN and +inf (NONFINITE); and a top-p row under the
    ROWS_TOPK promise, which the wide kernel reports as UNSUPPORTED instead
    of sampling it."""
    import torch

    from tensormark_amd.sampler import ROWS_ANY, ROWS_TOPK

    V = 100
    x = np.zeros((5, V), np.float32)
    x[3, 17] = np.nan
    x[4, 5] = np.inf
    p = params_array(5, top_k=40, temperature=0.7)
    p["temperature"][0] = 0.0
    mask = np.full((5, (V + 31) // 32), 0xFFFFFFFF, np.uint32)
    mask[1] = 0
    gpu = run_gpu(sampler, x, p, mask=mask)
    want = orc.sample_batch(x, p, mask=mask)
    assert list(gpu["status"]) == [1, 2, 0, 3, 3], gpu["status"]
    check(gpu, want)
    # a top-p row (top_k = 0 over 1000 ids) under the top-k promise
    p2 = params_array(2, top_k=40)
    p2["top_k"][1] = 0
    xs = np.random.default_rng(3).normal(0, 2, (2, 1000)).astype(np.float32)
    xs[1, 30:] = -100.0   # a top-p row the general kernel holds whole (30 live ids)
    out = sampler.sample(torch.from_numpy(xs).to("cuda:0"), p2, row_kinds=ROWS_TOPK)
    torch.cuda.synchronize()
    st = out["status"].cpu().numpy()
    want2 = orc.sample_batch(xs, p2)
    if sampler.kernel == "auto":
        assert st[1] == 4 and st[0] == 0, st
        assert out["tokens"].cpu().numpy()[0] == want2["tokens"][0]
    out = sampler.sample(torch.from_numpy(xs).to("cuda:0"), p2, row_kinds=ROWS_ANY)
    torch.cuda.synchronize()
    assert list(out["status"].cpu().numpy()) == [0, 0]
    assert np.array_equal(out["tokens"].cpu().numpy(), want2["tokens"])


@pytest.mark.parametrize("allowed", [60, 127, 140, 400])
def test_topp_lists_around_the_staged_words(sampler, orc, allowed):
    """Top-p rows over 4 chunks (V = 65536), the mask leaving about
    `allowed` ids a chunk: lists that fit the merger's 127 staged entries
    (ranked in place) and lists past them (the merge rounds), mixed in one
    batch; every row equals the oracle."""
    rng = np.random.default_rng(allowed)
    B, V = 8, 65536
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    bits = rng.random((B, V)) < (allowed + rng.integers(-15, 15, (B, 1))) / 16384.0
    mask = workloads.pack_bits(bits)
    p = params_array(B, temperature=1.0, top_k=0, top_p=0.9, seed=np.arange(B) + 17)
    p["top_p"][1::2] = 0.5
    p["min_p"][3] = 0.05
    want = orc.sample_batch(x, p, mask=mask, topk_cap=32)
    g = run_gpu(sampler, x, p, mask=mask, topk_cap=32)
    assert (g["status"] == 0).all()
    check(g, want, 32)


def test_whole_lists_over_more_than_16_chunks(orc):
    """V = 300,000 (19 chunks, past the sampled merge's 16 lists): top-k
    rows and a top-p row through the whole-list merge with the staged
    headers; every row equals the oracle."""
    import torch

    from tensormark_amd import Sampler

    rng = np.random.default_rng(19)
    B, V = 4, 300000
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    p = params_array(B, temperature=0.8, top_k=40, top_p=0.95, seed=np.arange(B) + 5)
    p["top_k"][2] = 0
    bits = np.ones((B, V), bool)
    bits[2] = rng.random(V) < 0.004
    mask = workloads.pack_bits(bits)
    want = orc.sample_batch(x, p, mask=mask, topk_cap=16)
    s = Sampler(max_batch=4, max_vocab=V)
    try:
        out = s.sample(torch.from_numpy(x).to("cuda:0"), p, mask=torch.from_numpy(mask.view(np.int32)).to("cuda:0"),
                       topk_cap=16)
        torch.cuda.synchronize()
        g = {k: v.cpu().numpy() for k, v in out.items()}
    finally:
        s.close()
    assert (g["status"] == 0).all(), g["status"]
    check(g, want, 16)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_topk_rows_of_a_grid_in_several_rounds(sampler, orc, dtype):
    """B = 80 rows of V = 262144 (1,280 workgroups of the general kernel, more
    than four a CU, in two rounds of residency): top-k 1..128 rows with a
    window, greedy and top-p rows, masked; every row equals the oracle."""
    rng = np.random.default_rng(81 if dtype == "f32" else 82)
    B, V = 80, 262144
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    x[:, rng.choice(V, 50, replace=False)] += 8.0
    recent = rng.integers(0, V, (B, 200)).astype(np.int32)
    recent[:, ::4] = rng.choice(V, 50)[rng.integers(0, 50, (B, 50))]
    p = params_array(B, temperature=0.8, top_k=40, top_p=0.95, seed=np.arange(B) + 300,
                     repeat_penalty=1.2, repeat_last_n=200)
    p["top_k"] = np.resize([1, 7, 40, 100, 128, 40, 0, 40], B)
    p["greedy"] = (np.arange(B) % 9 == 4).astype(np.int32)
    p["min_p"][::5] = 0.05
    bits = rng.random((B, V)) < 0.8
    mask = workloads.pack_bits(bits)
    if dtype == "bf16":
        xs = workloads.to_bf16_bits(x)
        xw = workloads.bf16_bits_to_f32(xs)
    else:
        xs = xw = x
    want = orc.sample_batch(xw, p, recent=recent, mask=mask, topk_cap=16)
    g = run_gpu(sampler, xs, p, recent=recent, mask=mask, topk_cap=16, dtype=dtype)
    assert (g["status"] == 0).all(), g["status"]
    check(g, want, 16)


def test_whole_row_regions_shared_by_more_rows_than_regions(sampler, orc):
    """300 flat top-p rows, each needing the whole-row path, against the
    context's 256 regions: rows r and r + 256 take turns on one region's
    lock; every row equals the oracle."""
    rng = np.random.default_rng(53)
    B, V = 300, 5000
    x = rng.normal(0.0, 0.5, (B, V)).astype(np.float32)
    p = params_array(B, temperature=1.0, top_k=0, top_p=0.95, seed=np.arange(B) + 3)
    want = orc.sample_batch(x, p, topk_cap=8)
    g = run_gpu(sampler, x, p, topk_cap=8)
    assert (g["status"] == 0).all()
    check(g, want, 8)


def test_broken_promise_rows_sampled_by_the_general_kernel(sampler, orc):
    """A ROWS_TOPK call the wide kernel does not take (a 600-id window, past
    its 1024): the general kernel samples the rows that break the promise
    like any other (top_k = 0 over a flat row, which needs the whole-row
    path, and top_k = 300), in the same launch."""
    import torch

    from tensormark_amd.sampler import ROWS_TOPK

    rng = np.random.default_rng(41)
    B, V, n = 6, 30000, 1100
    x = rng.normal(0.0, 0.3, (B, V)).astype(np.float32)
    x[:, :50] += 3.0
    p = params_array(B, temperature=0.9, top_k=40, top_p=0.95, seed=np.arange(B) + 60)
    p["top_k"][1] = 0          # flat row: thousands of entries within 40 of the maximum
    p["top_p"][1] = 0.999
    p["top_k"][3] = 300
    p["repeat_penalty"] = 1.1
    p["repeat_last_n"] = 64
    recent = rng.integers(0, 80, (B, n)).astype(np.int32)
    want = orc.sample_batch(x, p, recent=recent, topk_cap=16)
    out = sampler.sample(torch.from_numpy(x).to("cuda:0"), p, recent=torch.from_numpy(recent).to("cuda:0"),
                         topk_cap=16, row_kinds=ROWS_TOPK)
    torch.cuda.synchronize()
    g = {k: v.cpu().numpy() for k, v in out.items()}
    assert (g["status"] == 0).all(), g["status"]
    check(g, want, 16)


def test_wide_kernel_rows_with_a_wide_topk_cap(sampler, orc):
    """The wide top-k kernel (config 2's shape under the ROWS_TOPK promise)
    with per-row outputs wider than its merge waves (topk_cap 300 > 256
    threads): error rows (temperature 0, all masked, NaN) fill every output
    with -1 / 0, greedy rows put their one id first, sampled rows match the
    oracle over all 300 entries."""
    import torch

    from tensormark_amd.sampler import ROWS_TOPK

    rng = np.random.default_rng(31)
    B, V, cap = 64, 128256, 300
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    x[5, 70000] = np.nan
    p = params_array(B, temperature=0.8, top_k=40, top_p=0.95, seed=np.arange(B) + 900)
    p["top_k"] = np.where(np.arange(B) % 3 == 0, 128, 40)
    p["greedy"] = (np.arange(B) % 8 == 1).astype(np.int32)
    p["temperature"][2] = 0.0
    mask = np.full((B, (V + 31) // 32), 0xFFFFFFFF, np.uint32)
    mask[9] = 0
    out = sampler.sample(torch.from_numpy(x).to("cuda:0"), p,
                         mask=torch.from_numpy(mask.view(np.int32)).to("cuda:0"), topk_cap=cap,
                         row_kinds=ROWS_TOPK)
    torch.cuda.synchronize()
    gpu = {k: v.cpu().numpy() for k, v in out.items()}
    want = orc.sample_batch(x, p, mask=mask, topk_cap=cap)
    assert gpu["status"][2] == 1 and gpu["status"][9] == 2 and gpu["status"][5] == 3
    for b in (2, 5, 9):
        assert (gpu["topk_ids"][b] == -1).all() and (gpu["topk_probs"][b] == 0).all()
    check(gpu, want, cap)


def test_tie_fixture_rows(sampler, orc):
    """Rows full of exact ties (tests/golden/tie_golden.npz): the device gives
    the oracle's lowest-id-first order, keep and draws, in groups of equal
    shape (the reference's libstdc++ order is checked against the oracle on
    the CPU)."""
    import os

    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tie_golden.npz"),
                allow_pickle=False)
    meta = g["meta"]
    groups = {}
    for i, m in enumerate(meta):
        groups.setdefault((g[f"x{i}"].size, float(m["T"]), int(m["k"]), float(m["p"])), []).append(i)
    for (V, T, k, p), idx in groups.items():
        x = np.stack([g[f"x{i}"] for i in idx])
        draws = np.stack([g[f"draws{i}"][0, :2] for i in idx]).astype(np.uint32)
        prm = params_array(len(idx), temperature=T, top_k=k, top_p=p)
        want = orc.sample_batch(x, prm, draws=draws, topk_cap=k)
        got = run_gpu(sampler, x, prm, draws=draws, topk_cap=k)
        check(got, want, k)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_massive_ties_with_window_penalties(sampler, orc, dtype):
    """Rows whose entries all tie, with window penalties: the chunk's
    candidates overflow and its exact radix select reads the penalised values
    through the window counts, which it counts again (the candidate staging
    shares their LDS).  Top-k 100 at T = 2.5: the top 100 are the lowest
    allowed ids outside the window."""
    rng = np.random.default_rng({"f32": 61, "f16": 62, "bf16": 63}[dtype])
    B, V = 4, 40000
    x32 = np.full((B, V), 1.25, np.float32)
    x32[1, 1::2] = 1.0
    if dtype == "f16":
        xs = x32.astype(np.float16)
    elif dtype == "bf16":
        xs = workloads.to_bf16_bits(x32)
    else:
        xs = x32
    bits = rng.random((B, ((V + 31) // 32) * 32)) < 0.85
    bits[:, V:] = False
    mask = workloads.pack_bits(bits)
    recent = rng.integers(0, 200, (B, 512)).astype(np.int32)
    p = params_array(B, temperature=2.5, top_k=100, top_p=0.9, seed=np.arange(B) + 77)
    p["repeat_penalty"] = [1.05, 1.3, 1.0, 1.05]
    p["repeat_last_n"] = [512, 64, 512, 8]
    p["frequency_penalty"] = [0.1, 0.0, 0.2, 0.0]
    want = orc.sample_batch(x32 if dtype == "f32" else (xs.astype(np.float32) if dtype == "f16"
                                                        else workloads.bf16_bits_to_f32(xs)),
                            p, recent=recent, mask=mask, topk_cap=16)
    g = run_gpu(sampler, xs, p, recent=recent, mask=mask, topk_cap=16, dtype=dtype)
    check(g, want, 16)
