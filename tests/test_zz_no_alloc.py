"""The allocation-free entry point (tms_sample_batch_noalloc) against
tms_sample_batch: the same outputs, bit for bit, on two calls in a row, the
second with a smaller batch and vocabulary, each over both row-kind hints
(the top-k kernel and the general kernel with its whole-row path)."""
from __future__ import annotations

import numpy as np
import pytest

from tensormark_amd import workloads

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _run(sampler, x, params, recent, mask, noalloc, cap, row_kinds):
    import torch

    out = sampler.sample(_dev(x), params, recent=_dev(recent),
                         mask=_dev(mask.view(np.int32)), topk_cap=cap,
                         row_kinds=row_kinds, noalloc=noalloc)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


@pytest.mark.parametrize("row_kinds", [0, 1])
def test_noalloc_matches_context_entry_point(row_kinds):
    from tensormark_amd import Sampler

    s = Sampler(max_batch=64, max_vocab=262144)
    try:
        calls = [workloads.cfg2(B=64, V=128256, seed=5, with_mask=True),
                 workloads.cfg2(B=9, V=50000, seed=6, with_mask=True)]
        for i, w in enumerate(calls):
            p = w["params"].copy()
            if row_kinds == 0:
                # general kernel: top-p rows, three dense enough for the
                # whole-row path (they share the scratch's one region in turn)
                p["top_k"][::3] = 0
                for r in (1, 4, 7):
                    w["logits"][r] = np.random.default_rng(10 * i + r).normal(0, 0.5, w["logits"].shape[1])
                    p["top_k"][r] = 0
            x = w["logits"]
            want = _run(s, x, p, w["recent"], w["mask"], False, 40, row_kinds)
            got = _run(s, x, p, w["recent"], w["mask"], True, 40, row_kinds)
            assert (want["status"] == 0).all(), (i, want["status"])
            for k in ("status", "tokens", "keep", "topk_ids"):
                assert np.array_equal(got[k], want[k]), (i, k)
            assert np.array_equal(got["topk_probs"].view(np.uint32),
                                  want["topk_probs"].view(np.uint32)), i
    finally:
        s.close()


def test_noalloc_rejects_sizes_beyond_its_maximum():
    import ctypes

    from tensormark_amd import Sampler, make_params

    s = Sampler(max_batch=65, max_vocab=1000)
    try:
        x = _dev(np.zeros((65, 1000), np.float32))
        p = s.params_tensor(make_params(65))
        out = {"tokens": _dev(np.zeros(65, np.int32)), "status": _dev(np.zeros(65, np.int32))}
        a = s.make_args(x, p, out=out)
        assert s.lib.tms_sample_batch_noalloc(ctypes.byref(a), None) == -2   # TMS_ERR_CAPACITY
    finally:
        s.close()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_noalloc_history_rows_match_context(dtype):
    """The history pre-pass through the static scratch (its history-list
    regions) with the n-gram ban and DRY, 2-byte logits: bit for bit the
    context entry point's answers, on two calls in a row, the second
    smaller."""
    import torch

    from tensormark_amd import Sampler, make_history

    s = Sampler(max_batch=64, max_vocab=262144)
    try:
        for i, (B, V, n) in enumerate([(48, 60000, 300), (7, 20000, 120)]):
            rng = np.random.default_rng(70 + i)
            x32 = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
            recent = np.resize(rng.integers(0, 40, 9).astype(np.int32), (B, n)).copy()
            recent[:, ::7] = rng.integers(0, V, (B, len(range(0, n, 7))))
            x32[:, :40] += 5.0
            if dtype == "f16":
                x = torch.from_numpy(x32.astype(np.float16)).to("cuda:0")
            else:
                x = torch.from_numpy(workloads.to_bf16_bits(x32)).view(torch.bfloat16).to("cuda:0")
            from tests.helpers import params_array

            p = params_array(B, temperature=0.9, top_k=40, top_p=0.95, seed=np.arange(B) + 5)
            p["repeat_penalty"] = 1.2
            p["repeat_last_n"] = 64
            h = make_history(B, no_repeat_ngram=3, dry_multiplier=0.8, dry_base=1.75,
                             dry_allowed_length=2, dry_penalty_last_n=n)
            res = []
            for noalloc in (False, True):
                out = s.sample(x, p, recent=_dev(recent), topk_cap=16, history=h, noalloc=noalloc)
                torch.cuda.synchronize()
                res.append({k: v.cpu().numpy() for k, v in out.items()})
            want, got = res
            assert (want["status"] == 0).all(), (i, want["status"])
            for k in ("status", "tokens", "keep", "topk_ids"):
                assert np.array_equal(got[k], want[k]), (i, k)
            assert np.array_equal(got["topk_probs"].view(np.uint32), want["topk_probs"].view(np.uint32))
    finally:
        s.close()


def test_noalloc_call_replays_in_a_hip_graph():
    """One allocation-free call captured in a HIP graph after a warm-up call
    (inputs already on the device), replayed five times with eager work and
    synchronisations between the replays: every replay's outputs equal the
    eager call's."""
    import ctypes

    import torch

    from tensormark_amd import Sampler

    s = Sampler(max_batch=64, max_vocab=262144)
    try:
        w = workloads.cfg2(B=64, V=128256, seed=8, with_mask=True)
        x, rec, mask = _dev(w["logits"]), _dev(w["recent"]), _dev(w["mask"].view(np.int32))
        params = s.params_tensor(w["params"])
        from tensormark_amd.sampler import row_kinds_of

        out = {k: torch.full((64,), -7, dtype=torch.int32, device="cuda:0")
               for k in ("tokens", "status", "keep")}
        a = s.make_args(x, params, recent=rec, mask=mask, out=out, row_kinds=row_kinds_of(w["params"]))
        stream = torch.cuda.Stream()
        sp = ctypes.c_void_p(stream.cuda_stream)
        with torch.cuda.stream(stream):
            assert s.lib.tms_sample_batch_noalloc(ctypes.byref(a), sp) == 0   # warm-up (eager)
        torch.cuda.synchronize()
        want = {k: v.cpu().numpy().copy() for k, v in out.items()}
        assert (want["status"] == 0).all()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            assert s.lib.tms_sample_batch_noalloc(ctypes.byref(a), sp) == 0
        torch.cuda.synchronize()
        for r in range(5):
            for v in out.values():
                v.fill_(-7)          # eager work between the replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for k in out:
                assert np.array_equal(out[k].cpu().numpy(), want[k]), (r, k)
    finally:
        s.close()
