"""The allocation-free entry point (tms_sample_batch_noalloc) against
tms_sample_batch: the same outputs, bit for bit, on two calls in a row, the
second with a smaller batch and vocabulary, each over both row-kind hints
(the top-k kernel and the general kernel with its whole-row pass)."""
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
                # general kernel: top-p rows, one dense enough for the whole-row pass
                p["top_k"][::3] = 0
                w["logits"][1] = np.random.default_rng(i).normal(0, 0.5, w["logits"].shape[1])
                p["top_k"][1] = 0
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
