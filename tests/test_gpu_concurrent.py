"""The residency-dependent kernels beside concurrent GPU work.

The wide top-k kernel and the verify's waiting resolve are chosen only when
their grid fits the device at once; their workgroups wait on each other with
bounded waits.  Here they run on one stream while a second stream (default
priority) runs large matrix multiplications that hold compute units, so some
of their workgroups start late.  Every row must equal the oracle's answer or
report TMS_ROW_INTERNAL; after an internal error a workspace reset and a
repeat give the oracle's answer.  No row may carry a wrong token."""
from __future__ import annotations

import numpy as np
import pytest

from tensormark_amd import workloads

pytestmark = pytest.mark.gpu

INTERNAL = 5


def _dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to("cuda:0")


def _busy(stream, n=12, size=8192):
    """Queue n bf16 GEMMs of size^3 on `stream` (about 0.5 ms each)."""
    import torch

    with torch.cuda.stream(stream):
        a = torch.randn(size, size, device="cuda:0", dtype=torch.bfloat16)
        b = torch.randn(size, size, device="cuda:0", dtype=torch.bfloat16)
        c = None
        for _ in range(n):
            c = a @ b
    return a, b, c


def test_sampler_beside_a_busy_stream(sampler, orc):
    import torch

    from tensormark_amd.sampler import row_kinds_of

    w = workloads.cfg2(with_mask=True)
    want = orc.sample_batch(w["logits"], w["params"], recent=w["recent"], mask=w["mask"])
    x, rec, mask = _dev(w["logits"]), _dev(w["recent"]), _dev(w["mask"].view(np.int32))
    params = sampler.params_tensor(w["params"])
    kinds = row_kinds_of(w["params"]) if sampler.kernel == "auto" else 0
    torch.cuda.synchronize()
    busy = torch.cuda.Stream()
    keep = _busy(busy)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    outs = []
    for _ in range(16):
        out = sampler.sample(x, params, recent=rec, mask=mask, row_kinds=kinds)
        outs.append({k: v.clone() for k, v in out.items()})
    e1.record()
    torch.cuda.synchronize()
    # time of the sampler's calls, which ran while the GEMMs were queued on the other stream
    print(f"16 calls beside the GEMMs: {e0.elapsed_time(e1):.2f} ms")
    del keep
    internal = 0
    for i, o in enumerate(outs):
        st, tok = o["status"].cpu().numpy(), o["tokens"].cpu().numpy()
        ok = st == 0
        internal += int((st == INTERNAL).sum())
        assert ((st == 0) | (st == INTERNAL)).all(), (i, st)
        assert np.array_equal(tok[ok], want["tokens"][ok]), i
        assert np.array_equal(o["keep"].cpu().numpy()[ok], want["keep"][ok]), i
    print(f"beside a busy stream: {internal} internal-error rows of {16 * len(want['tokens'])}")
    if internal:
        sampler.reset_workspace()
    out = sampler.sample(x, params, recent=rec, mask=mask, row_kinds=kinds)
    torch.cuda.synchronize()
    assert (out["status"].cpu().numpy() == 0).all()
    assert np.array_equal(out["tokens"].cpu().numpy(), want["tokens"])


def test_verify_beside_a_busy_stream(sampler, orc):
    import torch

    from tests.test_gpu_spec import philox_words

    w = workloads.cfg4()
    tg, dr, tok = _dev(w["target"]), _dev(w["draft"]), _dev(w["tokens"].astype(np.int32))
    words = philox_words(orc, w["params"], w["tokens"].shape[1])
    want = [orc.spec_verify_seq(w["target"][b], w["draft"][b], w["tokens"][b],
                                float(w["params"]["temperature"][b]), words[b])
            for b in range(len(w["params"]))]
    torch.cuda.synchronize()
    busy = torch.cuda.Stream()
    keep = _busy(busy)
    params = sampler.params_tensor(w["params"])
    outs = [{k: v.clone() for k, v in sampler.spec_verify(tg, dr, tok, params).items()} for _ in range(8)]
    torch.cuda.synchronize()
    del keep
    internal = 0
    for i, o in enumerate(outs):
        st, acc, tk = (o[k].cpu().numpy() for k in ("status", "accepted", "token"))
        for b, (wst, wacc, wtok) in enumerate(want):
            if st[b] == INTERNAL:
                internal += 1
                continue
            assert (st[b], acc[b], tk[b]) == (wst, wacc, wtok), (i, b)
    print(f"verify beside a busy stream: {internal} internal-error sequences of {8 * len(want)}")
    if internal:
        sampler.reset_workspace()
    o = sampler.spec_verify(tg, dr, tok, params)
    torch.cuda.synchronize()
    for b, (wst, wacc, wtok) in enumerate(want):
        assert (o["status"][b].item(), o["accepted"][b].item(), o["token"][b].item()) == (wst, wacc, wtok), b
