"""The device-ordering facts the cross-workgroup exchanges rely on, checked on
the GPU, and the workspace reset.

tms_debug_ordering runs writer/reader kernel pairs with the writer and reader
workgroups on different XCDs (each XCD has its own L2) and counts violations:
a reader kernel that sees a value older than the previous kernel's store, a
store to one word of a 128-byte line that loses another workgroup's store to a
neighbouring word, and two kernels on one stream whose executions overlap.
It also counts lost words when each writer reads the line before writing its
words: a pattern no sampler kernel uses, reported rather than asserted.
It also reports the XCD count and whether workgroups land round-robin over
the XCDs: the launches are shaped for that placement, but it only decides
their speed, so it is reported, not asserted."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tensormark_amd import sampler as smod
from tensormark_amd import workloads

pytestmark = pytest.mark.gpu


def test_device_ordering_facts():
    import torch

    assert torch.cuda.is_available()
    lib = smod.load_library()
    counts = (C.c_int32 * 8)()
    rc = lib.tms_debug_ordering(64, counts)
    assert rc == 0, lib.tms_status_string(rc)
    stale, lost, overlap, misplaced, xcds, not_run, lost_rw = list(counts)[:7]
    print(f"ordering: stale={stale} lost={lost} overlap={overlap} misplaced={misplaced} xcds={xcds} "
          f"not_run={not_run} lost_after_read={lost_rw}")
    if xcds < 3:
        pytest.skip(f"{xcds} XCD(s): the cross-XCD cases need three")
    assert not_run < 2 * 64, "no trial found its XCD roles"
    assert stale == 0
    assert lost == 0
    assert overlap == 0


def test_workspace_reset_then_sample(sampler, orc):
    """A reset returns the workspace to its creation state: the calls after it
    give the oracle's answers, as the calls before it do."""
    import torch

    w = workloads.cfg2(B=16, V=40000, seed=21)
    want = orc.sample_batch(w["logits"], w["params"], recent=w["recent"], topk_cap=40)
    from tests.test_gpu_sample import check, run_gpu

    check(run_gpu(sampler, w["logits"], w["params"], recent=w["recent"], topk_cap=40), want, 40)
    sampler.reset_workspace()
    torch.cuda.synchronize()
    for _ in range(2):
        check(run_gpu(sampler, w["logits"], w["params"], recent=w["recent"], topk_cap=40), want, 40)


def test_noalloc_scratch_reset():
    """tms_workspace_reset(NULL) resets the current device's static scratch."""
    import torch

    lib = smod.load_library()
    s = torch.cuda.current_stream(0).cuda_stream
    assert lib.tms_workspace_reset(None, C.c_void_p(s)) == 0
    torch.cuda.synchronize()
