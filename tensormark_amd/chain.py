"""Chained device-resident decode over the C ABI's token slot and embedding
gather: gpu_chain_begin / gpu_chain_poll / end (tensormark/llama.h:
6047-6130) for a batch of sequences.

    chain = Chain(sampler, embed, forward, batch=B, n_max=64)
    chain.begin(first_ids, n, params_per_step)   # every step enqueued now
    chain.poll(i, row)   # the id chosen at step i, or -1 while it is pending
    chain.end()          # wait; returns the [n, B] ids and statuses

Step i gathers the embeddings of step i-1's ids (the first step: of
first_ids) into x on the device, runs ``forward(x) -> logits`` (the
caller's model, enqueued on the current stream), and samples into a device
row of ids; the gather of step i+1 publishes those ids into the token slot,
so the host sees them land while later steps still run.
"""
from __future__ import annotations

import ctypes as C
from typing import Callable, Sequence

import numpy as np

from .sampler import Sampler, _check, _dtype_code, load_library


class TokenSlot:
    """Host memory the device writes: one int32 per (step, row), -1 until written."""

    def __init__(self, capacity: int, device: int = 0):
        h = load_library().tms_token_slot_create(device, capacity)
        if not h:
            raise RuntimeError("tms_token_slot_create failed")
        self._h = C.c_void_p(h)
        self.capacity = capacity

    def device_ptr(self, entry: int = 0) -> int:
        return load_library().tms_token_slot_device(self._h) + 4 * entry

    def fill(self, value: int = -1) -> None:
        _check(load_library().tms_token_slot_fill(self._h, value), "tms_token_slot_fill")

    def peek(self, i: int) -> int:
        return int(load_library().tms_token_slot_peek(self._h, i))

    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            load_library().tms_token_slot_free(h)
            self._h = None

    def __del__(self):
        self.close()


def embed_gather(table, tokens, x, slot_ptr=None, stream=None) -> None:
    """x[b] = table[tokens[b]] (device tensors; table [rows, dim]); with
    slot_ptr, also publish tokens into the slot entries from there.  table
    None: publish only."""
    import torch

    dev = tokens.device
    s = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
    if table is None:
        rc = load_library().tms_embed_gather(None, 0, 0, 0, C.c_void_p(tokens.data_ptr()),
                                             tokens.numel(), None, C.c_void_p(slot_ptr), C.c_void_p(s))
    else:
        rc = load_library().tms_embed_gather(C.c_void_p(table.data_ptr()), _dtype_code(table),
                                             table.shape[0], table.shape[1],
                                             C.c_void_p(tokens.data_ptr()), tokens.numel(),
                                             C.c_void_p(x.data_ptr()),
                                             None if slot_ptr is None else C.c_void_p(slot_ptr),
                                             C.c_void_p(s))
    _check(rc, "tms_embed_gather")


class Chain:
    def __init__(self, sampler: Sampler, embed, forward: Callable, batch: int, n_max: int):
        import torch

        self.torch = torch
        self.sampler, self.embed, self.forward = sampler, embed, forward
        self.B, self.n_max = batch, n_max
        dev = embed.device
        self.slot = TokenSlot(n_max * batch, device=dev.index or 0)
        self.ids = torch.empty((n_max, batch), dtype=torch.int32, device=dev)
        self.status = torch.empty((n_max, batch), dtype=torch.int32, device=dev)
        self.keep = torch.empty((n_max, batch), dtype=torch.int32, device=dev)
        self.x = torch.empty((batch, embed.shape[1]), dtype=embed.dtype, device=dev)
        self.n = 0

    def begin(self, first: np.ndarray, n: int, params: Sequence[np.ndarray], **sample_kw) -> None:
        """Enqueue n steps; params[i] is step i's ROW_DTYPE array."""
        torch = self.torch
        if not 1 <= n <= self.n_max or self.n:
            raise ValueError("chain: 1 <= n <= n_max, one chain at a time")
        self.slot.fill(-1)
        dev = self.embed.device
        cur = torch.from_numpy(np.ascontiguousarray(first, np.int32)).to(dev)
        ptabs = [self.sampler.params_tensor(p) for p in params[:n]]
        B = self.B
        for i in range(n):
            src = cur if i == 0 else self.ids[i - 1]
            embed_gather(self.embed, src, self.x,
                         None if i == 0 else self.slot.device_ptr((i - 1) * B))
            logits = self.forward(self.x)
            out = {"tokens": self.ids[i], "status": self.status[i], "keep": self.keep[i]}
            self.sampler.sample(logits, ptabs[i], out=out, **sample_kw)
        embed_gather(None, self.ids[n - 1], None, self.slot.device_ptr((n - 1) * B))
        self._hold = (cur, ptabs)
        self.n = n

    def poll(self, i: int, row: int = 0) -> int:
        """Step i's id for `row`, -1 while pending (-2: the row had no id)."""
        if not 0 <= i < self.n:
            return -1
        return self.slot.peek(i * self.B + row)

    def end(self):
        self.torch.cuda.synchronize(self.embed.device)
        n, self.n = self.n, 0
        return self.ids[:n].cpu().numpy(), self.status[:n].cpu().numpy()
