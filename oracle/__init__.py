"""ctypes bindings for the CPU checkers (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this package, and only to check or time against.  The product
library never loads it.

``oracle()`` loads ``oracle/_build/libtms_oracle.so`` (the C restatement of
tensormark/tmsample.h, tms_oracle.c); ``reference()`` loads
``oracle/_ref/libtmsample_ref.so`` (the reference's own tmsample.h compiled by
oracle/Makefile), or returns None when it was not built.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libtms_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtmsample_ref.so")


class RowParams(C.Structure):
    """Same layout as tms_row_params (include/tmsample_hip.h)."""

    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_int32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("repeat_penalty", C.c_float),
        ("repeat_last_n", C.c_int32),
        ("frequency_penalty", C.c_float),
        ("presence_penalty", C.c_float),
        ("greedy", C.c_int32),
        ("flags", C.c_uint32),
        ("seed", C.c_uint64),
        ("offset", C.c_uint64),
    ]


ROW_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_k", "<i4"),
        ("top_p", "<f4"),
        ("min_p", "<f4"),
        ("repeat_penalty", "<f4"),
        ("repeat_last_n", "<i4"),
        ("frequency_penalty", "<f4"),
        ("presence_penalty", "<f4"),
        ("greedy", "<i4"),
        ("flags", "<u4"),
        ("seed", "<u8"),
        ("offset", "<u8"),
    ]
)
assert ROW_DTYPE.itemsize == C.sizeof(RowParams) == 56

HISTORY_DTYPE = np.dtype(
    [
        ("no_repeat_ngram", "<i4"),
        ("dry_multiplier", "<f4"),
        ("dry_base", "<f4"),
        ("dry_allowed_length", "<i4"),
        ("dry_penalty_last_n", "<i4"),
        ("reserved", "<i4"),
    ]
)


def build() -> None:
    """Compile the checkers (oracle/_ref only where the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _p(a, t):
    return None if a is None else a.ctypes.data_as(C.POINTER(t))


_ORACLE = None
_REF = None


def oracle() -> "Oracle":
    global _ORACLE
    if _ORACLE is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        _ORACLE = Oracle(C.CDLL(ORACLE_SO))
    return _ORACLE


def reference():
    global _REF
    if _REF is None and os.path.exists(REF_SO):
        _REF = Ref(C.CDLL(REF_SO))
    return _REF


class Oracle:
    def __init__(self, lib):
        self.lib = lib
        lib.tmo_canonical.restype = C.c_double
        lib.tmo_canonical.argtypes = [C.c_uint32, C.c_uint32]
        lib.tmo_exp64.restype = C.c_double
        lib.tmo_exp64.argtypes = [C.c_double]
        lib.tmo_q44.restype = C.c_int64
        lib.tmo_q44.argtypes = [C.c_double]

    def philox(self, ctr, key):
        c = (C.c_uint32 * 4)(*ctr)
        k = (C.c_uint32 * 2)(*key)
        o = (C.c_uint32 * 4)()
        self.lib.tmo_philox4x32_10(c, k, o)
        return list(o)

    def row_words(self, seed, offset, stream=0):
        w0, w1 = C.c_uint32(), C.c_uint32()
        self.lib.tmo_row_words(C.c_uint64(seed), C.c_uint64(offset), C.c_uint32(stream),
                               C.byref(w0), C.byref(w1))
        return w0.value, w1.value

    def canonical(self, w0, w1):
        return self.lib.tmo_canonical(w0, w1)

    def exp64(self, x):
        return self.lib.tmo_exp64(x)

    def apply_mask(self, row, mask):
        row = np.ascontiguousarray(row, np.float32).copy()
        m = np.ascontiguousarray(mask, np.uint32)
        self.lib.tmo_apply_mask(_p(row, C.c_float), C.c_int(row.size), _p(m, C.c_uint32))
        return row

    def apply_repeat_penalty(self, row, recent, window, penalty):
        row = np.ascontiguousarray(row, np.float32).copy()
        r = np.ascontiguousarray(recent, np.int32)
        self.lib.tmo_apply_repeat_penalty(_p(row, C.c_float), C.c_int(row.size),
                                          _p(r, C.c_int32), C.c_int(r.size),
                                          C.c_int(window), C.c_float(penalty))
        return row

    def apply_freq_presence(self, row, recent, window, freq, presence):
        row = np.ascontiguousarray(row, np.float32).copy()
        r = np.ascontiguousarray(recent, np.int32)
        self.lib.tmo_apply_freq_presence(_p(row, C.c_float), C.c_int(row.size),
                                         _p(r, C.c_int32), C.c_int(r.size), C.c_int(window),
                                         C.c_float(freq), C.c_float(presence))
        return row

    def no_repeat_ngram(self, row, recent, ngram):
        row = np.ascontiguousarray(row, np.float32).copy()
        r = np.ascontiguousarray(recent, np.int32)
        self.lib.tmo_no_repeat_ngram(_p(row, C.c_float), C.c_int(row.size), _p(r, C.c_int32),
                                     C.c_int(r.size), C.c_int(ngram))
        return row

    def dry(self, row, recent, multiplier, base, allowed_length, penalty_last_n, is_breaker=None):
        row = np.ascontiguousarray(row, np.float32).copy()
        r = np.ascontiguousarray(recent, np.int32)
        brk = None if is_breaker is None else np.ascontiguousarray(is_breaker, np.uint8)
        self.lib.tmo_dry(_p(row, C.c_float), C.c_int(row.size), _p(r, C.c_int32), C.c_int(r.size),
                         C.c_float(multiplier), C.c_float(base), C.c_int(allowed_length),
                         C.c_int(penalty_last_n), _p(brk, C.c_uint8))
        return row

    def sample_row(self, row, params: RowParams, w0, w1, topk_cap=0):
        row = np.ascontiguousarray(row, np.float32)
        tok, keep = C.c_int32(), C.c_int32()
        ids = np.full(max(topk_cap, 1), -1, np.int32)
        probs = np.zeros(max(topk_cap, 1), np.float32)
        st = self.lib.tmo_sample_row(_p(row, C.c_float), C.c_int(row.size), C.byref(params),
                                     C.c_uint32(w0), C.c_uint32(w1), C.byref(tok),
                                     C.byref(keep), _p(ids, C.c_int32), _p(probs, C.c_float),
                                     C.c_int(topk_cap))
        return st, tok.value, keep.value, ids[:topk_cap], probs[:topk_cap]

    def sample_batch(self, logits, params, recent=None, n_recent=None, mask=None, draws=None,
                     topk_cap=0, history=None, dry_breaker=None):
        """logits: float32 [B, V]; params: ROW_DTYPE [B]; history: HISTORY_DTYPE
        [B] or None (then no n-gram ban or DRY).  Returns a dict."""
        logits = np.ascontiguousarray(logits, np.float32)
        B, V = logits.shape
        params = np.ascontiguousarray(params, ROW_DTYPE)
        rs = 0
        if recent is not None:
            recent = np.ascontiguousarray(recent, np.int32)
            rs = recent.shape[1]
        if n_recent is not None:
            n_recent = np.ascontiguousarray(n_recent, np.int32)
        ms = 0
        if mask is not None:
            mask = np.ascontiguousarray(mask, np.uint32)
            ms = mask.shape[1]
        if draws is not None:
            draws = np.ascontiguousarray(draws, np.uint32)
        tokens = np.zeros(B, np.int32)
        status = np.zeros(B, np.int32)
        keep = np.zeros(B, np.int32)
        cap = max(topk_cap, 1)
        ids = np.full((B, cap), -1, np.int32)
        probs = np.zeros((B, cap), np.float32)
        hp = None if history is None else np.ascontiguousarray(history, HISTORY_DTYPE)
        brk = None if dry_breaker is None else np.ascontiguousarray(dry_breaker, np.uint8)
        self.lib.tmo_sample_batch_h(
            _p(logits, C.c_float), C.c_int(B), C.c_int(V), C.c_int64(V),
            params.ctypes.data_as(C.c_void_p),
            None if hp is None else hp.ctypes.data_as(C.c_void_p), _p(brk, C.c_uint8),
            _p(recent, C.c_int32), _p(n_recent, C.c_int32),
            C.c_int64(rs), _p(mask, C.c_uint32), C.c_int64(ms), _p(draws, C.c_uint32),
            _p(tokens, C.c_int32), _p(status, C.c_int32), _p(keep, C.c_int32),
            _p(ids, C.c_int32), _p(probs, C.c_float), C.c_int(topk_cap))
        return {"tokens": tokens, "status": status, "keep": keep,
                "topk_ids": ids[:, :topk_cap], "topk_probs": probs[:, :topk_cap]}

    def spec_verify_seq(self, target, draft, draft_tokens, temperature, words):
        target = np.ascontiguousarray(target, np.float32)
        draft = np.ascontiguousarray(draft, np.float32)
        k, V = draft.shape
        xs = np.ascontiguousarray(draft_tokens, np.int32)
        w = np.ascontiguousarray(words, np.uint32).reshape(-1)
        acc, tok = C.c_int32(), C.c_int32()
        st = self.lib.tmo_spec_verify_seq(_p(target, C.c_float), _p(draft, C.c_float),
                                          C.c_int(V), C.c_int(k), _p(xs, C.c_int32),
                                          C.c_float(temperature), _p(w, C.c_uint32),
                                          C.byref(acc), C.byref(tok))
        return st, acc.value, tok.value

    def spec_weights(self, row, temperature):
        row = np.ascontiguousarray(row, np.float32)
        e = np.zeros(row.size, np.int64)
        Z = C.c_int64()
        m = C.c_float()
        st = self.lib.tmo_spec_weights(_p(row, C.c_float), C.c_int(row.size),
                                       C.c_float(temperature), _p(e, C.c_int64), C.byref(Z),
                                       C.byref(m))
        return st, e, Z.value, m.value


class Ref:
    """The reference's compiled tmsample.h (oracle/_ref)."""

    def __init__(self, lib):
        self.lib = lib
        lib.ref_canonical.restype = C.c_double
        lib.ref_canonical.argtypes = [C.c_uint32, C.c_uint32]
        lib.ref_bench.restype = C.c_double

    def canonical(self, w0, w1):
        return self.lib.ref_canonical(w0, w1)

    def no_repeat_ngram(self, row, recent, ngram):
        row = np.ascontiguousarray(row, np.float32).copy()
        r = np.ascontiguousarray(recent, np.int32)
        self.lib.ref_no_repeat_ngram(_p(row, C.c_float), C.c_int(row.size), _p(r, C.c_int32),
                                     C.c_int(r.size), C.c_int(ngram))
        return row

    def dry(self, row, recent, multiplier, base, allowed_length, penalty_last_n, is_breaker=None):
        row = np.ascontiguousarray(row, np.float32).copy()
        r = np.ascontiguousarray(recent, np.int32)
        brk = None if is_breaker is None else np.ascontiguousarray(is_breaker, np.uint8)
        self.lib.ref_dry(_p(row, C.c_float), C.c_int(row.size), _p(r, C.c_int32), C.c_int(r.size),
                         C.c_float(multiplier), C.c_float(base), C.c_int(allowed_length),
                         C.c_int(penalty_last_n), None if brk is None else _p(brk, C.c_uint8))
        return row

    def discrete(self, pr, w0, w1):
        pr = np.ascontiguousarray(pr, np.float64)
        used = C.c_int()
        r = self.lib.ref_discrete(_p(pr, C.c_double), C.c_int(pr.size), C.c_uint32(w0),
                                  C.c_uint32(w1), C.byref(used))
        return r, used.value

    def apply_repeat_penalty(self, row, recent, window, penalty):
        row = np.ascontiguousarray(row, np.float32).copy()
        r = np.ascontiguousarray(recent, np.int32)
        self.lib.ref_apply_repeat_penalty(_p(row, C.c_float), C.c_int(row.size),
                                          _p(r, C.c_int32), C.c_int(r.size), C.c_int(window),
                                          C.c_float(penalty))
        return row

    def sample(self, row, temperature, top_k, top_p, greedy, seed, recent=None, window=0,
               penalty=1.0, mask=None):
        """One sample_token step; returns (token, w0, w1, words consumed)."""
        row = np.ascontiguousarray(row, np.float32)
        r = None if recent is None else np.ascontiguousarray(recent, np.int32)
        m = None if mask is None else np.ascontiguousarray(mask, np.uint32)
        w0, w1, used = C.c_uint32(), C.c_uint32(), C.c_int()
        tok = self.lib.ref_sample(_p(row, C.c_float), C.c_int(row.size),
                                  C.c_float(temperature), C.c_int(top_k), C.c_float(top_p),
                                  C.c_int(int(greedy)), C.c_uint32(seed), _p(r, C.c_int32),
                                  C.c_int(0 if r is None else r.size), C.c_int(window),
                                  C.c_float(penalty), _p(m, C.c_uint32), C.byref(w0),
                                  C.byref(w1), C.byref(used))
        return tok, w0.value, w1.value, used.value

    def bench(self, logits, temperature, top_k, top_p, recent=None, window=0, penalty=1.0,
              mask=None, threads=1, reps=1, greedy=False):
        logits = np.ascontiguousarray(logits, np.float32)
        B, V = logits.shape
        r = None if recent is None else np.ascontiguousarray(recent, np.int32)
        m = None if mask is None else np.ascontiguousarray(mask, np.uint32)
        toks = np.zeros(B, np.int32)
        dt = self.lib.ref_bench(_p(logits, C.c_float), C.c_int(B), C.c_int(V),
                                C.c_float(temperature), C.c_int(top_k), C.c_float(top_p),
                                C.c_int(1 if greedy else 0), _p(r, C.c_int32), C.c_int(0 if r is None else r.shape[1]),
                                C.c_int(window), C.c_float(penalty), _p(m, C.c_uint32),
                                C.c_int(0 if m is None else m.shape[1]), C.c_int(threads),
                                C.c_int(reps), _p(toks, C.c_int32))
        return dt, toks
