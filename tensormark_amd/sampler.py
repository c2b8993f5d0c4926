"""Python host side of the MI355X sampler: ctypes over libtmsample_hip.so.

Mirrors the reference sampler's interface (tensormark/tmsample.h:31-35 Opts,
52-63 apply_repeat_penalty, 173-200 sample) for batched device tensors:
``Opts`` carries the same three knobs, ``RowParams`` adds the per-row
penalties, min-p and the Philox seed/offset, and ``Sampler.sample`` runs the
composition of sample_token (tensormark/llama_chat.cpp:146-153) with the
grammar restriction in front (llama_chat.cpp:184-209) in one HIP launch.

PyTorch only supplies device memory and the stream.  There is no fallback:
if the HIP library is missing or no GPU is present, calls raise.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtmsample_hip.so")

TMS_OK = 0
ROWS_ANY, ROWS_TOPK, ROWS_SPARSE_MASK = 0, 1, 2
ROW_OK, ROW_BAD_PARAMS, ROW_ALL_MASKED, ROW_NONFINITE, ROW_UNSUPPORTED = 0, 1, 2, 3, 4
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

# Every symbol include/tmsample_hip.h declares.
EXPORTS = (
    "tms_abi_version",
    "tms_status_string",
    "tms_create",
    "tms_destroy",
    "tms_workspace_bytes",
    "tms_sample_batch",
    "tms_sample_batch_noalloc",
    "tms_spec_verify",
    "tms_workspace_reset",
    "tms_debug_ordering",
    "tms_debug_philox",
    "tms_debug_exp",
    "tms_host_repeat_penalty",
    "tms_host_no_repeat_ngram",
    "tms_host_dry",
    "tms_dry_scale_table",
    "tms_grammar_parse",
    "tms_grammar_free",
    "tms_grammar_rule_count",
    "tms_grammar_start",
    "tms_grammar_advance",
    "tms_grammar_can_end",
    "tms_grammar_accepts",
    "tms_gstate_copy",
    "tms_gstate_free",
    "tms_gstate_equal",
    "tms_vocab_create",
    "tms_vocab_free",
    "tms_vocab_node_count",
    "tms_vocab_allowed",
    "tms_vocab_mask",
    "tms_vocab_consume",
    "tms_vocab_clear_cache",
    "tms_token_table_spm",
    "tms_token_table_bpe",
    "tms_token_table_free",
    "tms_token_table_size",
    "tms_token_table_bytes",
    "tms_token_table_ws_only",
    "tms_vocab_from_table",
    "tms_filter_create",
    "tms_filter_free",
    "tms_filter_reset",
    "tms_filter_mask",
    "tms_filter_consume",
    "tms_filter_complete",
    "tms_filter_done",
    "tms_filter_stall",
    "tms_mask_pipe_create",
    "tms_mask_pipe_free",
    "tms_mask_pipe_set_row",
    "tms_mask_pipe_submit",
    "tms_mask_pipe_acquire",
    "tms_mask_pipe_release",
    "tms_token_slot_create",
    "tms_token_slot_free",
    "tms_token_slot_device",
    "tms_token_slot_capacity",
    "tms_token_slot_fill",
    "tms_token_slot_peek",
    "tms_embed_gather",
)


class RowParams(C.Structure):
    """tms_row_params: tmsample::Opts (tmsample.h:31-35) plus the extensions."""

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
        ("temperature", "<f4"), ("top_k", "<i4"), ("top_p", "<f4"), ("min_p", "<f4"),
        ("repeat_penalty", "<f4"), ("repeat_last_n", "<i4"), ("frequency_penalty", "<f4"),
        ("presence_penalty", "<f4"), ("greedy", "<i4"), ("flags", "<u4"), ("seed", "<u8"),
        ("offset", "<u8"),
    ]
)
assert ROW_DTYPE.itemsize == C.sizeof(RowParams) == 56


HISTORY_DTYPE = np.dtype(
    [
        ("no_repeat_ngram", "<i4"), ("dry_multiplier", "<f4"), ("dry_base", "<f4"),
        ("dry_allowed_length", "<i4"), ("dry_penalty_last_n", "<i4"), ("reserved", "<i4"),
    ]
)
HISTORY_MAX_IDS = 4096   # TMS_HISTORY_MAX_IDS
DRY_MAX_WINDOW = 8192    # TMS_DRY_MAX_WINDOW


def make_history(B: int, *, no_repeat_ngram=0, dry_multiplier=0.0, dry_base=1.75,
                 dry_allowed_length=2, dry_penalty_last_n=256) -> np.ndarray:
    """A [B] HISTORY_DTYPE array (tms_history_params): the n-gram ban and
    tmsample::DryOpts (tensormark/tmsample.h:141-146, same defaults);
    scalars broadcast, arrays give per-row values."""
    h = np.zeros(B, HISTORY_DTYPE)
    h["no_repeat_ngram"] = no_repeat_ngram
    h["dry_multiplier"] = dry_multiplier
    h["dry_base"] = dry_base
    h["dry_allowed_length"] = dry_allowed_length
    h["dry_penalty_last_n"] = dry_penalty_last_n
    return h


def dry_scale_table(history: np.ndarray) -> np.ndarray:
    """[B, n] float32 of tms_sample_args.dry_scale for a HISTORY_DTYPE array:
    row b holds std::pow(dry_base_b, (float)k) for k < n, from this host's C
    library through tms_dry_scale_table (the reference's own arithmetic,
    tensormark/tmsample.h:168); n covers every row's DRY window."""
    lib = load_library()
    h = np.asarray(history, HISTORY_DTYPE)
    n = int(min(max(1, int(np.max(h["dry_penalty_last_n"], initial=1))), DRY_MAX_WINDOW))
    out = np.zeros((len(h), n), np.float32)
    for b in range(len(h)):
        if h["dry_multiplier"][b] > 0.0:
            _check(lib.tms_dry_scale_table(C.c_float(float(h["dry_base"][b])), n,
                                           out[b].ctypes.data_as(C.POINTER(C.c_float))),
                   "tms_dry_scale_table")
    return out


@dataclasses.dataclass
class Opts:
    """tmsample::Opts (tensormark/tmsample.h:31-35), same defaults."""

    temperature: float = 0.7
    top_k: int = 40
    top_p: float = 0.9


def make_params(B: int, opts: Optional[Opts] = None, *, min_p=0.0, repeat_penalty=1.0,
                repeat_last_n=64, frequency_penalty=0.0, presence_penalty=0.0, greedy=False,
                seed=1234, offset=0) -> np.ndarray:
    """A [B] ROW_DTYPE array; scalars broadcast, arrays give per-row values."""
    o = opts or Opts()
    p = np.zeros(B, ROW_DTYPE)
    p["temperature"] = o.temperature
    p["top_k"] = o.top_k
    p["top_p"] = o.top_p
    p["min_p"] = min_p
    p["repeat_penalty"] = repeat_penalty
    p["repeat_last_n"] = repeat_last_n
    p["frequency_penalty"] = frequency_penalty
    p["presence_penalty"] = presence_penalty
    p["greedy"] = np.asarray(greedy).astype(np.int32)
    p["seed"] = seed
    p["offset"] = offset
    return p


class SampleArgs(C.Structure):
    _fields_ = [
        ("logits", C.c_void_p), ("dtype", C.c_int32), ("batch", C.c_int32),
        ("vocab", C.c_int32), ("topk_cap", C.c_int32), ("row_stride", C.c_int64),
        ("params", C.c_void_p), ("recent", C.c_void_p), ("n_recent", C.c_void_p),
        ("recent_stride", C.c_int64), ("mask", C.c_void_p), ("mask_stride", C.c_int64),
        ("draws", C.c_void_p), ("out_tokens", C.c_void_p), ("out_status", C.c_void_p),
        ("out_keep", C.c_void_p), ("out_topk_ids", C.c_void_p), ("out_topk_probs", C.c_void_p),
        ("row_kinds", C.c_uint32), ("reserved", C.c_uint32),
        ("history", C.c_void_p), ("dry_breaker", C.c_void_p),
        ("dry_scale", C.c_void_p), ("dry_scale_stride", C.c_int64),
    ]


class SpecArgs(C.Structure):
    _fields_ = [
        ("target_logits", C.c_void_p), ("draft_logits", C.c_void_p), ("dtype", C.c_int32),
        ("batch", C.c_int32), ("k", C.c_int32), ("vocab", C.c_int32),
        ("draft_tokens", C.c_void_p), ("params", C.c_void_p), ("draws", C.c_void_p),
        ("out_accepted", C.c_void_p), ("out_token", C.c_void_p), ("out_status", C.c_void_p),
    ]


_LIB = None


def row_kinds_of(params: np.ndarray) -> int:
    """ROWS_TOPK when every row is greedy or has 1 <= top_k <= 128 (the rows
    the library's top-k kernel serves), else ROWS_ANY."""
    p = np.asarray(params)
    ok = (p["greedy"] != 0) | ((p["top_k"] >= 1) & (p["top_k"] <= 128))
    return ROWS_TOPK if bool(np.all(ok)) else ROWS_ANY


SPARSE_MAX_IDS = 2048   # TMS_SPARSE_MAX_IDS


def mask_is_sparse(mask: np.ndarray) -> bool:
    """Whether every row of a host [B, W] uint32 allowed-bit mask allows at
    most SPARSE_MAX_IDS ids: the caller's ground for ROWS_SPARSE_MASK (a
    grammar engine knows each row's allowed count when it builds the mask)."""
    m = np.ascontiguousarray(mask, dtype=np.uint32)
    counts = np.unpackbits(m.view(np.uint8), axis=1).sum(axis=1)
    return bool(np.all(counts <= SPARSE_MAX_IDS))


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Load the HIP library; raises if it was not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} not built: run python -m tensormark_amd.build")
        lib = C.CDLL(path)
        lib.tms_status_string.restype = C.c_char_p
        lib.tms_workspace_bytes.restype = C.c_size_t
        lib.tms_create.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
        lib.tms_destroy.argtypes = [C.c_void_p]
        lib.tms_workspace_bytes.argtypes = [C.c_void_p]
        lib.tms_sample_batch.argtypes = [C.c_void_p, C.POINTER(SampleArgs), C.c_void_p]
        lib.tms_sample_batch_noalloc.argtypes = [C.POINTER(SampleArgs), C.c_void_p]
        lib.tms_spec_verify.argtypes = [C.c_void_p, C.POINTER(SpecArgs), C.c_void_p]
        lib.tms_debug_philox.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
        lib.tms_debug_ordering.argtypes = [C.c_int, C.POINTER(C.c_int32)]
        lib.tms_workspace_reset.argtypes = [C.c_void_p, C.c_void_p]
        lib.tms_debug_exp.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
        fp, ip = C.POINTER(C.c_float), C.POINTER(C.c_int32)
        lib.tms_host_repeat_penalty.argtypes = [fp, C.c_int, ip, C.c_int, C.c_int, C.c_float]
        lib.tms_host_no_repeat_ngram.argtypes = [fp, C.c_int, ip, C.c_int, C.c_int]
        lib.tms_dry_scale_table.argtypes = [C.c_float, C.c_int, fp]
        lib.tms_host_dry.argtypes = [fp, C.c_int, ip, C.c_int, C.c_float, C.c_float, C.c_int,
                                     C.c_int, C.c_void_p]
        for f in (lib.tms_host_repeat_penalty, lib.tms_host_no_repeat_ngram, lib.tms_host_dry):
            f.restype = None
        vp = C.c_void_p
        lib.tms_grammar_parse.restype = vp
        lib.tms_grammar_parse.argtypes = [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t]
        lib.tms_grammar_free.argtypes = [vp]
        lib.tms_grammar_free.restype = None
        lib.tms_grammar_rule_count.argtypes = [vp]
        lib.tms_grammar_start.restype = vp
        lib.tms_grammar_start.argtypes = [vp]
        lib.tms_grammar_advance.argtypes = [vp, vp, C.c_ubyte]
        lib.tms_grammar_can_end.argtypes = [vp, vp]
        lib.tms_grammar_accepts.argtypes = [vp, C.c_char_p, C.c_size_t]
        lib.tms_gstate_copy.restype = vp
        lib.tms_gstate_copy.argtypes = [vp]
        lib.tms_gstate_free.argtypes = [vp]
        lib.tms_gstate_free.restype = None
        lib.tms_gstate_equal.argtypes = [vp, vp]
        lib.tms_vocab_create.restype = vp
        lib.tms_vocab_create.argtypes = [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t), C.c_int,
                                         C.c_int, vp]
        lib.tms_vocab_free.argtypes = [vp]
        lib.tms_vocab_free.restype = None
        lib.tms_vocab_node_count.argtypes = [vp]
        lib.tms_vocab_allowed.argtypes = [vp, vp, vp, C.c_int]
        lib.tms_vocab_mask.argtypes = [vp, vp, vp, C.c_int]
        lib.tms_vocab_consume.argtypes = [vp, vp, vp, C.c_int]
        lib.tms_vocab_clear_cache.argtypes = [vp]
        lib.tms_vocab_clear_cache.restype = None
        cp, sp = C.POINTER(C.c_char_p), C.POINTER(C.c_size_t)
        lib.tms_token_table_spm.restype = vp
        lib.tms_token_table_spm.argtypes = [cp, sp, vp, C.c_int, C.c_char_p, C.c_size_t]
        lib.tms_token_table_bpe.restype = vp
        lib.tms_token_table_bpe.argtypes = [cp, sp, C.c_int, C.c_char_p, C.c_size_t]
        lib.tms_token_table_free.argtypes = [vp]
        lib.tms_token_table_free.restype = None
        lib.tms_token_table_size.argtypes = [vp]
        lib.tms_token_table_bytes.argtypes = [vp, C.c_int, C.POINTER(C.c_void_p), sp]
        lib.tms_token_table_ws_only.argtypes = [vp, C.c_int]
        lib.tms_vocab_from_table.restype = vp
        lib.tms_vocab_from_table.argtypes = [vp, vp, C.c_int, vp]
        lib.tms_filter_create.restype = vp
        lib.tms_filter_create.argtypes = [vp, vp, vp]
        lib.tms_filter_free.argtypes = [vp]
        lib.tms_filter_free.restype = None
        for f in (lib.tms_filter_reset, lib.tms_filter_done, lib.tms_filter_stall):
            f.argtypes = [vp]
        lib.tms_filter_mask.argtypes = [vp, vp, C.c_int]
        lib.tms_filter_consume.argtypes = [vp, C.c_int]
        lib.tms_filter_complete.argtypes = [vp, C.c_int]
        lib.tms_mask_pipe_create.restype = vp
        lib.tms_mask_pipe_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int]
        lib.tms_mask_pipe_free.argtypes = [vp]
        lib.tms_mask_pipe_free.restype = None
        lib.tms_mask_pipe_set_row.argtypes = [vp, C.c_int, vp]
        lib.tms_mask_pipe_submit.argtypes = [vp, vp]
        lib.tms_mask_pipe_acquire.argtypes = [vp, vp, C.POINTER(C.c_void_p), vp]
        lib.tms_mask_pipe_release.argtypes = [vp, vp]
        lib.tms_token_slot_create.restype = vp
        lib.tms_token_slot_create.argtypes = [C.c_int, C.c_int]
        lib.tms_token_slot_free.argtypes = [vp]
        lib.tms_token_slot_free.restype = None
        lib.tms_token_slot_device.restype = vp
        lib.tms_token_slot_device.argtypes = [vp]
        lib.tms_token_slot_capacity.argtypes = [vp]
        lib.tms_token_slot_fill.argtypes = [vp, C.c_int32]
        lib.tms_token_slot_peek.restype = C.c_int32
        lib.tms_token_slot_peek.argtypes = [vp, C.c_int]
        lib.tms_embed_gather.argtypes = [vp, C.c_int, C.c_int64, C.c_int64, vp, C.c_int, vp, vp, vp]
        _LIB = lib
    return _LIB


def _check(rc: int, what: str) -> None:
    if rc != TMS_OK:
        msg = load_library().tms_status_string(rc).decode()
        raise RuntimeError(f"{what} failed: {msg} ({rc})")


def _torch():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("tensormark_amd needs a HIP device; none is visible")
    return torch


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _dtype_code(t) -> int:
    import torch

    return {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16,
            torch.bfloat16: DTYPE_BF16}[t.dtype]


class Sampler:
    """A context (device workspace) for batches up to max_batch x max_vocab."""

    def __init__(self, max_batch: int, max_vocab: int, device: int = 0, kernel: str = "auto"):
        if kernel not in ("auto", "general"):
            raise ValueError("kernel must be 'auto' or 'general'")
        torch = _torch()
        self.torch = torch
        self.kernel = kernel
        self.lib = load_library()
        self.device = device
        h = C.c_void_p()
        _check(self.lib.tms_create(device, max_batch, max_vocab, C.byref(h)), "tms_create")
        self.handle = h

    def close(self) -> None:
        if self.handle:
            self.lib.tms_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset_workspace(self, stream=None) -> None:
        """Return the workspace to its creation state (zeroed counters and
        lists, all-ones mask row) on ``stream``.  Recovery after a call that
        reported TMS_ROW_INTERNAL; not for use inside graph capture."""
        import torch
        s = stream if stream is not None else torch.cuda.current_stream(self.device).cuda_stream
        _check(self.lib.tms_workspace_reset(self.handle, C.c_void_p(s)), "tms_workspace_reset")

    @property
    def workspace_bytes(self) -> int:
        return int(self.lib.tms_workspace_bytes(self.handle))

    def params_tensor(self, params: np.ndarray):
        raw = np.ascontiguousarray(params, ROW_DTYPE).view(np.uint8)
        return self.torch.from_numpy(raw.copy()).to(f"cuda:{self.device}")

    def sample(self, logits, params, *, recent=None, n_recent=None, mask=None, draws=None,
               topk_cap: int = 0, out=None, stream=None, row_kinds=None, noalloc=False,
               history=None, dry_breaker=None, dry_scale=None):
        """Sample one token per row of ``logits`` ([B, V] fp32/fp16/bf16, cuda).

        ``params`` is a device uint8 tensor from params_tensor() (or a numpy
        ROW_DTYPE array, uploaded here).  ``row_kinds`` is the hint of
        tms_sample_args (ROWS_ANY / ROWS_TOPK / ROWS_SPARSE_MASK); by default it is derived from
        numpy params (ROWS_ANY for device params), and a Sampler created with
        kernel="general" always passes ROWS_ANY.  ``noalloc`` takes the
        context-free entry point tms_sample_batch_noalloc (its static
        workspace) instead of this context's.  ``history`` (a
        HISTORY_DTYPE array from make_history, or a device uint8 tensor of
        one) turns on the n-gram ban and DRY, with ``dry_breaker`` an
        optional device uint8 [V] breaker table and ``dry_scale`` the
        [B, n] table of DRY scales (dry_scale_table(); built here from a
        numpy ``history`` when not given; pass False for the library's own
        correctly rounded powers).  Returns a dict of device
        tensors: tokens, status, keep, and topk_ids/topk_probs when
        topk_cap > 0.
        """
        torch = self.torch
        if row_kinds is None:
            row_kinds = ROWS_ANY
            if self.kernel == "auto" and isinstance(params, np.ndarray):
                row_kinds = row_kinds_of(params)
        if isinstance(params, np.ndarray):
            params = self.params_tensor(params)
        if isinstance(history, np.ndarray) and dry_scale is None:
            dry_scale = dry_scale_table(history)
        if dry_scale is False:
            dry_scale = None
        if isinstance(dry_scale, np.ndarray):
            dry_scale = torch.from_numpy(np.ascontiguousarray(dry_scale, np.float32)).to(
                f"cuda:{self.device}")
        if isinstance(history, np.ndarray):
            raw = np.ascontiguousarray(history, HISTORY_DTYPE).view(np.uint8)
            history = torch.from_numpy(raw.copy()).to(f"cuda:{self.device}")
        B, V = logits.shape
        dev = logits.device
        if out is None:
            out = {
                "tokens": torch.empty(B, dtype=torch.int32, device=dev),
                "status": torch.empty(B, dtype=torch.int32, device=dev),
                "keep": torch.empty(B, dtype=torch.int32, device=dev),
            }
            if topk_cap:
                out["topk_ids"] = torch.empty((B, topk_cap), dtype=torch.int32, device=dev)
                out["topk_probs"] = torch.empty((B, topk_cap), dtype=torch.float32, device=dev)
        a = self.make_args(logits, params, recent=recent, n_recent=n_recent, mask=mask,
                           draws=draws, topk_cap=topk_cap, out=out, row_kinds=row_kinds)
        a.history = _ptr(history)
        a.dry_breaker = _ptr(dry_breaker)
        a.dry_scale = _ptr(dry_scale)
        a.dry_scale_stride = dry_scale.shape[1] if dry_scale is not None else 0
        s = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
        if noalloc:
            _check(self.lib.tms_sample_batch_noalloc(C.byref(a), C.c_void_p(s)),
                   "tms_sample_batch_noalloc")
        else:
            _check(self.lib.tms_sample_batch(self.handle, C.byref(a), C.c_void_p(s)),
                   "tms_sample_batch")
        return out

    def make_args(self, logits, params, *, recent=None, n_recent=None, mask=None, draws=None,
                  topk_cap=0, out=None, row_kinds=ROWS_ANY) -> SampleArgs:
        B, V = logits.shape
        a = SampleArgs()
        a.logits = logits.data_ptr()
        a.dtype = _dtype_code(logits)
        a.batch = B
        a.vocab = V
        a.row_stride = logits.stride(0)
        a.params = params.data_ptr()
        a.recent = _ptr(recent)
        a.recent_stride = recent.shape[1] if recent is not None else 0
        a.n_recent = _ptr(n_recent)
        if isinstance(mask, tuple):   # (device address, words per row), e.g. from a MaskPipe
            a.mask, a.mask_stride = mask
        else:
            a.mask = _ptr(mask)
            a.mask_stride = mask.shape[1] if mask is not None else 0
        a.draws = _ptr(draws)
        a.out_tokens = out["tokens"].data_ptr()
        a.out_status = out["status"].data_ptr()
        a.out_keep = _ptr(out.get("keep"))
        a.topk_cap = topk_cap
        a.out_topk_ids = _ptr(out.get("topk_ids")) if topk_cap else None
        a.out_topk_probs = _ptr(out.get("topk_probs")) if topk_cap else None
        a.row_kinds = row_kinds
        return a

    def spec_verify(self, target, draft, draft_tokens, params, *, draws=None, stream=None):
        """Speculative verify: target [B, k+1, V], draft [B, k, V], tokens [B, k]."""
        torch = self.torch
        if isinstance(params, np.ndarray):
            params = self.params_tensor(params)
        B, k1, V = target.shape
        dev = target.device
        out = {
            "accepted": torch.empty(B, dtype=torch.int32, device=dev),
            "token": torch.empty(B, dtype=torch.int32, device=dev),
            "status": torch.empty(B, dtype=torch.int32, device=dev),
        }
        a = SpecArgs()
        a.target_logits = target.data_ptr()
        a.draft_logits = draft.data_ptr()
        a.dtype = _dtype_code(target)
        a.batch = B
        a.k = k1 - 1
        a.vocab = V
        a.draft_tokens = draft_tokens.data_ptr()
        a.params = params.data_ptr()
        a.draws = _ptr(draws)
        a.out_accepted = out["accepted"].data_ptr()
        a.out_token = out["token"].data_ptr()
        a.out_status = out["status"].data_ptr()
        s = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
        _check(self.lib.tms_spec_verify(self.handle, C.byref(a), C.c_void_p(s)),
               "tms_spec_verify")
        return out


def _f32_row(row):
    assert isinstance(row, np.ndarray) and row.dtype == np.float32 and row.flags.c_contiguous
    return row.ctypes.data_as(C.POINTER(C.c_float))


def _ids(recent):
    r = np.ascontiguousarray(recent, np.int32)
    return r, r.ctypes.data_as(C.POINTER(C.c_int32))


def apply_repeat_penalty(row, recent, window, penalty):
    """tmsample::apply_repeat_penalty (tmsample.h:52-63) on a host fp32 row, in place."""
    r, rp = _ids(recent)
    load_library().tms_host_repeat_penalty(_f32_row(row), row.size, rp, r.size, window, penalty)


def apply_no_repeat_ngram(row, recent, ngram):
    """tmsample::apply_no_repeat_ngram (tmsample.h:81-114) on a host fp32 row, in place."""
    r, rp = _ids(recent)
    load_library().tms_host_no_repeat_ngram(_f32_row(row), row.size, rp, r.size, ngram)


def apply_dry(row, recent, multiplier=0.0, base=1.75, allowed_length=2, penalty_last_n=256,
              is_breaker=None):
    """tmsample::apply_dry (tmsample.h:148-170) on a host fp32 row, in place."""
    r, rp = _ids(recent)
    brk = None
    if is_breaker is not None:
        brk = np.ascontiguousarray(is_breaker, np.uint8)
    load_library().tms_host_dry(_f32_row(row), row.size, rp, r.size, multiplier, base,
                                allowed_length, penalty_last_n,
                                None if brk is None else brk.ctypes.data_as(C.c_void_p))


def debug_philox(in6, out4=None):
    """Device Philox4x32-10 on a [n, 6] uint32 cuda tensor (as int32)."""
    torch = _torch()
    n = in6.shape[0]
    if out4 is None:
        out4 = torch.empty((n, 4), dtype=torch.int32, device=in6.device)
    s = torch.cuda.current_stream(in6.device).cuda_stream
    _check(load_library().tms_debug_philox(in6.data_ptr(), out4.data_ptr(), n, C.c_void_p(s)),
           "tms_debug_philox")
    return out4


def debug_exp(x, which: int):
    torch = _torch()
    out = torch.empty_like(x)
    s = torch.cuda.current_stream(x.device).cuda_stream
    _check(load_library().tms_debug_exp(x.data_ptr(), out.data_ptr(), x.numel(), which,
                                        C.c_void_p(s)), "tms_debug_exp")
    return out
