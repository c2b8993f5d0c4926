"""Python view of the host GBNF engine (tms_grammar_* / tms_vocab_* in the C
ABI), shaped like tmgbnf::Grammar / State / TokenMask (tensormark/gbnf.h:345-851).

    g = Grammar.parse(text)            # raises GrammarError on a bad grammar
    s = g.start(); g.advance(s, byte); g.can_end(s); g.accepts(b"...")
    m = TokenMask(g, token_bytes, eos=2, skip=None)
    m.allowed(s) -> list of ids;  m.mask(s, V) -> uint32 words for the sampler
    m.consume(s, id) -> bool
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np

from .sampler import load_library


class GrammarError(ValueError):
    pass


class State:
    """A parse state (value semantics: copy() before a speculative walk)."""

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)

    def copy(self) -> "State":
        return State(load_library().tms_gstate_copy(self._h))

    def __eq__(self, other) -> bool:
        return isinstance(other, State) and bool(load_library().tms_gstate_equal(self._h, other._h))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            load_library().tms_gstate_free(h)
            self._h = None


class Grammar:
    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)

    @classmethod
    def parse(cls, text) -> "Grammar":
        data = text.encode() if isinstance(text, str) else bytes(text)
        err = C.create_string_buffer(512)
        h = load_library().tms_grammar_parse(data, len(data), err, len(err))
        if not h:
            raise GrammarError(err.value.decode(errors="replace"))
        return cls(h)

    def rule_count(self) -> int:
        return load_library().tms_grammar_rule_count(self._h)

    def start(self) -> State:
        return State(load_library().tms_grammar_start(self._h))

    def advance(self, s: State, byte: int) -> bool:
        return bool(load_library().tms_grammar_advance(self._h, s._h, byte))

    def can_end(self, s: State) -> bool:
        return bool(load_library().tms_grammar_can_end(self._h, s._h))

    def accepts(self, text) -> bool:
        data = text.encode() if isinstance(text, str) else bytes(text)
        return bool(load_library().tms_grammar_accepts(self._h, data, len(data)))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            load_library().tms_grammar_free(h)
            self._h = None


class TokenMask:
    """Allowed token ids per parse state over a vocabulary of byte strings."""

    def __init__(self, g: Grammar, tokens: Sequence[bytes], eos: int = -1,
                 skip: Optional[Sequence[int]] = None):
        self.g = g
        toks = [t.encode() if isinstance(t, str) else bytes(t) for t in tokens]
        n = len(toks)
        self._bufs = (C.c_char_p * max(n, 1))(*toks)
        self._lens = (C.c_size_t * max(n, 1))(*[len(t) for t in toks])
        sk = None
        if skip is not None:
            self._skip = np.ascontiguousarray(np.asarray(skip, np.uint8))
            sk = self._skip.ctypes.data_as(C.c_void_p)
        h = load_library().tms_vocab_create(g._h, self._bufs, self._lens, n, eos, sk)
        if not h:
            raise ValueError("tms_vocab_create failed")
        self._h = C.c_void_p(h)
        self.n = n

    def node_count(self) -> int:
        return load_library().tms_vocab_node_count(self._h)

    def allowed(self, s: State) -> list:
        lib = load_library()
        n = lib.tms_vocab_allowed(self._h, s._h, None, 0)
        out = np.empty(max(n, 1), np.int32)
        lib.tms_vocab_allowed(self._h, s._h, out.ctypes.data_as(C.c_void_p), n)
        return out[:n].tolist()

    def mask(self, s: State, vocab: int, out: Optional[np.ndarray] = None) -> np.ndarray:
        words = (vocab + 31) // 32
        if out is None:
            out = np.empty(words, np.uint32)
        load_library().tms_vocab_mask(self._h, s._h, out.ctypes.data_as(C.c_void_p), words)
        return out

    def consume(self, s: State, token_id: int) -> bool:
        return bool(load_library().tms_vocab_consume(self._h, self.g._h, s._h, token_id))

    def clear_cache(self) -> None:
        load_library().tms_vocab_clear_cache(self._h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            load_library().tms_vocab_free(h)
            self._h = None


class TokenTable:
    """The bytes each vocabulary id contributes (tmtok.h:40-42 piece_bytes)
    and its whitespace-only flag, from SentencePiece or byte-level BPE
    pieces."""

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)

    @staticmethod
    def _pieces(pieces):
        toks = [None if t is None else (t.encode() if isinstance(t, str) else bytes(t)) for t in pieces]
        n = len(toks)
        bufs = (C.c_char_p * max(n, 1))(*toks)
        lens = (C.c_size_t * max(n, 1))(*[0 if t is None else len(t) for t in toks])
        return n, bufs, lens

    @classmethod
    def spm(cls, pieces: Sequence, types: Sequence[int]) -> "TokenTable":
        """SentencePiece pieces with their types (1 normal, 2 unknown,
        3 control, 6 byte)."""
        n, bufs, lens = cls._pieces(pieces)
        ty = np.ascontiguousarray(np.asarray(types, np.uint8))
        err = C.create_string_buffer(256)
        h = load_library().tms_token_table_spm(bufs, lens, ty.ctypes.data_as(C.c_void_p), n, err,
                                               len(err))
        if not h:
            raise ValueError(err.value.decode(errors="replace"))
        return cls(h)

    @classmethod
    def bpe(cls, pieces: Sequence) -> "TokenTable":
        """Byte-level BPE pieces (GPT-2 byte-to-unicode form); None for an id
        the vocabulary lacks."""
        n, bufs, lens = cls._pieces(pieces)
        err = C.create_string_buffer(256)
        h = load_library().tms_token_table_bpe(bufs, lens, n, err, len(err))
        if not h:
            raise ValueError(err.value.decode(errors="replace"))
        return cls(h)

    def __len__(self) -> int:
        return load_library().tms_token_table_size(self._h)

    def bytes(self, token_id: int) -> bytes:
        p, n = C.c_void_p(), C.c_size_t()
        load_library().tms_token_table_bytes(self._h, token_id, C.byref(p), C.byref(n))
        return C.string_at(p.value, n.value) if n.value else b""

    def ws_only(self, token_id: int) -> bool:
        return bool(load_library().tms_token_table_ws_only(self._h, token_id))

    def token_mask(self, g: Grammar, eos: int = -1) -> "TokenMask":
        return TokenMask.from_table(g, self, eos)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            load_library().tms_token_table_free(h)
            self._h = None


def _token_mask_from_table(cls, g: Grammar, table: TokenTable, eos: int = -1) -> TokenMask:
    h = load_library().tms_vocab_from_table(g._h, table._h, eos, None)
    if not h:
        raise ValueError("tms_vocab_from_table failed")
    m = cls.__new__(cls)
    m.g = g
    m._table = table
    m._h = C.c_void_p(h)
    m.n = len(table)
    return m


TokenMask.from_table = classmethod(_token_mask_from_table)


class Filter:
    """GrammarFilter (llama_chat.cpp:159-223): one decode's grammar state and
    no-progress count; mask() is restrict() as mask words."""

    def __init__(self, g: Grammar, mask: TokenMask, table: Optional[TokenTable] = None):
        h = load_library().tms_filter_create(g._h, mask._h, None if table is None else table._h)
        if not h:
            raise ValueError("tms_filter_create failed")
        self._h = C.c_void_p(h)
        self._keep = (g, mask, table)

    def reset(self) -> None:
        load_library().tms_filter_reset(self._h)

    def mask(self, vocab: int, out: Optional[np.ndarray] = None):
        """(words, count): count 0 means no id is allowed (all ones: fails open)."""
        words = (vocab + 31) // 32
        if out is None:
            out = np.empty(words, np.uint32)
        n = load_library().tms_filter_mask(self._h, out.ctypes.data_as(C.c_void_p), words)
        return out, n

    def consume(self, token_id: int) -> bool:
        return bool(load_library().tms_filter_consume(self._h, token_id))

    def complete(self, eos: int) -> bool:
        return bool(load_library().tms_filter_complete(self._h, eos))

    def done(self) -> bool:
        return bool(load_library().tms_filter_done(self._h))

    @property
    def stall(self) -> int:
        return load_library().tms_filter_stall(self._h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            load_library().tms_filter_free(h)
            self._h = None


class MaskPipe:
    """The next step's masks for a batch of filters on worker threads,
    uploaded on the pipe's own stream and ordered before the sampler."""

    def __init__(self, batch: int, vocab: int, threads: int = 2, device: int = 0):
        self.batch, self.words = batch, (vocab + 31) // 32
        h = load_library().tms_mask_pipe_create(device, batch, self.words, threads)
        if not h:
            raise RuntimeError("tms_mask_pipe_create failed")
        self._h = C.c_void_p(h)
        self._rows = [None] * batch

    def set_row(self, row: int, f: Optional[Filter]) -> None:
        rc = load_library().tms_mask_pipe_set_row(self._h, row, None if f is None else f._h)
        if rc != 0:
            raise RuntimeError(f"tms_mask_pipe_set_row: {rc}")
        self._rows[row] = f

    def submit(self, tokens: Optional[np.ndarray] = None) -> None:
        t = None if tokens is None else np.ascontiguousarray(tokens, np.int32)
        self._tokens = t   # kept alive until the workers have read it
        rc = load_library().tms_mask_pipe_submit(self._h, None if t is None else t.ctypes.data_as(C.c_void_p))
        if rc != 0:
            raise RuntimeError(f"tms_mask_pipe_submit: {rc}")

    def acquire(self, stream: int):
        """(device address of [batch][words] uint32, allowed counts)."""
        w = C.c_void_p()
        allowed = np.empty(self.batch, np.int32)
        rc = load_library().tms_mask_pipe_acquire(self._h, C.c_void_p(stream), C.byref(w),
                                                  allowed.ctypes.data_as(C.c_void_p))
        if rc != 0:
            raise RuntimeError(f"tms_mask_pipe_acquire: {rc}")
        return w.value, allowed

    def release(self, stream: int) -> None:
        rc = load_library().tms_mask_pipe_release(self._h, C.c_void_p(stream))
        if rc != 0:
            raise RuntimeError(f"tms_mask_pipe_release: {rc}")

    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            load_library().tms_mask_pipe_free(h)
            self._h = None

    def __del__(self):
        self.close()
