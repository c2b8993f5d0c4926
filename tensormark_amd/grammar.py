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
