"""Host side of constrained decoding: the vocabulary byte tables (against
the reference's own tokenizer headers, compiled into oracle/_ref, and
GPT-2's published bytes_to_unicode table) and the grammar filter
(GrammarFilter, llama_chat.cpp:159-223: restriction, stall narrowing,
fail-open, completion).  CPU only."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

from tensormark_amd.grammar import Filter, Grammar, TokenMask, TokenTable

REF_TOK = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                       "libtok_ref.so")


def gpt2_bytes_to_unicode():
    """OpenAI GPT-2 encoder.py bytes_to_unicode, as published."""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(ord("¡"), ord("¬") + 1)) + \
        list(range(ord("®"), ord("ÿ") + 1))
    cs = bs[:]
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return dict(zip(bs, [chr(c) for c in cs]))


B2U = gpt2_bytes_to_unicode()


def to_piece(raw: bytes) -> bytes:
    return "".join(B2U[b] for b in raw).encode()


@pytest.fixture(scope="module")
def reftok():
    if not os.path.exists(REF_TOK):
        pytest.skip("oracle/_ref/libtok_ref.so (the reference's tokenizer headers) not built here")
    lib = C.CDLL(REF_TOK)
    lib.ref_bpe_bytes.argtypes = [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t]
    lib.ref_spm_bytes.argtypes = [C.POINTER(C.c_char_p), C.POINTER(C.c_size_t), C.c_void_p, C.c_int,
                                  C.c_char_p, C.c_size_t, C.c_void_p]
    return lib


def test_bpe_table_round_trips_gpt2_pieces():
    rng = np.random.default_rng(1)
    raws = [bytes(rng.integers(0, 256, int(rng.integers(1, 9))).tolist()) for _ in range(500)]
    raws += [bytes([b]) for b in range(256)]
    t = TokenTable.bpe([to_piece(r) for r in raws] + [None])
    assert len(t) == len(raws) + 1
    for i, r in enumerate(raws):
        assert t.bytes(i) == r, i
    assert t.bytes(len(raws)) == b""          # an id the vocabulary lacks
    assert t.bytes(10 ** 6) == b""            # outside the table


def test_bpe_table_matches_reference(reftok):
    rng = np.random.default_rng(2)
    pieces = [to_piece(bytes(rng.integers(0, 256, int(rng.integers(1, 7))).tolist())) for _ in range(300)]
    pieces += ["Ġhello".encode(), "Ċ".encode(), "ĠĠ".encode(), "ĉ".encode()]
    t = TokenTable.bpe(pieces)
    buf = C.create_string_buffer(64)
    for i, p in enumerate(pieces):
        n = reftok.ref_bpe_bytes(p, len(p), buf, len(buf))
        assert n >= 0 and t.bytes(i) == buf.raw[:n], i
    assert t.bytes(len(pieces) - 4) == b" hello" and t.bytes(len(pieces) - 3) == b"\n"
    # codepoints outside the table: both refuse
    for bad in ["€".encode(), "\U0001F600".encode(), b"\xc4"]:
        assert reftok.ref_bpe_bytes(bad, len(bad), buf, len(buf)) == -1
        with pytest.raises(ValueError):
            TokenTable.bpe([bad])


SPM_PIECES = [("<unk>", 2), ("<s>", 3), ("</s>", 3), ("<0x0A>", 6), ("<0x20>", 6), ("<0xFF>", 6),
              ("▁hello", 1), ("▁▁", 1), ("world▁", 1), ("▁", 1), ("<0x0A0>", 6), ("\t", 1),
              ("a▁b▁", 1), ("▁\n", 1), ("<0x09>", 6), ("x", 4)]


def test_spm_table_closed_form():
    t = TokenTable.spm([p for p, _ in SPM_PIECES], [k for _, k in SPM_PIECES])
    want = [b"<unk>", b"", b"", b"\n", b" ", b"\xff", b" hello", b"  ", b"world ", b" ", b"", b"\t",
            b"a b ", b" \n", b"\t", b"x"]
    assert [t.bytes(i) for i in range(len(SPM_PIECES))] == want
    ws = [t.ws_only(i) for i in range(len(SPM_PIECES))]
    assert ws == [False, False, False, True, True, False, False, True, False, True, False, True,
                  False, True, True, False]
    with pytest.raises(ValueError):
        TokenTable.spm(["<0xZZ>"], [6])


def test_spm_table_matches_reference(reftok):
    pieces = [p.encode() for p, _ in SPM_PIECES]
    types = np.array([k for _, k in SPM_PIECES], np.uint8)
    n = len(pieces)
    bufs = (C.c_char_p * n)(*pieces)
    lens = (C.c_size_t * n)(*[len(p) for p in pieces])
    out = C.create_string_buffer(4096)
    lo = np.zeros(n, np.int32)
    tot = reftok.ref_spm_bytes(bufs, lens, types.ctypes.data_as(C.c_void_p), n, out, len(out),
                               lo.ctypes.data_as(C.c_void_p))
    assert tot >= 0
    t = TokenTable.spm([p for p, _ in SPM_PIECES], types)
    at = 0
    for i in range(n):
        assert t.bytes(i) == out.raw[at:at + lo[i]], i
        at += lo[i]
    bad = [b"<0xZZ>"]
    assert reftok.ref_spm_bytes((C.c_char_p * 1)(*bad), (C.c_size_t * 1)(6),
                                np.array([6], np.uint8).ctypes.data_as(C.c_void_p), 1, out, len(out),
                                lo.ctypes.data_as(C.c_void_p)) == -1


def test_token_mask_from_table_equals_byte_list():
    g = Grammar.parse('root ::= "{" ws "\\"k\\"" ws ":" ws [0-9]+ ws "}"\nws ::= [ \\t\\n]*')
    pieces = ["{", "}", "▁", "\n", '"k"', ":", "1", "23", "▁▁", "x", "</s>"]
    types = [1] * 10 + [3]
    t = TokenTable.spm(pieces, types)
    a = TokenMask.from_table(g, t, eos=10)
    b = TokenMask(g, [t.bytes(i) for i in range(len(pieces))], eos=10)
    s = g.start()
    for tok in [0, 2, 4, 5, 6, 7, 3, 1]:
        assert a.allowed(s) == b.allowed(s)
        assert a.consume(s, tok)
    assert a.allowed(s) == b.allowed(s) == [10]


def _json_filter():
    g = Grammar.parse('root ::= "{" ws "}" ws\nws ::= [ \\t\\n]*')
    pieces = ["{", "}", "▁", "\n", "▁▁", "x", "</s>", "▁}"]
    t = TokenTable.spm(pieces, [1, 1, 1, 1, 1, 1, 3, 1])
    m = TokenMask.from_table(g, t, eos=6)
    return g, m, t, Filter(g, m, t)


def bits_to_ids(words):
    return [i for i in range(len(words) * 32) if (int(words[i >> 5]) >> (i & 31)) & 1]


def test_filter_stall_narrows_whitespace():
    """GrammarFilter: once four consumed tokens leave the state unchanged,
    the whitespace-only ids drop out of the mask (if anything else stays)."""
    g, m, t, f = _json_filter()
    V = 8
    w, n = f.mask(V)
    assert bits_to_ids(w) == [0] and n == 1
    assert f.consume(0) and f.stall == 0
    full = [1, 2, 3, 4, 7]
    w, n = f.mask(V)
    assert bits_to_ids(w) == full
    for k in range(1, 5):
        assert f.consume(2)                       # " " keeps ws's state
        assert f.stall == k
        w, n = f.mask(V)
        assert bits_to_ids(w) == (full if k < 4 else [1, 7]), k
        assert n == len(bits_to_ids(w))
    assert f.consume(7) and f.stall == 0          # " }" moves on
    w, _ = f.mask(V)
    assert bits_to_ids(w) == [2, 3, 4, 6]         # trailing ws or EOS
    assert not f.complete(6) and f.done()
    for k in range(4):
        f.consume(3)
    w, n = f.mask(V)
    # only whitespace and EOS remain: narrowing keeps EOS
    assert bits_to_ids(w) == [6] and n == 1
    f.reset()
    assert f.stall == 0 and bits_to_ids(f.mask(V)[0]) == [0]


def test_filter_fails_open_when_nothing_is_allowed():
    g, m, t, f = _json_filter()
    assert not f.consume(5)                        # "x" kills the state
    w, n = f.mask(40)
    assert n == 0 and (w == 0xFFFFFFFF).all()


def test_filter_complete_on_eos_only():
    g = Grammar.parse('root ::= "ab"')
    t = TokenTable.spm(["a", "b", "</s>"], [1, 1, 3])
    m = TokenMask.from_table(g, t, eos=2)
    f = Filter(g, m, t)
    assert not f.complete(2)
    f.consume(0)
    f.consume(1)
    assert f.complete(2) and f.done()
