"""The host GBNF engine (C ABI tms_grammar_* / tms_vocab_*, Python view in
tensormark_amd.grammar) against the reference's gbnf.h.

* test_gbnf.cpp's accept/reject and token-mask cases (tensormark/test_gbnf.cpp:
  the grammar texts and strings below are its vectors);
* golden vectors from the compiled reference (tests/golden/gbnf_golden.npz,
  written by make_gbnf_golden.py): accept verdicts, and allowed-id sets plus
  can_end along 60 seeded token walks over a byte-level vocabulary;
* the bitmask <-> allowed-list invariant the sampler relies on.
CPU only."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from tensormark_amd.grammar import Grammar, GrammarError, TokenMask

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gbnf_golden.npz")

JSON_GBNF = r'''
root   ::= ws value ws
value  ::= object | array | string | number | "true" ws | "false" ws | "null" ws
object ::= "{" ws ( string ":" ws value ( "," ws string ":" ws value )* )? "}" ws
array  ::= "[" ws ( value ( "," ws value )* )? "]" ws
string ::= "\"" ( [^"\\] | "\\" ( ["\\/bfnrt] | "u" hhhh ) )* "\"" ws
hhhh   ::= [0-9a-fA-F] [0-9a-fA-F] [0-9a-fA-F] [0-9a-fA-F]
number ::= "-"? ( "0" | [1-9] [0-9]* ) ( "." [0-9]+ )? ( [eE] [-+]? [0-9]+ )? ws
ws     ::= [ \t\n\r]*
'''

# (grammar, accepted strings, rejected strings) -- test_gbnf.cpp:43-139, 182-197, 265-282
KATS = [
    ('root ::= "hello"', ["hello"], ["hell", "helloo", "Hello", ""]),
    ('root ::= "a" | "b"+', ["a", "b", "bbbb"], ["", "ab", "ba"]),
    ('root ::= "x" "y"* "z"', ["xz", "xyz", "xyyyz"], ["xyy"]),
    ('root ::= "a"? "b"', ["b", "ab"], ["a"]),
    ('root ::= [a-c]+ [0-9]', ["abc7", "a0"], ["d0", "abc"]),
    ('root ::= [^,]+ ","', ["abc,", "a b,"], [",,"]),
    ('root ::= . . .', ["abc"], ["ab", "abcd"]),
    ('root ::= ("ab" | "cd")+ "!"', ["ab!", "cdab!"], ["abcd"]),
    ('root ::= "a\\nb\\t\\"c"', ['a\nb\t"c'], ["ab"]),
    ('root ::= [\\t ] "["', ["\t[", " ["], ["x["]),
    (JSON_GBNF,
     ["{}", "[]", "null", "true", "-12.5e-3", '{"a":1}', '{"a":1,"b":[1,2,{"c":"x"}]}',
      '[[[]],{"k":[[{"n":null}]]}]', '{"esc":"a\\"b\\\\c\\u00ff"}', '  {"ws" : [ 1 , 2 ] }  '],
     ['{"a":}', '{"a":1,}', "[1,]", "{'a':1}", '{"a":"unterminated}', '{"a":1}}', "nul", "01",
      "1.", '{"a":1} trailing']),
    ('root ::= "é" [\\u00e0-\\u00ff]', ["éé", "éà"], ["éa"]),
]


@pytest.mark.parametrize("i", range(len(KATS)))
def test_accept_reject_kats(i):
    text, good, bad = KATS[i]
    g = Grammar.parse(text)
    for s in good:
        assert g.accepts(s), s
    for s in bad:
        assert not g.accepts(s), s


def test_deep_recursion():
    g = Grammar.parse(JSON_GBNF)
    deep = "[" * 200 + "1" + "]" * 200
    assert g.accepts(deep)
    assert not g.accepts(deep[:-1] + "}")


def test_byte_at_a_time_utf8():
    g = Grammar.parse('root ::= "é" [\\u00e0-\\u00ff]')
    s = g.start()
    assert all(g.advance(s, b) for b in "éé".encode())
    assert g.can_end(s)


@pytest.mark.parametrize("text", [
    'thing ::= "a"', "root ::= missing", 'root ::= "a"\nroot ::= "b"', "root ::= [0-9]{4}",
    'root ::= "unterminated', "root ::= [abc", 'root ::= ("a"', 'root ::= "a")', "root ::= *",
    'root ::= "a"**', '::= "a"', "root ::= [z-a]", 'root ::= "\\x4"', "root ::= @",
    'root ::= ( "a" x ::= "b" )'])
def test_parse_errors(text):
    with pytest.raises(GrammarError, match="gbnf:"):
        Grammar.parse(text)


def test_state_identity():
    g = Grammar.parse(JSON_GBNF)
    a, b = g.start(), g.start()
    assert a == b
    for ch in b'{"a':
        assert g.advance(a, ch) and g.advance(b, ch)
    assert a == b
    assert g.advance(b, ord('"'))
    assert not (a == b)


def test_token_mask_kats():
    g = Grammar.parse('root ::= "{" ws "\\"n\\"" ":" ws num "}" ws\nws  ::= " "*\nnum ::= [0-9]+')
    toks = [b"{", b'"n"', b":", b" ", b"1", b"2", b"}", b"x", b"1x"]
    EOS = 100
    m = TokenMask(g, toks, EOS)
    s = g.start()
    ok = lambda i: i in m.allowed(s)   # noqa: E731
    assert ok(0) and not ok(4) and not ok(7) and not ok(EOS)
    for t in (0, 1, 2):
        assert m.consume(s, t)
    assert ok(4) and not ok(0)
    assert m.consume(s, 4) and m.consume(s, 5)
    assert not ok(EOS)
    assert m.consume(s, 6)
    assert ok(EOS) and not ok(4)
    s2 = g.start()
    for t in (0, 1, 2):
        m.consume(s2, t)
    assert 8 not in m.allowed(s2)          # '1x' leaves the grammar as a whole
    skip = [0] * len(toks)
    skip[4] = 1
    m2 = TokenMask(g, toks, EOS, skip)
    s3 = g.start()
    for t in (0, 1, 2):
        m2.consume(s3, t)
    a3 = m2.allowed(s3)
    assert 4 not in a3 and 5 in a3


def test_invalid_utf8_rejected():
    dot = Grammar.parse("root ::= . .")
    for bad in (b"\xff\xfe", b"\x80\x80", b"\xe2\x28\xa1"):
        assert not dot.accepts(bad)
    assert not Grammar.parse('root ::= [^"]+ ').accepts(b"ok\xffbad")
    assert dot.accepts("éè".encode())


# ---------------------------------------------------------------- golden vectors

@pytest.fixture(scope="module")
def gg():
    return np.load(GOLDEN, allow_pickle=False)


def _tokens(gg):
    lens = gg["token_lens"]
    flat = gg["tokens"].tobytes()
    out, o = [], 0
    for n in lens:
        out.append(flat[o:o + n])
        o += n
    return out


def test_accepts_match_reference(gg):
    grammars = json.loads(str(gg["grammars"]))
    strings = json.loads(str(gg["strings"]))
    acc = gg["accepts"]
    for gi, text in enumerate(grammars):
        g = Grammar.parse(text)
        for si, st in enumerate(strings):
            b = b"ok\xffbad" if st == "<ok\\xffbad>" else st.encode()
            assert int(g.accepts(b)) == acc[gi, si], (gi, st)


def test_allowed_sets_match_reference_walks(gg):
    grammars = json.loads(str(gg["grammars"]))
    toks = _tokens(gg)
    eos = int(gg["eos"])
    V = len(toks) + 1
    steps = 0
    for gi, text in enumerate(grammars):
        g = Grammar.parse(text)
        m = TokenMask(g, toks, eos, gg["skip"])
        for w in range(6):
            ids, off = gg[f"w{gi}_{w}_ids"], gg[f"w{gi}_{w}_off"]
            chosen, can_end = gg[f"w{gi}_{w}_chosen"], gg[f"w{gi}_{w}_can_end"]
            s = g.start()
            for k in range(len(chosen)):
                want = ids[off[k]:off[k + 1]].tolist()
                got = m.allowed(s)
                assert got == want, (gi, w, k, len(got), len(want))
                assert int(g.can_end(s)) == can_end[k]
                # the bitmask form holds exactly the same ids
                words = m.mask(s, V)
                bits = np.unpackbits(words.view(np.uint8), bitorder="little")[:V]
                assert np.flatnonzero(bits).tolist() == want
                steps += 1
                c = int(chosen[k])
                if c < 0 or c == eos:
                    break
                assert m.consume(s, c)
    assert steps > 300
