"""Writes tests/golden/gbnf_golden.npz from the reference's compiled gbnf.h
(oracle/_ref/libgbnf_ref.so): allowed-id sets along seeded token walks over a
synthetic byte-level vocabulary, and accept/reject verdicts on strings, for a
set of grammars.  The host GBNF engine (tms_grammar_* / tms_vocab_*) is pinned
on these.

    make -C oracle && python tests/golden/make_gbnf_golden.py
"""
from __future__ import annotations

import ctypes as C
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gbnf_golden.npz")
LIB = os.path.join(ROOT, "oracle", "_ref", "libgbnf_ref.so")

JSON = r'''
root   ::= ws value ws
value  ::= object | array | string | number | "true" ws | "false" ws | "null" ws
object ::= "{" ws ( string ":" ws value ( "," ws string ":" ws value )* )? "}" ws
array  ::= "[" ws ( value ( "," ws value )* )? "]" ws
string ::= "\"" ( [^"\\] | "\\" ( ["\\/bfnrt] | "u" hhhh ) )* "\"" ws
hhhh   ::= [0-9a-fA-F] [0-9a-fA-F] [0-9a-fA-F] [0-9a-fA-F]
number ::= "-"? ( "0" | [1-9] [0-9]* ) ( "." [0-9]+ )? ( [eE] [-+]? [0-9]+ )? ws
ws     ::= [ \t\n\r]*
'''

GRAMMARS = [
    JSON,
    'root ::= "{" ws "\\"n\\"" ":" ws num "}" ws\nws ::= " "*\nnum ::= [0-9]+',
    'root ::= item ("," ws item)*\nitem ::= [a-z]+ | "(" root ")"\nws ::= [ ]?',
    'root ::= expr\nexpr ::= term (("+" | "-") term)*\nterm ::= factor (("*" | "/") factor)*\n'
    'factor ::= [0-9]+ | "(" expr ")"',
    'root ::= "é" [\\u00e0-\\u00ff]+ "!"?',
    'root ::= [^"\\x00-\\x1f]* "\\""   # negated class with a control range',
    'root ::= . . [^b-c a-b]',
    'root ::= ("yes" | "no") ( "," ( "yes" | "no" ) )* # comment\n',
    'root ::= root*',                               # an epsilon cycle (closure caps)
    'root ::= a\na ::= b? "x" a?\nb ::= "y" a?',     # mutual recursion
]

STRINGS = ['{}', '[]', 'null', 'true', '-12.5e-3', '{"a":1}', '{"a":1,"b":[1,2,{"c":"x"}]}',
           '[[[]],{"k":[[{"n":null}]]}]', '{"esc":"a\\"b\\\\c\\u00ff"}', '  {"ws" : [ 1 , 2 ] }  ',
           '{"a":}', '{"a":1,}', '[1,]', "{'a':1}", '{"a":"unterminated}', '{"a":1}}', 'nul',
           '01', '1.', '{"a":1} trailing', '', 'abc', 'a,b', '(a,b),c', '1+2*3', '(1+2', 'éàü!',
           'éa', 'xyz"', 'x\x01"', 'ab"', 'abc', 'abb', 'yes,no,yes', 'yes,,no', 'x', 'yxx',
           'yyxx', 'éè', '"', 'ok\xff']


def vocab(rng):
    toks = [bytes([b]) for b in range(256)]                       # every single byte
    pieces = ['{', '}', '[', ']', ':', ',', '"', '{"', '":', '", "', '"}', ' ', '  ', '\n', '\t',
              'true', 'false', 'null', 'nul', 'tr', 'ue', '0', '1', '12', '123', '-', '-1', '.',
              '.5', 'e', 'e-', 'E+', '\\', '\\"', '\\u', '00ff', 'ab', 'abc', '(', ')', '+', '*',
              '/', 'yes', 'no', ',yes', ',no', 'x', 'y', 'yx', '1x', '\\n', 'é', 'àü', '!', 'é!']
    toks += [p.encode() for p in pieces]
    toks += ['é'.encode()[:1], 'é'.encode()[1:] + b'x', 'ü'.encode()[:1], b'\xe2\x82', b'\xf0\x9f',
             b'\xff', b'\x80a']                                     # codepoint fragments
    for _ in range(600):                                           # random ASCII words
        n = int(rng.integers(1, 6))
        toks.append(bytes(rng.choice(list(b'abcdefxyz0123456789 ,:{}[]"-.+e'), n).tolist()))
    toks += [b'{', b'true', b'"']                                  # duplicate texts: first id wins
    return toks


def main():
    if not os.path.exists(LIB):
        raise SystemExit("oracle/_ref/libgbnf_ref.so not built: make -C oracle")
    lib = C.CDLL(LIB)
    lib.ref_gbnf_accepts.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
    lib.ref_gbnf_walk.argtypes = [C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t),
                                  C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_uint64,
                                  C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    rng = np.random.default_rng(20261203)
    toks = vocab(rng)
    n = len(toks)
    eos = n                 # EOS id just past the text tokens
    skip = np.zeros(n, np.uint8)
    skip[[5, 300, 301]] = 1
    bufs = (C.c_char_p * n)(*toks)
    lens = (C.c_size_t * n)(*[len(t) for t in toks])
    d = {"tokens": np.frombuffer(b"".join(toks), np.uint8),
         "token_lens": np.array([len(t) for t in toks], np.int32), "skip": skip,
         "eos": np.int32(eos), "grammars": np.array(json.dumps(GRAMMARS))}
    acc = np.zeros((len(GRAMMARS), len(STRINGS)), np.int32)
    for gi, g in enumerate(GRAMMARS):
        for si, st in enumerate(STRINGS):
            b = st.encode("utf-8", "surrogateescape") if "\xff" not in st else b"ok\xffbad"
            acc[gi, si] = lib.ref_gbnf_accepts(g.encode(), b, len(b))
    d["strings"] = np.array(json.dumps([s if "\xff" not in s else "<ok\\xffbad>" for s in STRINGS]))
    d["accepts"] = acc
    walks = 0
    for gi, g in enumerate(GRAMMARS):
        for w in range(6):
            steps, cap = 60, 400000
            ids = np.zeros(cap, np.int32)
            off = np.zeros(steps + 1, np.int32)
            chosen = np.zeros(steps, np.int32)
            can_end = np.zeros(steps, np.int32)
            k = lib.ref_gbnf_walk(g.encode(), bufs, lens, n, eos, skip.ctypes.data, steps,
                                  1000 * gi + w, ids.ctypes.data, cap, off.ctypes.data,
                                  chosen.ctypes.data, can_end.ctypes.data)
            assert k > 0, (gi, k)
            d[f"w{gi}_{w}_ids"] = ids[:off[k]].copy()
            d[f"w{gi}_{w}_off"] = off[:k + 1].copy()
            d[f"w{gi}_{w}_chosen"] = chosen[:k].copy()
            d[f"w{gi}_{w}_can_end"] = can_end[:k].copy()
            walks += 1
    np.savez_compressed(OUT, **d)
    print(f"{len(GRAMMARS)} grammars, {walks} walks, {len(STRINGS)} strings -> {OUT}")


if __name__ == "__main__":
    main()
