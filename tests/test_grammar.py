"""JSON validator (src/grammar.zig): the oracle restatement and the product's
host state machine, on the CPU.

Pinning: the reference's own KATs (grammar.zig:482-513); documents written by
json.dumps are accepted with every prefix and end finished; every ASCII text
the validator accepts to the finished state parses with json.loads (and, for
object roots without \\u escapes, the converse); hand-derived cases for the
reference's quirks (a \\u escape ends after three hex digits, depth limit 64,
object-only roots).  The product's state machine (bit-packed stack) then has
to agree with the oracle (64-entry stack array) byte by byte."""
import json
import random

import numpy as np
import pytest

from oracle import pyoracle as po
from zinfer_amd.api import JsonValidator

KATS = [  # src/grammar.zig:482-513: (text, consume ok, finished afterwards)
    ('{\n  "name": "zinfer",\n  "fast": true,\n  "version": 2\n}', True, True),
    ("123", False, None),
    ('{"items": [1, 2, {"sub": null}]}', True, True),
    ('{"x":-}', False, None),
    ('{"x":1,}', False, None),
    ('{"x":"\\q"}', False, None),
    ('{"text": "hello\\nworld\\u12af\\""}', True, True),
]


class Both:
    """Oracle and product validators stepped together."""

    def __init__(self, object_only=True):
        self.o = po.json_init(object_only)
        self.p = JsonValidator(object_only)

    def consume(self, text):
        a = po.json_consume(self.o, text)
        b = self.p.consume(text)
        assert a == b, text
        return a

    def finished(self):
        a = po.json_is_finished(self.o)
        assert a == self.p.is_finished()
        return a


@pytest.mark.parametrize("text,ok,fin", KATS)
def test_reference_kats(text, ok, fin):
    b = Both(True)
    assert b.consume(text) == ok
    if fin is not None:
        assert b.finished() == fin


def _rand_value(r: random.Random, depth: int):
    k = r.random()
    if depth > 0 and k < 0.25:
        return {_rand_str(r): _rand_value(r, depth - 1) for _ in range(r.randint(0, 4))}
    if depth > 0 and k < 0.45:
        return [_rand_value(r, depth - 1) for _ in range(r.randint(0, 4))]
    if k < 0.6:
        return _rand_str(r)
    if k < 0.7:
        return r.randint(-10**12, 10**12)
    if k < 0.8:
        return r.choice([0.0, -0.0, 1.5, -2.25e-7, 3.0e21, r.uniform(-1e6, 1e6)])
    return r.choice([True, False, None])


def _rand_str(r: random.Random):
    alphabet = 'ab c"\\/\n\t\x01\x1fé€😀{}[]:,'
    return "".join(r.choice(alphabet) for _ in range(r.randint(0, 8)))


def _docs(n, seed):
    r = random.Random(seed)
    for _ in range(n):
        obj = {_rand_str(r): _rand_value(r, r.randint(0, 6)) for _ in range(r.randint(0, 5))}
        indent = r.choice([None, 0, 1, 2, 4, "\t"])
        seps = r.choice([None, (",", ":"), (", ", ": ")])
        yield json.dumps(obj, indent=indent, separators=seps, ensure_ascii=r.random() < 0.5)


def test_json_dumps_documents_and_prefixes():
    for doc in _docs(150, 1):
        data = doc.encode()
        b = Both(True)
        for i in range(len(data)):  # every prefix is accepted, byte by byte
            assert b.consume(data[i:i + 1]), (doc, i)
            assert b.finished() == (i == len(data) - 1)
        assert b.consume(b" \n\t\r")  # trailing whitespace after the root
        assert not b.consume(b"x")
        # array roots need initAny
        arr = json.dumps([json.loads(doc)]).encode()
        assert not Both(True).consume(arr)
        assert Both(False).consume(arr)


def _json_ok(text: str) -> bool:
    try:
        json.loads(text)
        return True
    except ValueError:
        return False


def test_accepted_texts_parse_with_json_module():
    """Random texts over a JSON alphabet: finished => json.loads accepts; and
    json.loads accepts an object root (no \\u, no NaN/Infinity) => finished."""
    r = random.Random(2)
    alphabet = list('{}[]:," \n0123456789-+.eEtrufalsn\\/ab')
    finished = parsed_objects = 0
    for _ in range(20000):
        text = "".join(r.choice(alphabet) for _ in range(r.randint(1, 14)))
        text = r.choice(["", "{", '{"a":', '{"a":[', '{"k":"']) + text
        text += r.choice(["", "}", '"}', "]}", '"]}', "1}", "}}", " } "])
        b = Both(True)
        fin = b.consume(text) and b.finished()
        if fin:
            finished += 1
            assert _json_ok(text), text
        if "\\u" not in text and _json_ok(text) and isinstance(json.loads(text), dict):
            parsed_objects += 1
            assert fin, text
    assert finished > 50 and parsed_objects > 50


@pytest.mark.parametrize("text,ok,fin", [
    ('{"a":"\\u123"}', True, True),      # three hex digits end the escape (hex3 -> none)
    ('{"a":"\\u12"}', False, None),      # '"' is not a hex digit
    ('{"a":"\\u12af"}', True, True),     # the fourth hex digit is a plain character
    ('{"a":"\\u12G"}', False, None),
    ('{"a":"x\x1f"}', False, None),      # control byte inside a string
    ('{"a":"\\\x1f"}', False, None),
    ('{"a":01}', False, None),           # no leading zeros
    ('{"a":-0.5e+7}', True, True),
    ('{"a":1.}', False, None),
    ('{"a":1e}', False, None),
    ('{"a":.5}', False, None),
    ('{"a":tru}', False, None),
    ('{"a":truex}', False, None),
    ('{"a":nul', True, False),
    ('{}', True, True),
    ('{,}', False, None),
    ('{"a":1}}', False, None),
    ('{"a":[1,]}', False, None),         # value required after a comma in an array
    ('{"a":[]}', True, True),
    ('{"a":{}}', True, True),
    ('{"a" "b"}', False, None),
    ('  {"a":1} \n', True, True),
    ('{"a":1 , "b":2}', True, True),
    ('{"a":1]', False, None),
    ('{"a":[1}', False, None),
])
def test_hand_derived_cases(text, ok, fin):
    b = Both(True)
    assert b.consume(text) == ok
    if fin is not None:
        assert b.finished() == fin


def test_depth_limit_and_roots():
    b = Both(False)
    assert b.consume("[" * 64)
    assert not b.consume("[")  # stack full (64 entries)
    b = Both(False)
    assert b.consume("[" * 64 + "]" * 64) and b.finished()
    b = Both(True)
    assert b.consume('{"a":' + "[" * 63)
    assert not b.consume("{")
    assert not Both(True).consume("[")
    assert Both(False).consume("[")
    assert not Both(False).consume('"a"')  # scalar roots are never accepted


def _canon_oracle(j):
    """The oracle state in the C ABI's canonical form (zi_json_state fields)."""
    st, esc, num, depth = j.state, j.escape, j.num, j.depth
    stack = 0
    for d in range(depth):
        stack |= int(j.stack[d]) << d
    lit = bytes(j.lit_expected[: j.lit_len]) if st == 9 else b""
    return (st, esc if st in (3, 7) else 0, num if st == 8 else 0, depth, stack, j.object_only,
            (j.lit_len, j.lit_idx, lit) if st == 9 else None)


def _canon_product(v):
    s = v.st
    st = s.state
    stack = s.stack & ((1 << s.depth) - 1) if s.depth < 64 else s.stack
    lit = bytes(s.lit_expected[: s.lit_len]) if st == 9 else b""
    return (st, s.escape if st in (3, 7) else 0, s.num if st == 8 else 0, s.depth, stack, s.object_only,
            (s.lit_len, s.lit_idx, lit) if st == 9 else None)


def test_product_state_machine_matches_oracle_bytewise():
    """Random byte streams biased towards valid JSON: after every byte the
    product (bit-packed stack) and the oracle agree on acceptance and state;
    try_consume leaves its input untouched and returns the consumed state."""
    r = random.Random(3)
    docs = list(_docs(40, 4))
    for t in range(400):
        base = docs[t % len(docs)].encode()
        cut = r.randint(0, len(base))
        tail = bytes(r.choice(b'{}[]:,"\\ \n0123456789-+.eEtrufalsnu\x01\xc3') for _ in range(r.randint(0, 30)))
        data = base[:cut] + tail
        o = po.json_init(t % 3 != 0)
        p = JsonValidator(t % 3 != 0)
        for i, byte in enumerate(data):
            before = p.copy()
            tc = p.try_consume(bytes([byte]))
            assert bytes(p.st) == bytes(before.st)  # try_consume works on a copy
            a = po.json_consume(o, bytes([byte]))
            bb = p.step_byte(byte)
            assert a == bb == (tc is not None), (data, i)
            if not a:
                break
            assert _canon_oracle(o) == _canon_product(p), (data[: i + 1])
            assert _canon_product(tc) == _canon_product(p)


def test_oracle_mask_rules():
    """applyMask's rules (src/grammar.zig:446-479) on a hand-made vocabulary."""
    pieces = [b"{", b"}", b" ", b"", b"\n\n", b"x", b'{"', b"<eos>", b"<eot>", b" }", b"  \t"]
    off = np.zeros(len(pieces) + 1, np.uint32)
    off[1:] = np.cumsum([len(p) for p in pieces])
    buf = np.frombuffer(b"".join(pieces), np.uint8)
    eog, eos = [8], 7

    def allowed(j):
        m = po.json_mask(j, off, buf, eog, eos)
        return [i for i in range(len(pieces)) if (m[i >> 5] >> (i & 31)) & 1]

    j = po.json_init(True)
    assert allowed(j) == [0, 2, 3, 4, 6, 10]  # eos / eog forbidden, empty piece passes
    po.json_consume(j, "{}")
    assert allowed(j) == [2, 4, 7, 8, 10]     # finished: eos, eog, all-whitespace (not empty)
    assert allowed(po.json_init(True)) != allowed(j)
    j2 = po.json_init(True)
    po.json_consume(j2, "{")
    assert allowed(j2) == [1, 2, 3, 4, 9, 10]
    assert list(po.json_mask(j, off, buf, eog, None)) != list(po.json_mask(j, off, buf, eog, eos))
