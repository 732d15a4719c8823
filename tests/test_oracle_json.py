"""Pins the oracle's JSON prefix classifier (src/json.br:227-426, oracle/json_prefix.cpp): the reference's own
known answers (test/test_json.br:67-99, transliterated), a property that Python's json module fixes (every
prefix of a serialised object is viable, the whole complete, trailing text after it impossible), and a planted
mistake (oracle/Makefile `mutants`, 7: a leading zero followed by digits) that the known answers catch."""
import ctypes
import json
import random

import _oracle as O


def _lib(L):
    L.orc_json_prefix_state.restype = ctypes.c_int
    L.orc_json_prefix_state.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_int64, ctypes.c_int]
    return L


def state(L, s, obj=False):
    cps = (ctypes.c_uint32 * max(len(s), 1))(*[ord(c) for c in s])
    return L.orc_json_prefix_state(cps, len(s), 1 if obj else 0)


def known_answer_failures(L):
    L = _lib(L)
    bad = []
    constrained = '{"name": "café", "args": [1, -2.5e+3, true, null]}'
    for n in range(len(constrained)):
        if state(L, constrained[:n]) != 0:
            bad.append(("prefix", n))
    if state(L, constrained) != 1:
        bad.append("complete")
    if state(L, "  " + constrained + " \n\t") != 1:
        bad.append("whitespace")
    for s in ['{]', '[}', '{"a",', '{"a": truX', '{"a": 01', '{"a": "bad\\q']:
        if state(L, s) != -1:
            bad.append(("impossible", s))
    for s in ["", "  ", "{", '{"a', '{"a":', '{"a": [1,', '{"a": 1e+']:
        if state(L, s) != 0:
            bad.append(("possible", s))
    if state(L, '  {"ok": true}', True) != 1:
        bad.append("object")
    if state(L, "[1, 2]", True) != -1 or state(L, '"scalar"', True) != -1:
        bad.append("object root")
    # json_object_candidate_allowed (:408-418): prefix + piece viable; EOS only after a complete object
    if state(L, "  {", True) < 0 or state(L, '{"a": 1', True) < 0 or state(L, '{"a": nope', True) >= 0:
        bad.append("candidates")
    if state(L, '{"a": 1}', True) != 1 or state(L, '{"a": 1', True) == 1 or state(L, '{"a": 1} trailing', True) >= 0:
        bad.append("eos")
    if state(L, '{"x": "caf�', True) < 0 or state(L, '{"x": "café', True) < 0:
        bad.append("decoded")
    return bad


def random_value(rng, depth):
    k = rng.randrange(7 if depth < 4 else 4)
    if k == 0:
        return rng.choice([True, False, None])
    if k == 1:
        return rng.choice([0, -7, 12345, 3.25, -0.5, 1e-9, 6.02e23])
    if k in (2, 3):
        return "".join(rng.choice('ab "\\/\n\té€\U0001F600\x01') for _ in range(rng.randrange(6)))
    if k in (4, 5):
        return {f"k{i}": random_value(rng, depth + 1) for i in range(rng.randrange(4))}
    return [random_value(rng, depth + 1) for _ in range(rng.randrange(4))]


def property_failures(L):
    L = _lib(L)
    rng = random.Random(3)
    bad = 0
    for _ in range(60):
        doc = json.dumps({f"k{i}": random_value(rng, 1) for i in range(rng.randrange(1, 4))},
                         ensure_ascii=rng.random() < 0.5, indent=rng.choice([None, 1]))
        bad += sum(state(L, doc[:n], True) != 0 for n in range(len(doc)))
        bad += state(L, doc, True) != 1
        bad += state(L, doc + rng.choice([" x", ",", "}", "]", " {}"]), True) != -1
    return bad


def test_json_prefix_known_answers():
    assert known_answer_failures(O.lib()) == []


def test_json_prefix_property():
    assert property_failures(O.lib()) == 0


def test_json_prefix_check_fails_on_planted_mistake():
    assert known_answer_failures(O.mutant(7)) != []
