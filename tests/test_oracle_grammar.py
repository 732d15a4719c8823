"""Pins the oracle's grammar, schema, UTF-8 and drafting restatements.

Transliterates test/test_grammar.br, test/test_schema_grammar.br, test/test_speculative.br and
test/test_tokenizer.br:52-58 of the reference; checks the JSON-Schema compiler's output for the
workload-3 schema against the GBNF text hand-derived from src/schema_grammar.br (tests/golden); and
checks that the carry form of a candidate's piece equals the reference's literal re-decode of the
whole reply (src/server.br:342-351) on random byte replies.
"""
import ctypes
import os

import numpy as np
import pytest

import _oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def G(text):
    return O.Grammar(text)


# ------------------------------------------------------------ test/test_grammar.br

JSON_GBNF = r'''root   ::= object
value  ::= object | array | string | number | ("true" | "false" | "null") ws
object ::=
  "{" ws (
            string ":" ws value
    ("," ws string ":" ws value)*
  )? "}" ws
array  ::=
  "[" ws (
            value
    ("," ws value)*
  )? "]" ws
string ::=
  "\"" (
    [^"\\\x7F\x00-\x1F] |
    "\\" (["\\bfnrt] | "u" [0-9a-fA-F]{4})
  )* "\"" ws
number ::= ("-"? ([0-9] | [1-9] [0-9]{0,15})) ("." [0-9]+)? ([eE] [-+]? [0-9]+)? ws
ws ::= | " " | "\n" [ \t]{0,20}
'''


def test_grammar_language():  # :14-40
    g1 = G('root ::= "yes" | "no"')
    assert g1.accepts("yes") and g1.accepts("no")
    assert not g1.accepts("ye") and g1.viable("ye") and not g1.viable("x")
    g2 = G('root ::= [a-c]+ "!"?  # letters then an optional bang\n')
    assert g2.accepts("abca") and g2.accepts("ab!") and not g2.accepts("") and not g2.viable("d")
    assert not g2.viable("a!b")
    g3 = G('root ::= item ("," item)*\nitem ::= [0-9]{2,3}')
    assert g3.accepts("12") and g3.accepts("123,45,678") and not g3.accepts("1") and not g3.viable("1234")
    g4 = G('root ::= "a"{3}')
    assert g4.accepts("aaa") and not g4.accepts("aa") and not g4.viable("aaaa")
    g5 = G('root ::= "a"{2,}')
    assert g5.accepts("aa") and g5.accepts("aaaaa") and not g5.accepts("a")
    g6 = G('root ::= greeting " " name\ngreeting ::= (\n  "hi" |\n  "hello"\n)\nname ::= [^ \\n]+')
    assert g6.accepts("hello bob") and g6.accepts("hi x") and not g6.viable("hey")
    assert not g6.accepts("hi ")
    g7 = G(r'root ::= . "\x41" "é"')
    assert g7.accepts("zAé") and not g7.accepts("zBé")
    gj = G(JSON_GBNF)
    assert gj.accepts('{"a": [1, 2.5, true], "b": {"c": null}}')
    assert not gj.accepts('{"a": }') and not gj.viable("[1]")
    partial = chr(0xFFFD)  # :42-45
    assert not g1.viable(partial) and g6.viable("hi " + partial)
    assert not g2.viable(partial) and G("root ::= [^x]+").viable("a" + partial)


@pytest.mark.parametrize("text,ok", [
    ("root ::= foo", False), ('main ::= "x"', False), ('root ::= "x', False),
    ('root ::= "a"{2000000000}', False), ('root ::= "a"{0,2000000000}', False),
    ('root ::= "a"{99999999999999999999999999}', False), ('root ::= (("ab"{2000}){2000}){2000}', True),
    ("root ::= " + "(" * 5000 + "[a]" + ")" * 5000, False),
])
def test_grammar_errors_and_limits(text, ok):  # :47-72
    if ok:
        G(text)
    else:
        with pytest.raises(ValueError, match="grammar"):
            G(text)


def test_grammar_nesting_counts():  # :73
    assert G('root ::= ((("a"{3})))').accepts("aaa")


def test_grammar_error_messages():
    with pytest.raises(ValueError, match="undefined rule 'foo'"):
        G("root ::= foo")
    with pytest.raises(ValueError, match="there is no `root` rule"):
        G('main ::= "x"')
    with pytest.raises(ValueError, match="unterminated string literal"):
        G('root ::= "x')


def test_left_recursion_guard():
    g = G('root ::= root "a" | "b"')
    with pytest.raises(RuntimeError, match="left-recursive or too ambiguous"):
        g.viable("b")


# ------------------------------------------------------------ test/test_schema_grammar.br

def S(schema):
    return G(O.json_schema_to_gbnf(schema))


def test_schema_language():  # :22-51
    g1 = S('{"type":"object","properties":{"n":{"type":"integer"},"s":{"type":"string"},"b":{"type":"boolean"}},'
           '"required":["n"]}')
    assert g1.accepts('{"n": 5}') and g1.accepts('{"n":5,"s":"x","b":true}') and g1.accepts('{"n": -12, "b": false}')
    assert not g1.accepts('{"s": "x"}') and not g1.viable('{"x"') and not g1.viable('"') and not g1.viable("5")
    assert not g1.viable('{"n": 5} ')
    assert not g1.accepts('{"n": 5.5}') and not g1.accepts('{"n": "5"}')
    g2 = S('{"type":"object","properties":{"n":{"type":"integer"}},"required":["n"]}')
    assert not g2.viable('"') and g2.viable("{") and g2.viable('{"n": 2')
    g3 = S('{"type":"object","properties":{"a":{"type":"integer"},"b":{"enum":["x","y"]}}}')
    assert g3.accepts("{}") and g3.accepts('{"b": "y"}') and g3.accepts('{"a": 1, "b": "x"}')
    assert not g3.accepts('{"b": "z"}') and not g3.viable("{,")
    g4 = S('{"type":"array","items":{"type":"integer"},"minItems":2,"maxItems":3}')
    assert g4.accepts("[1, 2]") and g4.accepts("[1,2,3]") and not g4.accepts("[1]") and not g4.viable("[1,2,3,")
    g5 = S('{"anyOf":[{"type":"string"},{"type":"null"}]}')
    assert g5.accepts("null") and g5.accepts('"hi"') and not g5.accepts("5")
    g6 = S('{"type":["integer","boolean"]}')
    assert g6.accepts("42") and g6.accepts("true") and not g6.accepts('"x"')
    g7 = S('{"const":"fixed"}')
    assert g7.accepts('"fixed"') and not g7.accepts('"other"')
    g8 = S('{"type":"object","additionalProperties":{"type":"integer"}}')
    assert g8.accepts("{}") and g8.accepts('{"a": 1, "b": 2}') and not g8.accepts('{"a": "x"}')
    g9 = S('{"type":"string","minLength":2,"maxLength":3}')
    assert g9.accepts('"ab"') and g9.accepts('"abc"') and not g9.accepts('"a"') and not g9.viable('"abcd')
    g10 = S('{"$ref":"#/$defs/node","$defs":{"node":{"type":"object","properties":{"v":{"type":"integer"},'
            '"next":{"anyOf":[{"$ref":"#/$defs/node"},{"type":"null"}]}},"required":["v","next"]}}}')
    assert g10.accepts('{"v": 1, "next": {"v": 2, "next": null}}') and not g10.accepts('{"v": 1}')


C3_SCHEMA = ('{"type":"object","properties":{"name":{"type":"string","pattern":"^[a-z_]+$"},'
             '"count":{"type":"integer"},"tags":{"type":"array","items":{"type":"string"}}},'
             '"required":["name","count","tags"]}')


def test_workload3_gbnf_matches_hand_derivation():
    # tests/golden/c3_schema.gbnf was derived by hand from src/schema_grammar.br:146-337 (`pattern` dropped)
    with open(os.path.join(GOLDEN, "c3_schema.gbnf")) as f:
        want = f.read()
    assert O.json_schema_to_gbnf(C3_SCHEMA) == want
    g = G(want)
    assert g.accepts('{"name": "x_y", "count": -3, "tags": ["a", "b"]}')
    assert g.accepts('{"name":"Not A Pattern","count":0,"tags":[]}')  # pattern is not enforced
    assert not g.viable('{"count"')


# ------------------------------------------------------------ test/test_speculative.br

def test_ngram_draft():
    t = [1, 2, 5, 6, 7, 8, 9, 3, 4, 5, 6, 7]
    assert O.ngram_draft(t, 8, 3, 2) == [8, 9, 3, 4, 5, 6, 7]
    assert O.ngram_draft(t, 2, 3, 2) == [8, 9]
    u = [9, 6, 7, 1, 2, 3, 4, 8, 6, 7]
    assert O.ngram_draft(u, 4, 3, 2) == [1, 2, 3, 4]
    assert O.ngram_draft(u, 4, 3, 3) == []
    v = [1, 2, 3, 9, 1, 2, 3, 8, 1, 2, 3]
    assert O.ngram_draft(v, 1, 3, 3) == [8]
    assert O.ngram_draft([1, 2], 4, 3, 1) == []
    assert O.ngram_draft([4, 4], 4, 1, 1) == [4]


# ------------------------------------------------------------ test/test_tokenizer.br:44-58

def test_bytes_to_str():
    ff = "�"
    assert O.bytes_to_cps(b"A") == "A"
    assert O.bytes_to_cps(bytes([0xC3, 0xA9])) == "é"
    assert O.bytes_to_cps(bytes([0xC3])) == ff
    assert O.bytes_to_cps(bytes([65, 0xE6, 0x97])) == "A" + ff + ff
    assert O.bytes_to_cps(bytes([0xF0, 0x9F, 0x98])) == ff * 3
    assert O.bytes_to_cps(bytes([0xF0, 0x9F, 0x98, 0x80])) == "😀"
    assert O.bytes_to_cps(bytes([0x80, 66])) == ff + "B"
    assert O.bytes_to_cps(bytes([0xE6, 0x97, 0xA5])) == "日"


def test_bytes_to_str_matches_python_on_valid_utf8():
    rng = np.random.default_rng(0)
    for _ in range(200):
        s = "".join(chr(int(c)) for c in rng.integers(0x20, 0x2FFFF, 8) if not 0xD800 <= c <= 0xDFFF)
        assert O.bytes_to_cps(s.encode()) == s
        assert O.lib().orc_is_valid_utf8(s.encode(), len(s.encode())) == 1


# ------------------------------------------------------------ carry form == literal re-decode

def _slot_with_grammar(gbnf, vocab_tokens, reply):
    blob = b"".join(vocab_tokens)
    offs = np.zeros(len(vocab_tokens) + 1, np.uint32)
    offs[1:] = np.cumsum([len(t) for t in vocab_tokens])
    hist = O.i32(reply or [0])
    h = O.lib().orc_slot_new(O.params(), 1, O.ip(hist), len(reply), O.ip(hist), len(reply), O.ip(hist), O.fp(O.f32([0])), 0)
    assert O.lib().orc_slot_set_grammar(h, gbnf.encode(), blob, O.up(offs), len(vocab_tokens), len(vocab_tokens) - 1) == 0
    return h


@pytest.mark.parametrize("gbnf", [r'root ::= [^\x00]*', r'root ::= [a-z ]* ([^a-z] [a-z]*)?', r'root ::= "x" [^x]*'])
def test_carry_piece_equals_literal(gbnf):
    rng = np.random.default_rng(abs(hash(gbnf)) % 1000)
    interesting = [0x41, 0x61, 0x78, 0x80, 0x9F, 0xA9, 0xBF, 0xC0, 0xC3, 0xE0, 0xE6, 0xED, 0xF0, 0xF4, 0xF5, 0xFF]
    toks = []
    for _ in range(300):
        n = int(rng.integers(1, 5))
        toks.append(bytes(int(b) for b in rng.choice(interesting, n)))
    toks.append(b"<|eos|>")
    V = len(toks)
    L = O.lib()
    agree = 0
    for trial in range(60):
        reply = [int(t) for t in rng.integers(0, V - 1, int(rng.integers(0, 6)))]
        h = _slot_with_grammar(gbnf, toks, reply)
        m1 = np.zeros((V + 31) // 32, np.uint32)
        m2 = np.zeros_like(m1)
        a, b = ctypes.c_int(), ctypes.c_int()
        r1 = L.orc_slot_grammar_mask(h, V, O.up(m1), ctypes.byref(a), 1)
        r2 = L.orc_slot_grammar_mask(h, V, O.up(m2), ctypes.byref(b), 0)
        L.orc_slot_free(h)
        assert r1 == r2
        if r1 == 1:
            assert np.array_equal(m1, m2) and a.value == b.value
            agree += 1
    assert agree > 5


# ------------------------------------------------------------ speculative verification (src/server.br:1173-1216)

@pytest.mark.parametrize("temperature", [0.0, 0.7])
def test_spec_verify_equals_sequential_decoding(temperature):
    """The invariant the reference states for speculation (CHANGELOG.md:92, "greedy output with spec ==
    without spec"), extended to sampled rows: spec_verify's per-row tokens equal plain sequential
    decode steps on those rows with the drafts appended to the history, its accepted length is the
    first mismatch, and the slot ends in the sequential run's RNG state (accepted + 1 draws)."""
    V, K = 997, 6
    rng = np.random.default_rng(11)
    L = O.lib()
    p = O.params(temperature=temperature, top_k=0, repeat_penalty=1.2, repeat_last_n=8,
                 frequency_penalty=0.3, presence_penalty=0.1)
    hist = O.i32(rng.integers(0, V, 12))
    for trial in range(6):
        rows = (rng.standard_normal((K + 1) * V) * 3.0).astype(np.float32)
        spec = L.orc_slot_new(O.C.byref(p), 1000 + trial, O.ip(hist), len(hist), O.ip(hist), len(hist), None, None, 0)
        seq = L.orc_slot_new(O.C.byref(p), 1000 + trial, O.ip(hist), len(hist), O.ip(hist), len(hist), None, None, 0)
        ref = L.orc_slot_new(O.C.byref(p), 1000 + trial, O.ip(hist), len(hist), O.ip(hist), len(hist), None, None, 0)
        try:
            # the sequential tokens when every draft is accepted (history grows with the drafts)
            want = []
            for i in range(K + 1):
                t = np.zeros(1, np.int32)
                assert L.orc_slot_step(ref, O.fp(rows[i * V:(i + 1) * V]), V, 0, 1, O.ip(t), None, None, None, None) == 0
                want.append(int(t[0]))
            cut = trial % (K + 1)  # drafts agree with the sequential tokens up to `cut`
            drafts = want[:K]
            if cut < K:
                drafts[cut] = (drafts[cut] + 1) % V
            toks = np.zeros(K + 1, np.int32)
            acc = O.C.c_int32()
            assert L.orc_slot_spec_verify(spec, O.fp(rows), V, O.ip(O.i32(drafts)), K, O.ip(toks),
                                          O.C.byref(acc)) == 0
            assert acc.value == cut
            assert list(toks[:cut + 1]) == want[:cut + 1]
            # the slot continues exactly as a sequential run of cut + 1 steps
            for i in range(cut + 1):
                t = np.zeros(1, np.int32)
                assert L.orc_slot_step(seq, O.fp(rows[i * V:(i + 1) * V]), V, 0, 1, O.ip(t), None, None, None, None) == 0
                assert int(t[0]) == want[i]
            assert L.orc_slot_rng(spec) == L.orc_slot_rng(seq)
        finally:
            for h in (spec, seq, ref):
                L.orc_slot_free(h)
