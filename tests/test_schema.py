"""The library's JSON Schema -> GBNF compiler (bl_json_schema_to_gbnf, host code of libbl_select) against the
oracle's restatement of src/schema_grammar.br + src/json.br: the same grammar text, or the same error
message, for every schema below. Host-only: no GPU call is made.

The oracle itself is pinned by test_oracle_grammar.py (test/test_schema_grammar.br's assertions and the
hand-derived workload-3 grammar in tests/golden/c3_schema.gbnf)."""
import os

import pytest

import _oracle as O
import bl_select as BL

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

REFERENCE_SCHEMAS = [  # test/test_schema_grammar.br:22-51
    '{"type":"object","properties":{"n":{"type":"integer"},"s":{"type":"string"},"b":{"type":"boolean"}},'
    '"required":["n"]}',
    '{"type":"object","properties":{"n":{"type":"integer"}},"required":["n"]}',
    '{"type":"object","properties":{"a":{"type":"integer"},"b":{"enum":["x","y"]}}}',
    '{"type":"array","items":{"type":"integer"},"minItems":2,"maxItems":3}',
    '{"anyOf":[{"type":"string"},{"type":"null"}]}',
    '{"type":["integer","boolean"]}',
    '{"const":"fixed"}',
    '{"type":"object","additionalProperties":{"type":"integer"}}',
    '{"type":"string","minLength":2,"maxLength":3}',
    '{"$ref":"#/$defs/node","$defs":{"node":{"type":"object","properties":{"v":{"type":"integer"},'
    '"next":{"anyOf":[{"$ref":"#/$defs/node"},{"type":"null"}]}},"required":["v","next"]}}}',
]

EDGE_SCHEMAS = [
    # const / enum values printed as jv_to_json prints them
    '{"const": 1.5}', '{"const": 1e20}', '{"const": 1.0}', '{"const": -0.0}', '{"const": 1e-7}',
    '{"const": 12345678901234567890}', '{"const": -9223372036854775808}', '{"const": 0.1}',
    '{"const": 123.456e-3}', '{"const": 5e-324}', '{"const": 1.7976931348623157e308}', '{"const": 1e400}',
    '{"const": null}', '{"const": true}', '{"const": [1, "a", null, {"k": false}]}',
    '{"const": {"b": 1, "a": [], "b": 2}}', '{"const": "q\\"uote\\\\ \\n\\t\\r \\u0001 \\u00e9 \\ud83d\\ude00 /\\/"}',
    '{"enum": ["x", 1, 2.50, null, false, {"a": {"b": [1.25]}}]}', '{"enum": 5}',
    # keys: escaping, non-ASCII names, duplicates
    '{"type":"object","properties":{"a\\"b":{"type":"integer"},"new\\nline":{"type":"string"},'
    '"\\u043a\\u043b\\u044e\\u0447":{"type":"boolean"},"emoji\\ud83d\\ude00":{"type":"null"}},'
    '"required":["a\\"b"]}',
    '{"type":"object","properties":{"a":{"type":"integer"},"a":{"type":"string"}},"required":["a"]}',
    '{"type":"object","properties":{"x y":{"type":"integer"},"x-y":{"type":"string"}}}',
    # combinators
    '{"anyOf":[{"type":"string"}],"oneOf":[{"type":"integer"},{"type":"string"}]}',
    '{"anyOf":[]}', '{"oneOf":[true,{"type":"number"}]}',
    '{"type":["object","array","string"],"properties":{"k":{"type":"integer"}},"items":{"type":"null"}}',
    '{"type":"object","properties":{"p":{"type":["string","integer"]},"q":{"anyOf":[{"type":"string"},'
    '{"type":"string"}]}},"required":["q"]}',
    # objects
    '{"properties":{"a":{"type":"integer"}}}', '{"type":"object"}', '{"type":"object","additionalProperties":true}',
    '{"type":"object","additionalProperties":false,"properties":{"a":{}}}',
    '{"type":"object","additionalProperties":{},"properties":{"a":{"type":"integer"},"b":{"type":"string"}}}',
    '{"type":"object","additionalProperties":true,"properties":{"a":{"type":"integer"}},"required":["a"]}',
    '{"type":"object","properties":{"a":{"type":"integer"},"b":{"type":"integer"},"c":{"type":"integer"}},'
    '"required":["c",1,"a"]}',
    '{"type":"object","properties":{"":{"type":"integer"}},"required":[0]}',
    '{"type":"object","properties":{"o":{"type":"object","properties":{"i":{"type":"object","properties":'
    '{"z":{"const":3}}}}}}}',
    # arrays and strings
    '{"type":"array"}', '{"type":"array","maxItems":0}', '{"type":"array","minItems":1}',
    '{"type":"array","minItems":1,"maxItems":1}', '{"type":"array","minItems":0,"maxItems":5,"items":true}',
    '{"type":"array","minItems":2.0,"maxItems":4.0,"items":{"type":"boolean"}}',
    '{"type":"array","items":{"type":"array","items":{"type":"array"}}}',
    '{"type":"string","minLength":3}', '{"type":"string","maxLength":0}', '{"type":"string","minLength":2.9}',
    '{"type":"string","maxLength":4.0}', '{"type":"string","minLength":0,"maxLength":7}',
    # references
    '{"$ref":"#"}', '{"type":"object","properties":{"self":{"$ref":"#"}}}',
    '{"definitions":{"a":{"type":"integer"}},"type":"object","properties":{"x":{"$ref":"#/definitions/a"},'
    '"y":{"$ref":"#/definitions/a"}}}',
    '{"$ref":"", "type":"integer"}', '{"$ref": 3, "type":"boolean"}',
    # root aliases and whitespace
    'true', 'false', '{}', '{"type":"integer"}', '{"type":"null"}', '  {"type" : "number"}\n\t ',
    '{"type": 7}',
]

ERROR_SCHEMAS = [
    '5', '"s"', '[]', '{"type": [1, "string"]}', '{"type":"object","properties":{"a":5}}',
    '{"type":"object","properties":{"a":null}}',
    '{"type":"tuple"}', '{"type":["string","date"]}', '{"enum":[]}', '{"$ref":"http://x/y"}', '{"$ref":"#foo"}',
    '{"$ref":"#/definitions/missing"}', '{"$ref":"#/"}', '{"type":"array","minItems":3,"maxItems":2}',
    '{"type":"object","properties":{' + ",".join(f'"p{i}":{{}}' for i in range(129)) + '}}',
    # json_parse errors, positions counted in code points
    '', '   ', '{"a":1} x', '{"é":1} ]', '{"a" 1}', '{"a":1,}', '{"a":1 "b":2}', '[1 2]', '[1,', '{"a":',
    '"abc', '"a\\q"', '"\\u12"', '"\\u12é3"', '"\\u12g4"', '"\\uD800"', '"\\uD800\\u0041"', '"\\uDC00"',
    '"a\x01b"', '"\\', '-', '1.', '1e', '1e+', 'tru', 'nul', '01', '{"é": 1 , éx}', '{1: 2}',
    '[' * 129 + ']' * 129,
]


def lib_gbnf(schema):
    return BL.json_schema_to_gbnf(schema)


@pytest.mark.parametrize("schema", REFERENCE_SCHEMAS + EDGE_SCHEMAS)
def test_schema_text_matches_oracle(schema):
    assert lib_gbnf(schema) == O.json_schema_to_gbnf(schema)


def test_deep_nesting_at_the_limit():
    ok = '[' * 128 + ']' * 128
    assert lib_gbnf('{"const": ' + ok + '}') == O.json_schema_to_gbnf('{"const": ' + ok + '}')


@pytest.mark.parametrize("schema", ERROR_SCHEMAS)
def test_schema_errors_match_oracle(schema):
    with pytest.raises(ValueError) as want:
        O.json_schema_to_gbnf(schema)
    with pytest.raises(BL.BLError) as got:
        lib_gbnf(schema)
    assert got.value.code == BL.BL_ESCHEMA
    assert str(got.value) == f"{want.value} (code {BL.BL_ESCHEMA})"


def test_workload3_schema_is_the_golden_grammar():
    from test_oracle_grammar import C3_SCHEMA
    with open(os.path.join(GOLDEN, "c3_schema.gbnf")) as f:
        assert lib_gbnf(C3_SCHEMA) == f.read()


def test_library_grammar_keeps_the_reference_language():
    # test/test_schema_grammar.br:22-27, on the library's text (parsed and walked by the oracle's grammar engine)
    from test_oracle_grammar import G
    g1 = G(lib_gbnf(REFERENCE_SCHEMAS[0]))
    assert g1.accepts('{"n": 5}') and g1.accepts('{"n":5,"s":"x","b":true}') and not g1.accepts('{"s": "x"}')
    assert not g1.viable('{"n": 5} ') and not g1.accepts('{"n": 5.5}')
    g4 = G(lib_gbnf(REFERENCE_SCHEMAS[3]))
    assert g4.accepts("[1, 2]") and not g4.accepts("[1]") and not g4.viable("[1,2,3,")


def test_invalid_utf8_and_buffer_size():
    with pytest.raises(BL.BLError) as e:
        lib_gbnf(b'{"const": "\xff"}')
    assert e.value.code == BL.BL_ESCHEMA
    import ctypes as C
    t = b'{"type":"integer"}'
    n = C.c_size_t(0)
    assert BL.lib().bl_json_schema_to_gbnf(t, len(t), None, 0, C.byref(n)) == 0 and n.value > 0
    small = C.create_string_buffer(n.value)  # no room for the NUL
    assert BL.lib().bl_json_schema_to_gbnf(t, len(t), small, n.value, None) == BL.BL_EPARAM


def _random_schema(rng, depth=0):
    """A random schema over the keywords json_schema_to_gbnf reads (seeded: the cases are fixed)."""
    import json
    def lit():
        return rng.choice([0, -3, 2.5, 1e21, "s", "a\"b", "é", True, False, None, [1, "x"], {"k": [None]}])
    keys = ["alpha", "b-c", "d e", "ü", "", "x1"]
    kind = rng.randrange(12 if depth < 3 else 7)
    if kind == 0:
        return {"type": rng.choice(["string", "integer", "number", "boolean", "null"])}
    if kind == 1:
        return {"const": lit()}
    if kind == 2:
        return {"enum": [lit() for _ in range(rng.randrange(1, 4))]}
    if kind == 3:
        s = {"type": "string"}
        if rng.random() < 0.7:
            s["minLength"] = rng.choice([0, 1, 3, 2.0])
        if rng.random() < 0.6:
            s["maxLength"] = rng.choice([0, 4, 9, 5.0])
        return s
    if kind == 4:
        return rng.choice([True, False, {}])
    if kind == 5:
        return {"type": [rng.choice(["string", "integer", "boolean", "null", "number"]) for _ in range(2)]}
    if kind == 6:
        return {"$ref": "#/$defs/" + rng.choice(["n", "m"])}
    if kind in (7, 8):
        props = {k: _random_schema(rng, depth + 1) for k in rng.sample(keys, rng.randrange(0, 4))}
        s = {"type": "object", "properties": props}
        if props and rng.random() < 0.6:
            s["required"] = rng.sample(list(props), rng.randrange(0, len(props) + 1))
        if rng.random() < 0.4:
            s["additionalProperties"] = rng.choice([True, False, {"type": "integer"}, {}])
        return s
    if kind == 9:
        s = {"type": "array"}
        if rng.random() < 0.7:
            s["items"] = _random_schema(rng, depth + 1)
        lo = rng.choice([None, 0, 1, 2, 3])
        hi = rng.choice([None, 0, 1, 2, 4])
        if lo is not None:
            s["minItems"] = lo
        if hi is not None and (lo is None or hi >= lo):
            s["maxItems"] = hi
        return s
    key = rng.choice(["anyOf", "oneOf"])
    return {key: [_random_schema(rng, depth + 1) for _ in range(rng.randrange(1, 4))]}


def test_random_schemas_match_oracle():
    import json
    import random
    rng = random.Random(1234)
    for case in range(400):
        root = _random_schema(rng)
        if isinstance(root, dict) and rng.random() < 0.5:
            root = dict(root)
            root["$defs"] = {"n": _random_schema(rng, 2), "m": {"type": "integer"}}
        text = json.dumps(root, ensure_ascii=rng.random() < 0.5)
        try:
            want = O.json_schema_to_gbnf(text)
        except ValueError as e:
            with pytest.raises(BL.BLError) as got:
                lib_gbnf(text)
            assert str(got.value) == f"{e} (code {BL.BL_ESCHEMA})", (case, text)
            continue
        assert lib_gbnf(text) == want, (case, text)


def test_mutated_schema_texts_match_oracle():
    # byte-level mutations of valid schema texts exercise json_parse's error paths and positions
    import random
    rng = random.Random(99)
    alphabet = '{}[]":,\\ \n\tu0123456789abcdefé-+.eEtrnl'
    for case in range(1500):
        base = rng.choice(REFERENCE_SCHEMAS + EDGE_SCHEMAS[:20])
        s = list(base)
        for _ in range(rng.randrange(1, 4)):
            op, i = rng.randrange(3), rng.randrange(len(s) + 1)
            if op == 0 and s:
                del s[min(i, len(s) - 1)]
            elif op == 1:
                s.insert(i, rng.choice(alphabet))
            elif s:
                s[min(i, len(s) - 1)] = rng.choice(alphabet)
        text = "".join(s)
        try:
            want = O.json_schema_to_gbnf(text)
        except ValueError as e:
            with pytest.raises(BL.BLError) as got:
                lib_gbnf(text)
            assert str(got.value) == f"{e} (code {BL.BL_ESCHEMA})", (case, text)
            continue
        assert lib_gbnf(text) == want, (case, text)
