"""GPU parity of the grammar-constrained path (libbl_select.so through its C ABI) against the oracle.

Allow-bitmasks and tokens must be identical. Workload 3: greedy decode of 256
steps over the synthetic 151936-token vocabulary under the JSON-Schema grammar of tests/golden, the
mask's CRC32, the forced-EOS flag and the token compared at every step with the oracle's literal
restatement of src/server.br:308-361. Seven small grammars over a byte-level vocabulary of lone bytes,
UTF-8 fragments and whole characters check the carry of unfinished UTF-8 sequences, the
trailing-U+FFFD rule and the reference's error outcomes. The same harness runs on the CPU emulator
(tests/test_simt_kernels.py); here its buffers are device memory.
"""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import bl_select as BL  # noqa: E402
import _oracle as O  # noqa: E402

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpu", "simt"))
import run_parity as RP  # noqa: E402
from _devmem import TorchMem  # noqa: E402


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module", autouse=True)
def device_memory():
    assert torch.cuda.is_available(), "a GPU test ran without a GPU"
    old = RP.MEM
    RP.MEM = TorchMem()
    yield
    RP.MEM = old


def test_workload3_masks_and_tokens():
    say("workload 3: 256 greedy grammar steps, masks and tokens")
    err = RP.run_w3(BL, 256)
    assert err is None, err


def test_workload3_through_the_schema_entry_point():
    # response_format json_schema (src/server.br:733-745): the schema text itself, compiled by the library
    from test_oracle_grammar import C3_SCHEMA
    say("workload 3 via bl_slot_schema: 64 greedy grammar steps, masks and tokens")
    err = RP.run_w3(BL, 64, schema=C3_SCHEMA)
    assert err is None, err


def test_schema_errors_on_a_slot():
    say("schema errors on a slot")
    blob, off, eos = RP.grammar_vocab(np.random.default_rng(1), 50)
    V = len(off) - 1
    ctx = BL.Context(V, 1, 1)
    ctx.set_eog(eos, [])
    ctx.set_vocab(blob, off)
    ctx.slot_reset(0, BL.Params(), 1)
    with pytest.raises(BL.BLError) as e:
        ctx.slot_schema(0, '{"type":"tuple"}')
    assert e.value.code == BL.BL_ESCHEMA
    assert "the JSON schema is not supported: unsupported schema type 'tuple'" in str(e.value)
    with pytest.raises(BL.BLError) as e:  # a recursive schema has no finite automaton
        ctx.slot_schema(0, '{"$ref":"#/$defs/n","$defs":{"n":{"type":"object","properties":'
                           '{"next":{"anyOf":[{"$ref":"#/$defs/n"},{"type":"null"}]}}}}}')
    assert e.value.code == BL.BL_EUNSUPPORTED
    ctx.slot_schema(0, '{"enum":["{", "{}"]}')  # a valid schema attaches
    x = np.full(V, -1.0, np.float32)
    x[ord("}")] = 7.0
    x[ord('"')] = 5.0
    buf = torch.from_numpy(x).to("cuda:0")
    assert ctx.sample_step([0], buf.data_ptr(), V)[0][0] == ord('"')
    ctx.close()


@pytest.mark.parametrize("case", range(len(RP.GRAMMAR_CASES)))
def test_grammar_cases(case):
    say(f"grammar case {case}: {RP.GRAMMAR_CASES[case]!r}")
    err = RP.run_grammar_case(BL, case, 120)
    assert err is None, err


@pytest.mark.parametrize("case", range(len(RP.GRAMMAR_SAMPLED)))
def test_sampled_grammar_cases(case):
    gc, kw, sigma = RP.GRAMMAR_SAMPLED[case]
    say(f"sampled grammar case {case}: grammar {gc}, {kw}, logits N(0, {sigma}^2)")
    err = RP.run_grammar_case(BL, gc, 120, kw, sigma)
    assert err is None, err


@pytest.mark.parametrize("top_k", [0, 40])
@pytest.mark.parametrize("case", range(len(RP.GRAMMAR_CASES)))
def test_greedy_grammar_ties(case, top_k):
    """Greedy grammar rows on logits in steps of 0.5 (equal allowed maxima at most steps): the lowest index
    while the widening levels rank by top_k_select, the heap's first allowed token once a level reaches V."""
    say(f"grammar ties: case {case}, top_k {top_k}")
    err = RP.run_grammar_case(BL, case, 80, {"top_k": top_k} if top_k else None, quant=0.5)
    assert err is None, err


@pytest.mark.parametrize("top_k", [0, 40])
@pytest.mark.parametrize("case", range(len(RP.GRAMMAR_CASES)))
def test_sampled_grammar_ties(case, top_k):
    """Sampled grammar rows (T 0.8) on logits in steps of 0.5: a draw on equal allowed values takes the
    allowed token the heap's extraction order puts at the drawn position (top_k 0, or a level of V)."""
    say(f"sampled grammar ties: case {case}, top_k {top_k}")
    kw = {"temperature": 0.8}
    if top_k:
        kw["top_k"] = top_k
    err = RP.run_grammar_case(BL, case, 80, kw, quant=0.5)
    assert err is None, err


@pytest.mark.parametrize("case", range(len(RP.JSON_CASES)))
def test_json_object_cases(case):
    say(f"JSON-object case {case}: {RP.JSON_CASES[case]}")
    err = RP.run_json_case(BL, case, 150)
    assert err is None, err


def test_json_object_errors():
    say("JSON-object errors")
    blob, off, eos = RP.json_vocab(np.random.default_rng(2), 20)
    V = len(off) - 1
    ctx = BL.Context(V, 1, 1)
    ctx.set_eog(eos, [])
    ctx.set_vocab(blob, off)
    ctx.slot_reset(0, BL.Params(temperature=1.0, mirostat=2), 1)
    with pytest.raises(BL.BLError) as e:
        ctx.slot_json_object(0)
    assert e.value.code == BL.BL_EPARAM and "cannot be combined with constrained decoding" in str(e.value)
    ctx.slot_reset(0, BL.Params(temperature=0.0), 1)
    ctx.slot_json_object(0)
    x = np.zeros(V, np.float32)
    x[[i for i in range(V) if blob[off[i]:off[i + 1]] == b"{"]] = 5.0
    buf = torch.from_numpy(x).to("cuda:0")
    assert blob[off[ctx.sample_step([0], buf.data_ptr(), V)[0][0]]:][:1] == b"{"
    ctx.close()


def test_grammar_errors():
    say("grammar errors")
    blob, off, eos = RP.grammar_vocab(np.random.default_rng(1), 50)
    V = len(off) - 1
    ctx = BL.Context(V, 2, 2)
    ctx.set_eog(eos, [])
    ctx.set_vocab(blob, off)
    ctx.slot_reset(0, BL.Params(), 1)
    with pytest.raises(BL.BLError) as e:
        ctx.slot_grammar(0, 'root ::= "a" b\n')
    assert e.value.code == BL.BL_EGRAMMAR and "grammar: undefined rule 'b'" in str(e.value)
    with pytest.raises(BL.BLError) as e:
        ctx.slot_grammar(0, 'root ::= "a"{3,1}\n')
    assert e.value.code == BL.BL_EGRAMMAR and "repetition maximum is smaller than its minimum" in str(e.value)
    with pytest.raises(BL.BLError) as e:  # reachable recursion: no finite automaton
        ctx.slot_grammar(0, 'root ::= v\nv ::= "[" v? "]"\n')
    assert e.value.code == BL.BL_EUNSUPPORTED
    with pytest.raises(BL.BLError) as e:  # the reference's 20,000-stack guard
        ctx.slot_grammar(0, 'root ::= a\na ::= a "x" | "y"\n')
    assert e.value.code == BL.BL_EGRAMMAR_AMBIG
    ctx.slot_reset(1, BL.Params(temperature=0.8), 1)
    ctx.slot_grammar(1, 'root ::= "a"\n')  # sampled grammar rows have a device path
    ctx.slot_reset(1, BL.Params(temperature=0.8, top_n_sigma=1.0), 1)
    with pytest.raises(BL.BLError) as e:
        ctx.slot_grammar(1, 'root ::= "a"\n')
    assert e.value.code == BL.BL_EUNSUPPORTED
    # a finished sentence: forced EOS (src/server.br:319-321); with ignore_eos nothing is allowed (:361)
    x = np.full(V, -1.0, np.float32)
    x[ord("{")] = 5.0
    buf = torch.from_numpy(x).to("cuda:0")
    for ignore in (0, 1):
        ctx.slot_reset(0, BL.Params(ignore_eos=ignore), 1)
        ctx.slot_grammar(0, 'root ::= "{"\n')
        assert ctx.sample_step([0], buf.data_ptr(), V)[0][0] == ord("{")
        if ignore:
            with pytest.raises(BL.BLError) as e:
                ctx.sample_step([0], buf.data_ptr(), V)
            assert e.value.code == BL.BL_EGRAMMAR_REJECT
        else:
            assert ctx.sample_step([0], buf.data_ptr(), V)[0][0] == eos
    ctx.close()
