"""GPU parity of kernel paths beyond the fixed workloads, through the shared harness with device buffers:
full-vocabulary draws on equal values (bfloat16-rounded, quantised and floored logits: the heap's order),
top_k 250 with 256 logprob alternatives at V=151936 (38 chunks x 256 candidates per row, the merged
list found by radix selection), two small configurations stepped as rows 0 and 1 of an odd-length
vocabulary (row 1 not 16-byte aligned), small configurations on logits floored to a few integers (thousands
of ties at each chunk's top-K bound) and on a ramp (the index-order sum crosses a power of two in nearly
every group), full-vocabulary rows without top-p or min-p (the draw's own candidate cut), and the
bound-rows asynchronous step against the synchronous one."""
import os
import sys

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import bl_select as BL  # noqa: E402

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpu", "simt"))
import run_parity as RP  # noqa: E402
from _devmem import TorchMem  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def device_memory():
    assert torch.cuda.is_available(), "a GPU test ran without a GPU"
    old = RP.MEM
    RP.MEM = TorchMem()
    yield
    RP.MEM = old


def test_top_n_sigma_full_size():
    print("top-n-sigma rows, V=151936: 20 steps", flush=True)
    err = RP.run_tns(BL, 20)
    assert err is None, err


def test_large_top_k_and_alternatives():
    print("top_k 250, n_probs 256, V=151936: 20 steps", flush=True)
    err = RP.run_bigk(BL, 20)
    assert err is None, err


@pytest.mark.parametrize("pair", [(3, 8), (9, 5), (6, 10)])
def test_two_rows_odd_vocabulary(pair):
    print(f"small cases {pair} stepped together, V=5003: 25 steps", flush=True)
    err = RP.run_pair(BL, pair[0], pair[1], 25)
    assert err is None, err


@pytest.mark.parametrize("case", [0, 1, 4, 5, 8, 10])
def test_coarse_logits_tie_at_the_bound(case):
    print(f"small case {case}, logits floored to a few integers: 20 steps", flush=True)
    err = RP.run_small(BL, case, 20, coarse=True)
    assert err is None, err


@pytest.mark.parametrize("case", [7, 8, 10])
def test_ramp_logits_many_crossings(case):
    print(f"small case {case}, logits on a ramp (a power of two crossed in nearly every group): 20 steps", flush=True)
    err = RP.run_small(BL, case, 20, ramp=True)
    assert err is None, err


@pytest.mark.parametrize("quant", ["bf16", "q4", "coarse"])
@pytest.mark.parametrize("case", [2, 3, 6, 9])
def test_full_vocabulary_ties_heap_order(case, quant):
    print(f"small case {case}, {quant} logits (draws on equal values, the heap's order): 20 steps", flush=True)
    err = RP.run_small(BL, case, 20, coarse=quant == "coarse", quant=None if quant == "coarse" else quant)
    assert err is None, err


def test_bf16_ties_full_vocabulary():
    print("two full-vocabulary rows on bfloat16 logits, V=151936: 10 steps", flush=True)
    err = RP.run_bigties(BL, 10)
    assert err is None, err


def test_unfiltered_full_vocabulary_rows():
    print("six full-vocabulary rows without top-p / min-p, V=151936: 12 steps", flush=True)
    err = RP.run_unfiltered(BL, 12)
    assert err is None, err


def test_halfway_tail_terms():
    """A plain draw ranks only the head of its list and counts the tail's ulps of 2^K in any order; a tail
    term exactly halfway between two multiples of u rounds by the parity of the running sum before it. Row 0
    holds 3 copies of such a value (resolved from the parities), row 1 holds 20 (past the eight the split
    resolves: the whole list is ranked)."""
    print("two constructed rows with halfway tail terms, V=151936: 16 steps", flush=True)
    err = RP.run_halfway(BL, 16)
    assert err is None, err


@pytest.mark.parametrize("V", [3000, 5003, 20000])
def test_typical_full_vocabulary_rows(V):
    """typical_p over full-vocabulary lists (the LDS sort at V=3000, the bucket sort above 4096 candidates):
    entropy, the selection order merged from the ranked list's two monotone runs, the walk to typical_p and
    min_keep, then top-p / min-p / dynamic temperature and the draw, against the oracle's slot step."""
    print(f"five typical rows, V={V}", flush=True)
    err = RP.run_typical(BL, 6 if V < 10000 else 2, V)
    assert err is None, err


def test_mirostat_v2_rows():
    print("three mirostat v2 rows, V=5003: 40 steps", flush=True)
    err = RP.run_mirostat(BL, 40)
    assert err is None, err


@pytest.mark.parametrize("case", range(len(RP.DRY_CASES)))
def test_dry_rows(case):
    print(f"DRY case {case}: {RP.DRY_CASES[case]}: 40 steps", flush=True)
    err = RP.run_dry(BL, case, 40)
    assert err is None, err


def test_adaptive_p_rows():
    print("four adaptive-p rows, V=5003: 40 steps; V=151936: 10 steps", flush=True)
    err = RP.run_adaptive(BL, 40)
    assert err is None, err
    err = RP.run_adaptive(BL, 10, 151936)
    assert err is None, err


def test_mirostat_v1_rows():
    print("three mirostat v1 rows, V=5003: 40 steps; V=151936: 12 steps", flush=True)
    err = RP.run_mirostat(BL, 40, 1)
    assert err is None, err
    err = RP.run_mirostat(BL, 12, 1, 151936)
    assert err is None, err


def test_async_step_equals_sync():
    print("bound rows, asynchronous step: 4 steps", flush=True)
    err = RP.run_async(BL, 4)
    assert err is None, err


def test_spec_verify_with_penalties():
    # src/server.br:1173-1216 with frequency/presence/repeat penalties: row i's counts include the drafts before it
    print("speculative rows with penalties: 12 rounds x 4 sequences x 7 rows", flush=True)
    err = RP.run_spec_penalties(BL, 12)
    assert err is None, err
    # 100 drafts: the last row carries up to 200 count corrections
    print("speculative rows with penalties: 3 rounds x 4 sequences x 101 rows", flush=True)
    err = RP.run_spec_penalties(BL, 3, 100)
    assert err is None, err
