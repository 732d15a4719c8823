"""Long full-size parity runs of the GPU path against the oracle (src/server.br:939-1037 per step;
:1173-1216 for speculative rows), through the shared harness with device buffers: workload 2 for 300 steps
(8 rows, V=151936: tokens, logprobs and 10 alternatives per row, histories growing by one token a step),
workload 4 for 30 steps (32 rows, V=262144), workload 5 for 10 verifications (16 sequences x 9 rows, greedy
and sampled), workload 3 for 256 grammar-constrained steps through the JSON-schema entry point, and 40 rounds
of speculative rows with penalties."""
import os
import sys

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import bl_select as BL  # noqa: E402

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpu", "simt"))
import run_parity as RP  # noqa: E402
from _devmem import TorchMem  # noqa: E402
from test_oracle_grammar import C3_SCHEMA  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def device_memory():
    assert torch.cuda.is_available(), "a GPU test ran without a GPU"
    old = RP.MEM
    RP.MEM = TorchMem()
    yield
    RP.MEM = old


def test_workload2_300_steps():
    print("workload 2: 300 steps x 8 rows", flush=True)
    err = RP.run_w2(BL, 300)
    assert err is None, err


def test_workload4_30_steps():
    print("workload 4: 30 steps x 32 rows", flush=True)
    err = RP.run_w4(BL, 30, 32)
    assert err is None, err


def test_workload5_10_verifications():
    print("workload 5: 10 verifications x 16 sequences x 9 rows", flush=True)
    err = RP.run_w5(BL, 10)
    assert err is None, err


def test_workload3_schema_256_steps():
    print("workload 3 through bl_slot_schema: 256 steps", flush=True)
    err = RP.run_w3(BL, 256, schema=C3_SCHEMA)
    assert err is None, err


def test_speculative_penalties_40_rounds():
    print("speculative rows with penalties: 40 rounds", flush=True)
    err = RP.run_spec_penalties(BL, 40)
    assert err is None, err
