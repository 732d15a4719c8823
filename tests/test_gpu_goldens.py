"""The device against the committed golden vectors of workload 2 (tests/golden/c2_golden.npz: 12 steps of
8 rows: tokens, logprobs and the 10 alternatives, bit for bit)."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import bl_select as BL  # noqa: E402

V, B, SEED = 151936, 8, 2


def test_device_matches_c2_golden():
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c2_golden.npz"))
    steps = len(g["tokens"]) // B
    ctx = BL.Context(V, B, B)
    for r in range(B):
        p = BL.Params(temperature=[0.0, 0.7, 1.0][r % 3], top_k=[0, 20, 64][r // 3], top_p=[1.0, 0.9][r % 2],
                      frequency_penalty=0.5, presence_penalty=0.3, logprobs=1, n_probs=10)
        reply = BL.workload_ids(1, 2, SEED, r, 4096, V)
        ctx.slot_reset(r, p, BL.seed_rng(SEED + r), history=reply, reply=reply,
                       bias=BL.workload_bias(2, SEED, r, 300, V, -100.0, 100.0))
    buf = torch.empty(B * V, dtype=torch.float32, device="cuda:0")
    for t in range(steps):
        ctx.synth_logits(buf.data_ptr(), V, 2, SEED, t, B, V)
        tok, lp, ti, tl = ctx.sample_step(list(range(B)), buf.data_ptr(), V, top_stride=10)
        sl = slice(t * B, (t + 1) * B)
        assert tok == g["tokens"][sl].tolist(), f"step {t}"
        assert np.array_equal(np.array(lp, np.float32), g["logprobs"][sl]), f"step {t}"
        assert np.array_equal(np.array(ti, np.int32).ravel(), g["top_ids"][t * B * 10:(t + 1) * B * 10])
        assert np.array_equal(np.array(tl, np.float32).ravel(), g["top_logprobs"][t * B * 10:(t + 1) * B * 10])
    ctx.close()
