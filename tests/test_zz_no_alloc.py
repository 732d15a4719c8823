"""The allocation-free step (bl_sample_rows_noalloc) against the synchronous step of a context
(bl_sample_step): two calls in a row on the one device array, the second with fewer rows and a smaller
vocabulary, each bit-identical to bl_sample_step over slots reset with the same parameters and RNG states and
no history; sizes past the array are rejected."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import bl_select as BL  # noqa: E402

SEED = 5
TOPS = 10

ROWS = [
    dict(temperature=0.0, logprobs=1, n_probs=10),
    dict(temperature=0.7, top_k=20, frequency_penalty=0.5, presence_penalty=0.3, logprobs=1, n_probs=10),
    dict(temperature=1.0, top_p=0.9, logprobs=1, n_probs=10),
    dict(temperature=0.8, top_k=64, min_p=0.05, repeat_penalty=1.1),
    dict(temperature=1.0, mirostat=2, mirostat_tau=5.0, mirostat_eta=0.1),
    dict(temperature=0.9, top_p=0.95, logprobs=1, n_probs=5, post_sampling_probs=1),
    dict(temperature=1.0, top_k=40, xtc_probability=0.5, xtc_threshold=0.1),
    dict(temperature=0.6, logprobs=1, n_probs=3, frequency_penalty=0.2),
]


def bits(xs):
    return np.asarray(xs, np.float32).view(np.uint32).tolist()


def context_step(params, rngs, ptr, ld, V):
    """bl_sample_step over fresh slots: (tokens, logprobs, top ids, top logprobs, RNG states after)."""
    B = len(params)
    ctx = BL.Context(V, B, B)
    try:
        for r in range(B):
            ctx.slot_reset(r, params[r], rngs[r])
        tok, lp, ti, tl = ctx.sample_step(list(range(B)), ptr, ld, top_stride=TOPS)
        return tok, lp, ti, tl, [ctx.slot_rng(r) for r in range(B)]
    finally:
        ctx.close()


def synth(B, V, ld, step):
    buf = torch.full((B * ld,), -7.0, dtype=torch.float32, device="cuda:0")
    gen = BL.Context(V, 1, 1)
    gen.synth_logits(buf.data_ptr(), ld, 2, SEED, step, B, V)
    gen.close()
    torch.cuda.synchronize()
    return buf


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_step_matches_the_context_step_twice(order):
    stream = torch.cuda.current_stream().cuda_stream
    for B, V, ld, step in ((8, 151936, 151936, 0), (3, 50000, 50048, 1)):
        print(f"noalloc case B={B} V={V} ld={ld}", flush=True)
        params = [BL.Params(**ROWS[(r + step) % len(ROWS)]) for r in range(B)]
        rngs = [BL.seed_rng(SEED * 100 + 10 * step + r) for r in range(B)]
        buf = synth(B, V, ld, step)
        got = BL.sample_rows_noalloc(params, rngs, buf.data_ptr(), ld, V, top_stride=TOPS, stream=stream)
        want = context_step(params, rngs, buf.data_ptr(), ld, V)
        assert got[0] == want[0], (B, V, got[0], want[0])
        assert bits(got[1]) == bits(want[1])
        assert got[2] == want[2]
        assert [bits(x) for x in got[3]] == [bits(x) for x in want[3]]
        assert got[4] == want[4] and got[4] != rngs


def test_noalloc_rejects_sizes_past_its_array():
    buf = synth(1, 4096, 4096, 0)
    p = BL.Params(temperature=0.0)
    with pytest.raises(BL.BLError) as e:
        BL.sample_rows_noalloc([p] * (BL.NOALLOC_ROWS + 1), [1] * (BL.NOALLOC_ROWS + 1), buf.data_ptr(), 4096, 4096)
    assert e.value.code == BL.BL_EPARAM
    big = torch.empty(16 * 151936, dtype=torch.float32, device="cuda:0")
    with pytest.raises(BL.BLError) as e:
        BL.sample_rows_noalloc([p] * 16, [1] * 16, big.data_ptr(), 151936, 151936)
    assert e.value.code == BL.BL_EPARAM and "bytes of its array" in str(e.value)
    # the array is intact after a rejection
    tok = BL.sample_rows_noalloc([p], [1], buf.data_ptr(), 4096, 4096)[0]
    assert tok == [int(torch.argmax(buf[:4096]).item())]
