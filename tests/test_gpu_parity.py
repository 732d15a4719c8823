"""GPU parity: the HIP path (libbl_select.so through its C ABI) against the CPU oracle.

Token ids, accepted-prefix lengths, logprobs and probabilities must be bit-identical (the device
reproduces the reference's sequential float32 sums exactly, and its expf/logf are glibc's). Inputs
are the seeded synthetic workloads, generated on the device by the library and on the host by the
oracle from the same integer hash.
"""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import bl_select as BL  # noqa: E402
import _oracle as O  # noqa: E402
from _cases import CASES, EOGS, EOS, SMALL_V, small_case_inputs, small_case_logits  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
V_QWEN, V_GEMMA = 151936, 262144


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def cuda():
    assert torch.cuda.is_available(), "a GPU test ran without a GPU"
    return torch.device("cuda:0")


def lp_close(a, b):
    """logprobs and probabilities are bit-identical (NaN equal to NaN)"""
    a, b = np.float32(a), np.float32(b)
    return (a != a and b != b) or a.view(np.uint32) == b.view(np.uint32)


# ------------------------------------------------------------------ device math, exhaustive
def test_math_exhaustive(cuda):
    say("math digest: expf/tanhf/logf and three powf families over all 2^32 inputs")
    want = np.fromfile(os.path.join(GOLDEN, "math_digest.bin"), dtype="<u8").reshape(6, 4096)
    ctx = BL.Context(1024, 1, 1)
    for fn, name in ((0, "expf"), (1, "tanhf"), (2, "logf"), (3, "powf(x, 0.7)"), (4, "powf(2, x)"),
                     (5, "powf(x, y)")):
        got = np.array(ctx.math_digest(fn, 0, 4096), dtype=np.uint64)
        bad = np.nonzero(got != want[fn])[0]
        assert len(bad) == 0, f"{name}: {len(bad)} blocks differ, first {bad[:8]}"
    ctx.close()


def test_synth_device_equals_host(cuda):
    ctx = BL.Context(V_QWEN, 1, 2)
    buf = torch.empty(2 * V_QWEN, dtype=torch.float32, device=cuda)
    for cfg, seed, step in ((1, 1234, 3), (2, 2, 5), (5, 5, 1)):
        ctx.synth_logits(buf.data_ptr(), V_QWEN, cfg, seed, step, 2 if cfg != 1 else 1, V_QWEN)
        torch.cuda.synchronize()
        got = buf.cpu().numpy()
        for r in range(2 if cfg != 1 else 1):
            want = O.synth_logits(cfg, seed, step, r, V_QWEN)
            assert np.array_equal(got[r * V_QWEN:(r + 1) * V_QWEN].view(np.uint32), want.view(np.uint32)), (cfg, r)
    ctx.close()


# ------------------------------------------------------------------ workload 1
def test_workload1_tokens(cuda):
    steps = 300
    say(f"workload 1: {steps} steps")
    V, seed = V_QWEN, 1234
    want = np.zeros(steps, np.int32)
    assert O.lib().orc_run_c1(seed, steps, O.ip(want), None) == 0, O.last_error()
    golden = np.loadtxt(os.path.join(GOLDEN, "c1_tokens.txt"), dtype=np.int64)
    assert np.array_equal(want[:len(golden)], golden), "oracle drifted from its committed stream"
    ctx = BL.Context(V, 1, 1)
    p = BL.Params(temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64)
    ctx.slot_reset(0, p, BL.seed_rng(seed), history=BL.workload_ids(0, 1, seed, 0, 512, V))
    buf = torch.empty(V, dtype=torch.float32, device=cuda)
    got = []
    for t in range(steps):
        ctx.synth_logits(buf.data_ptr(), V, 1, seed, t, 1, V)
        tok, _, _, _ = ctx.sample_step([0], buf.data_ptr(), V)
        got.append(tok[0])
    got = np.array(got)
    assert np.array_equal(got, want), f"first divergence at step {int(np.argmax(got != want))}"
    assert ctx.slot_rng(0) != BL.seed_rng(seed)
    ctx.close()


# ------------------------------------------------------------------ workload 2 (the benchmark workload)
def c2_context(V, seed, cuda):
    ctx = BL.Context(V, 8, 8)
    for r in range(8):
        T = [0.0, 0.7, 1.0][r % 3]
        k = [0, 20, 64][r // 3]
        tp = [1.0, 0.9][r % 2]
        p = BL.Params(temperature=T, top_k=k, top_p=tp, frequency_penalty=0.5, presence_penalty=0.3, logprobs=1,
                      n_probs=10)
        reply = BL.workload_ids(1, 2, seed, r, 4096, V)
        ctx.slot_reset(r, p, BL.seed_rng(seed + r), history=reply, reply=reply,
                       bias=BL.workload_bias(2, seed, r, 300, V, -100.0, 100.0))
    return ctx


def test_workload2_tokens_logprobs(cuda):
    steps = 40
    say(f"workload 2: {steps} steps x 8 rows")
    V, seed, B = V_QWEN, 2, 8
    wt = np.zeros(steps * B, np.int32)
    wl = np.zeros(steps * B, np.float32)
    wi = np.zeros(steps * B * 10, np.int32)
    wp = np.zeros(steps * B * 10, np.float32)
    assert O.lib().orc_run_c2(seed, steps, B, O.ip(wt), O.fp(wl), O.ip(wi), O.fp(wp), None) == 0, O.last_error()
    ctx = c2_context(V, seed, cuda)
    buf = torch.empty(B * V, dtype=torch.float32, device=cuda)
    for t in range(steps):
        ctx.synth_logits(buf.data_ptr(), V, 2, seed, t, B, V)
        tok, lp, ti, tl = ctx.sample_step(list(range(B)), buf.data_ptr(), V, top_stride=10)
        for r in range(B):
            a = t * B + r
            assert tok[r] == wt[a], f"step {t} row {r}: token {tok[r]} != {wt[a]}"
            assert lp_close(lp[r], wl[a]), f"step {t} row {r}: logprob {lp[r]!r} vs {wl[a]!r}"
            assert ti[r] == list(wi[a * 10:(a + 1) * 10]), f"step {t} row {r}: alternatives differ"
            for q in range(10):
                assert lp_close(tl[r][q], wp[a * 10 + q]), f"step {t} row {r} alt {q}"
    ctx.close()


# ------------------------------------------------------------------ workload 4
def test_workload4_softcap_topk(cuda):
    steps, B = 6, 32
    say(f"workload 4: {steps} steps x {B} rows")
    V, seed = V_GEMMA, 7
    wt = np.zeros(steps * B, np.int32)
    wl = np.zeros(steps * B, np.float32)
    wi = np.zeros(steps * B * 20, np.int32)
    wp = np.zeros(steps * B * 20, np.float32)
    assert O.lib().orc_run_c4(seed, steps, B, O.ip(wt), O.fp(wl), O.ip(wi), O.fp(wp), None) == 0, O.last_error()
    ctx = BL.Context(V, B, B)
    for r in range(B):
        p = BL.Params(temperature=1.0, top_k=64, top_p=0.95, logprobs=1, n_probs=20, final_softcap=30.0)
        ctx.slot_reset(r, p, BL.seed_rng(seed + r))
    buf = torch.empty(B * V, dtype=torch.float32, device=cuda)
    for t in range(steps):
        ctx.synth_logits(buf.data_ptr(), V, 4, seed, t, B, V)
        tok, lp, ti, tl = ctx.sample_step(list(range(B)), buf.data_ptr(), V, top_stride=20)
        for r in range(B):
            a = t * B + r
            assert tok[r] == wt[a], f"step {t} row {r}"
            assert lp_close(lp[r], wl[a]), f"step {t} row {r}: {lp[r]!r} vs {wl[a]!r}"
            assert ti[r] == list(wi[a * 20:(a + 1) * 20])
            for q in range(20):
                assert lp_close(tl[r][q], wp[a * 20 + q]), (t, r, q, ti[r][q], tl[r][q], float(wp[a * 20 + q]), lp[r])
    ctx.close()


# ------------------------------------------------------------------ workload 5
def test_workload5_spec_verify(cuda):
    steps, S, K = 2, 16, 8
    say(f"workload 5: {steps} steps x {S} sequences x {K + 1} rows")
    V, seed = V_QWEN, 5
    R = S * (K + 1)
    wgt = np.zeros(steps * R, np.int32)
    wga = np.zeros(steps * S, np.int32)
    wst = np.zeros(steps * R, np.int32)
    wsa = np.zeros(steps * S, np.int32)
    assert O.lib().orc_run_c5(seed, steps, S, O.ip(wgt), O.ip(wga), O.ip(wst), O.ip(wsa), None) == 0, O.last_error()
    g = BL.Context(V, S, R)
    s = BL.Context(V, S, R)
    for b in range(S):
        g.slot_reset(b, BL.Params(), BL.seed_rng(seed + b))
        s.slot_reset(b, BL.Params(temperature=0.7), BL.seed_rng(seed + b))
    buf = torch.empty(R * V, dtype=torch.float32, device=cuda)
    for t in range(steps):
        g.synth_logits(buf.data_ptr(), V, 5, seed, t, R, V)
        am = torch.argmax(buf.view(R, V), dim=1).cpu().numpy()
        drafts = []
        for b in range(S):
            drafts += BL.workload_drafts(seed, t, b, [int(x) for x in am[b * (K + 1):b * (K + 1) + K]], V)
        gt, ga = g.spec_verify(list(range(S)), K, buf.data_ptr(), V, drafts)
        st, sa = s.spec_verify(list(range(S)), K, buf.data_ptr(), V, drafts)
        assert gt == list(wgt[t * R:(t + 1) * R]) and ga == list(wga[t * S:(t + 1) * S]), f"greedy step {t}"
        assert sa == list(wsa[t * S:(t + 1) * S]), f"sampled accepted lengths, step {t}"
        assert st == list(wst[t * R:(t + 1) * R]), f"sampled tokens, step {t}"
    g.close()
    s.close()


# ------------------------------------------------------------------ many small configurations
@pytest.mark.parametrize("case", range(len(CASES)))
def test_small_vocab_cases(cuda, case):
    V, steps = SMALL_V, 25
    kw = CASES[case]
    say(f"small case {case}: {kw}")
    rng, hist, reply, bias = small_case_inputs(case)
    eos, eogs = EOS, EOGS
    ctx = BL.Context(V, 2, 2)
    ctx.set_eog(eos, eogs)
    p = BL.Params(**kw)
    ctx.slot_reset(1, p, BL.seed_rng(100 + case), history=hist, reply=reply, bias=bias)
    op = O.params(**kw)
    hh, rr = O.i32(hist), O.i32(reply)
    bi, bv = O.i32(list(bias.keys())), O.f32(list(bias.values()))
    L = O.lib()
    # the oracle takes the end-of-generation set from its registry (src/sampling.br:200-213)
    L.orc_set_eog_tokens(O.ip(O.i32([eos] + eogs)), 1 + len(eogs), -1)
    h = L.orc_slot_new(O.C.byref(op), BL.seed_rng(100 + case),
                       O.ip(hh), len(hist), O.ip(rr), len(reply), O.ip(bi), O.fp(bv), len(bias))
    buf = torch.empty(V, dtype=torch.float32, device=cuda)
    wants = 1 if kw.get("logprobs") else 0
    n_probs = kw.get("n_probs", 0)
    try:
        for t in range(steps):
            x = small_case_logits(rng)
            buf.copy_(torch.from_numpy(x))
            torch.cuda.synchronize()
            tok, lp, ti, tl = ctx.sample_step([1], buf.data_ptr(), V, top_stride=max(n_probs, 1))
            ot = np.zeros(1, np.int32)
            olp = np.zeros(1, np.float32)
            oti = np.full(max(n_probs, 1), -1, np.int32)  # no alternative: -1, as the library writes
            otl = np.zeros(max(n_probs, 1), np.float32)
            eog = O.C.c_int()
            assert L.orc_slot_step(h, O.fp(x), V, wants, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl),
                                   O.C.byref(eog)) == 0
            assert tok[0] == ot[0], f"case {case} step {t}: {tok[0]} vs {ot[0]}"
            if wants and not eog.value:
                assert lp_close(lp[0], olp[0]), f"case {case} step {t}: logprob {lp[0]} vs {olp[0]}"
                assert ti[0][:n_probs] == list(oti[:n_probs])
                assert all(lp_close(tl[0][q], otl[q]) for q in range(n_probs))
        assert ctx.slot_rng(1) == L.orc_slot_rng(h)
    finally:
        L.orc_slot_free(h)
        L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
        ctx.close()


def test_errors_are_reported(cuda):
    ctx = BL.Context(1000, 2, 2)
    ctx.slot_reset(0, BL.Params(temperature=1.0, top_n_sigma=1.5), 1)  # top-n-sigma has a device path
    ctx.slot_reset(0, BL.Params(temperature=1.0, dynatemp_range=0.5, dynatemp_exponent=2.0), 1)  # device path
    ctx.slot_reset(0, BL.Params(temperature=1.0, mirostat=1), 1)  # device path
    ctx.slot_reset(0, BL.Params(temperature=1.0, dry_multiplier=0.8), 1)  # device path
    ctx.slot_reset(0, BL.Params(temperature=1.0, adaptive_target=0.3), 1)  # device path
    with pytest.raises(BL.BLError) as e:
        ctx.slot_reset(0, BL.Params(temperature=1.0, adaptive_target=0.3, logprobs=1, post_sampling_probs=1), 1)
    assert e.value.code == BL.BL_EPARAM
    with pytest.raises(BL.BLError) as e:
        ctx.slot_reset(0, BL.Params(temperature=1.0, dry_multiplier=0.8, dry_penalty_last_n=4096), 1)
    assert e.value.code == BL.BL_EUNSUPPORTED
    with pytest.raises(BL.BLError) as e:
        ctx.slot_reset(0, BL.Params(temperature=1.0, mirostat=2, logprobs=1, post_sampling_probs=1), 1)
    assert e.value.code == BL.BL_EPARAM and "standard unconstrained sampling chain" in str(e.value)
    # the typical filter over a full-vocabulary list longer than the short-list path: drawn on the device
    ctx.slot_reset(0, BL.Params(temperature=1.0, typical_p=0.5), 1)
    row = torch.randn(1000, device=cuda)
    assert 0 <= ctx.sample_step([0], row.data_ptr(), 1000)[0][0] < 1000
    with pytest.raises(BL.BLError) as e:
        ctx.slot_reset(0, BL.Params(), 1, bias={5000: 1.0})
    assert e.value.code == BL.BL_EPARAM and "outside the vocabulary" in str(e.value)
    buf = torch.zeros(1000, device=cuda)
    with pytest.raises(BL.BLError):
        ctx.sample_step([1], buf.data_ptr(), 1000)  # slot 1 was never set up
    ctx.close()
