"""Pins the oracle's sampling restatement (oracle/sampling.cpp).

Part 1 transliterates every assertion of the reference's test/test_sampling.br (line numbers cited).
Part 2 adds checks the mathematics fixes: the xorshift64 stream and its float conversion computed with
Python integers, rankings against an independent lexicographic sort, the log-softmax against float64,
and the candidate sampler's distribution against its closed form.
"""
import ctypes
import math
from fractions import Fraction

import numpy as np
import pytest

import _oracle as O

F = np.float32


# ---------------------------------------------------------------- test/test_sampling.br

def test_resolve_seed():  # :7-13
    L = O.lib()
    assert L.orc_resolve_seed(42, 1000, 1) == 42
    a = L.orc_resolve_seed(-1, 1000, 1)
    b = L.orc_resolve_seed(-1, 1000, 2)
    c = L.orc_resolve_seed(-1, 1001, 1)
    assert a > 0 and a != b and a != c


def test_greedy():  # :16
    assert O.sample_greedy([1.0, 5.0, 3.0, -2.0]) == 1


def test_logprob_known_answers():  # :19-26
    eq = O.token_logprob([0.0, 0.0], 0)
    assert -0.70 < eq < -0.69
    hi = O.token_logprob([0.0, 2.0], 1)
    lo = O.token_logprob([0.0, 2.0], 0)
    assert hi > lo
    m, s = O.logprob_normalizer([0.0, 2.0])
    assert F(F(2.0) - F(m)) - F(s) == F(hi)
    a = O.apply_repeat_penalty([2.0, -2.0], [0], 2.0, 64)
    assert list(a) == [1.0, -2.0]


def test_rng_determinism():  # :29-39
    ua, sa = O.rng_next_u64(O.seed_rng(42))
    ub, _ = O.rng_next_u64(O.seed_rng(42))
    assert ua == ub
    f, _ = O.rng_next_f32(sa)
    assert 0.0 <= f < 1.0
    uc, _ = O.rng_next_u64(O.seed_rng(7))
    assert ua != uc


def test_top_k_select_known():  # :42-49
    vals, idxs = O.top_k_select([1.0, 5.0, 3.0, -2.0, 9.0, 0.5], 3)
    assert len(vals) == 3
    assert list(idxs) == [4, 1, 2]
    assert list(vals) == [9.0, 5.0, 3.0]


def test_heap_rank_known():  # :52-61
    v, i = O.all_candidates_sorted([1.0, 5.0, 3.0, -2.0, 9.0, 0.5])
    assert v[0] == 9.0 and i[0] == 4 and v[1] == 5.0 and i[1] == 1 and v[5] == -2.0 and i[5] == 3
    # rank_candidates(.., top_k 0) takes the heap path (src/sampling.br:367-371)
    uv, ui = O.all_candidates_sorted([1.0, 5.0, 3.0])
    assert len(uv) == 3 and ui[0] == 1


def test_top_n_sigma_known():  # :63-71
    f = O.top_n_sigma([10.0, 8.0, 0.0], 0.2)
    assert f[0] == 10.0 and f[1] < -1e29
    assert O.top_n_sigma([10.0, 8.0, 0.0], -1.0)[2] == 0.0
    assert O.top_n_sigma([10.0, 8.0, 0.0], 0.0)[2] == 0.0
    assert O.top_n_sigma([10.0, 9.0, -1e30], 3.0)[1] == 9.0


def test_filtered_candidates():  # :75-93
    tok, st = O.sample_candidates(O.seed_rng(9), [5.0, 3.0], [7, 2], 0.0)
    assert tok == 7
    before, _ = O.rng_next_u64(O.seed_rng(9))
    after, _ = O.rng_next_u64(st)
    assert before == after
    tok, st, probs, ids = O.sample_candidates(O.seed_rng(9), [2.0, 1.0], [7, 2], 1.0, with_probs=True)
    assert tok in (7, 2)
    assert len(ids) == 2 and ids[0] == 7 and probs[0] > probs[1]
    assert abs(float(probs[0]) + float(probs[1]) - 1.0) < 1e-5
    for seed in range(1, 11):
        tok, _ = O.sample_candidates(O.seed_rng(seed), [30.0, 0.0], [4, 8], 1.0)
        assert tok == 4


def test_min_keep():  # :97-107
    st = O.seed_rng(1)
    saw = False
    for _ in range(100):
        tok, st = O.sample_candidates(st, [1.0, 1.0], [4, 8], 1.0, top_p=0.1, min_keep=2)
        saw |= tok == 8
    assert saw


def test_typical_known():  # :112-122
    tok, _ = O.sample_candidates(O.seed_rng(1), [0.916, 0.405, 0.0], [4, 8, 9], 1.0, typical_p=0.1, min_keep=1)
    assert tok == 8
    L = O.lib()
    p, lg, ids = O.f32([0.5, 0.3, 0.2]), O.f32([9.0, 4.0, 1.0]), O.i32([10, 20, 30])
    kp, kl, ki = np.zeros(3, F), np.zeros(3, F), np.zeros(3, np.int32)
    n = L.orc_typical_filter(O.fp(p), O.fp(lg), O.ip(ids), 3, 0.1, 1, O.fp(kp), O.fp(kl), O.ip(ki))
    assert n == 1 and kl[0] == 4.0 and ki[0] == 20


def test_mirostat_adaptive():  # :124-150
    L = O.lib()
    lg = O.f32([4.0, 2.0, 0.0])
    s = ctypes.c_uint64(O.seed_rng(1))
    mu = ctypes.c_float(1.0)
    assert L.orc_mirostat(2, ctypes.byref(s), O.fp(lg), 3, 1.0, 5.0, 0.1, ctypes.byref(mu)) == 0
    assert mu.value > 1.0
    s = ctypes.c_uint64(O.seed_rng(2))
    mu = ctypes.c_float(10.0)
    t = L.orc_mirostat(1, ctypes.byref(s), O.fp(lg), 3, 1.0, 5.0, 0.1, ctypes.byref(mu))
    assert 0 <= t < 3
    s0 = O.seed_rng(2)
    s = ctypes.c_uint64(s0)
    mu = ctypes.c_float(10.0)
    assert L.orc_mirostat(1, ctypes.byref(s), O.fp(lg), 3, 0.0, 5.0, 0.1, ctypes.byref(mu)) == 0
    assert s.value == s0 and mu.value == F(10.0)
    target, decay = F(0.3), F(0.9)
    w = F(target / F(F(1.0) - decay))
    tw = F(F(1.0) / F(F(1.0) - decay))
    s = ctypes.c_uint64(O.seed_rng(3))
    ws_, tw_ = ctypes.c_float(w), ctypes.c_float(tw)
    t = L.orc_adaptive_p(ctypes.byref(s), O.fp(O.f32([3.0, 1.0, 0.0])), 3, target, decay, ctypes.byref(ws_),
                         ctypes.byref(tw_))
    assert 0 <= t < 3 and ws_.value > decay * w
    assert tw_.value == F(F(1.0) + F(decay * tw))


def test_dynatemp():  # :152-161
    L = O.lib()
    u = L.orc_dynamic_temperature(O.fp(O.f32([0.5, 0.5])), 2, 0, 2, 0.8, 0.4, 1.0)
    assert 1.199 < u < 1.201
    p = L.orc_dynamic_temperature(O.fp(O.f32([0.999, 0.001])), 2, 0, 2, 0.8, 0.4, 1.0)
    assert 0.4 < p < 0.5
    assert L.orc_dynamic_temperature(O.fp(O.f32([1.0, 0.0])), 2, 0, 2, 0.5, 1.0, 1.0) == 0.0


def test_xtc_known():  # :163-167
    tok, _ = O.sample_candidates(O.seed_rng(1), [0.47, 0.336, 0.0], [4, 8, 9], 1.0, xtc_p=1.0, xtc_t=0.2, min_keep=1)
    assert tok == 9


def test_sample_greedy_keeps_rng():  # :169-175
    s0 = O.seed_rng(1)
    tok, s1 = O.sample(s0, [1.0, 5.0, 3.0, -2.0], O.params())
    assert tok == 1 and s1 == s0


def test_peaked():  # :177-185
    for seed in range(1, 11):
        tok, _ = O.sample(O.seed_rng(seed), [0.0, 0.0, 30.0, 0.0, 0.0], O.params(temperature=1.0, top_k=3))
        assert tok == 2


def test_repeat_penalty_known():  # :187-211
    assert list(O.apply_repeat_penalty([1.0, 5.0, -3.0], [1], 1.0, 64)) == [1.0, 5.0, -3.0]
    assert list(O.apply_repeat_penalty([4.0, -4.0, 9.0], [0, 1, 0], 2.0, 64)) == [2.0, -8.0, 9.0]
    assert list(O.apply_repeat_penalty([4.0, 4.0], [0, 1], 2.0, 1)) == [4.0, 2.0]
    assert list(O.apply_repeat_penalty([4.0, 4.0], [0, 1], 2.0, 0)) == [4.0, 4.0]
    assert list(O.apply_repeat_penalty([4.0, 4.0], [0, 1], 2.0, -1)) == [2.0, 2.0]


def test_dry_known():  # :213-224
    h = [0, 1, 2, 2, 1, 2, 3, 0, 1, 2]
    d = O.apply_dry([10.0] * 4, h, 2.0, 2.0, 2, 64, [])
    assert d[2] == 6.0 and d[3] == 8.0
    assert O.apply_dry([10.0] * 4, h, 2.0, 2.0, 2, 64, [[3]])[2] == 10.0
    assert O.apply_dry([10.0, 10.0], [0, 1, 0], 2.0, 2.0, 1, 64, [[1]])[1] == 10.0


def test_penalty_flips_greedy():  # :228-230
    tok, _ = O.sample(O.seed_rng(1), [10.0, 9.0], O.params(repeat_penalty=2.0), history=[0])
    assert tok == 1


def test_presence_frequency_known():  # :233-255
    assert list(O.apply_presence_frequency([1.0, 5.0, -3.0], [1, 1], 0.0, 0.0)) == [1.0, 5.0, -3.0]
    assert list(O.apply_presence_frequency([10.0, 10.0, 10.0], [0, 0, 0, 1], 0.5, 2.0)) == [6.5, 7.5, 10.0]
    assert O.apply_presence_frequency([1.0, 2.0], [0], 0.0, -1.5)[0] == 2.5
    L = O.lib()
    out = np.zeros(3, F)
    L.orc_suppress_token(O.fp(O.f32([1.0, 9.0, 3.0])), 3, 1, O.fp(out))
    assert out[0] == 1.0 and out[1] < -1e6 and out[2] == 3.0
    tok, _ = O.sample(O.seed_rng(1), O.apply_presence_frequency([10.0, 9.0], [0], 0.0, 2.0), O.params())
    assert tok == 1
    assert O.apply_presence_frequency([10.0, 9.0], [], 1.0, 1.0)[0] == 10.0


def test_logit_bias_known():  # :257-264
    assert list(O.apply_logit_bias([4.0, 2.0, 1.0], {0: -5.0, 2: 3.0})) == [-1.0, 2.0, 4.0]
    assert O.apply_logit_bias([1.0, 2.0], {})[1] == 2.0


def test_min_p_one():  # :268-272
    for seed in range(1, 11):
        tok, _ = O.sample(O.seed_rng(seed), [4.0, 3.0, 2.0], O.params(temperature=1.0, top_k=3, min_p=1.0))
        assert tok == 0


def test_eog_registry():  # :274-283
    L = O.lib()
    assert L.orc_is_eog_token(1, 1) and not L.orc_is_eog_token(106, 1)
    assert L.orc_turn_close_token(1) == 1
    ids = O.i32([1, 106])
    L.orc_set_eog_tokens(O.ip(ids), 2, 106)
    try:
        assert L.orc_is_eog_token(106, 1) and L.orc_is_eog_token(1, 1) and not L.orc_is_eog_token(5, 1)
        assert L.orc_turn_close_token(1) == 106
        out = np.zeros(4, F)
        L.orc_suppress_eog_tokens(O.fp(O.f32([0.0, 1.0, 2.0, 3.0])), 4, 1, O.fp(out))
        assert out[1] < -1000.0 and out[0] == 0.0 and out[3] == 3.0
    finally:
        L.orc_set_eog_tokens(O.ip(ids), 0, -1)


# ---------------------------------------------------------------- closed forms and brute force

MASK = (1 << 64) - 1


def xorshift(x):
    x ^= (x << 13) & MASK
    x ^= x >> 7
    x ^= (x << 17) & MASK
    return x


def u64_to_f32(x):
    """Round-to-nearest-even of an integer to binary32, exactly (Fraction arithmetic)."""
    if x == 0:
        return 0.0
    e = x.bit_length() - 1
    sh = max(e - 23, 0)
    m = Fraction(x, 1 << sh)
    q = m.numerator // m.denominator
    r = m - q
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and q & 1):
        q += 1
    return float(np.float32(q * (1 << sh)))


@pytest.mark.parametrize("seed", [0, 1, 7, 42, 1234, -5])
def test_rng_stream_closed_form(seed):
    # src/sampling.br:35-54 recomputed with Python integers
    s = 88172645463325252 if seed == 0 else (seed & MASK) ^ 88172645463325252
    assert O.seed_rng(seed) == s
    st = s
    for _ in range(64):
        x = xorshift(s)
        v, st2 = O.rng_next_u64(st)
        assert v == x and st2 == x
        f, _ = O.rng_next_f32(st)
        assert f == u64_to_f32(x) / 2.0 ** 64
        s, st = x, st2


def test_rng_f32_can_reach_one():
    # the u64 -> f32 rounding maps x >= 2^64 - 2^39 to 2^64, so the draw is exactly 1.0 (a known edge)
    assert u64_to_f32(MASK) / 2.0 ** 64 == 1.0


@pytest.mark.parametrize("trial", range(20))
def test_rankings_against_lexsort(trial):
    rng = np.random.default_rng(trial)
    n = int(rng.integers(2, 400))
    # many ties: values on a coarse grid
    x = (rng.integers(-20, 20, n) * 0.25).astype(F)
    k = int(rng.integers(1, n + 3))
    order = np.lexsort((np.arange(n), -x))  # value desc, index asc
    v, i = O.top_k_select(x, k)
    kk = min(k, n)
    assert list(i) == list(order[:kk]) and np.array_equal(v, x[order[:kk]])
    hv, hi = O.all_candidates_sorted(x)
    assert np.array_equal(hv, np.sort(x)[::-1])
    assert sorted(hi) == list(range(n)) and np.array_equal(x[hi], hv)
    assert O.sample_greedy(x) == int(order[0])


def test_top_k_excludes_sentinel():
    v, i = O.top_k_select([-1e30, -2e30, 3.0], 3)
    assert list(i) == [2, 0, 0] and v[1] == F(-1e30)


@pytest.mark.parametrize("trial", range(10))
def test_logprob_vs_float64(trial):
    rng = np.random.default_rng(100 + trial)
    x = (rng.standard_normal(5000) * 4).astype(F)
    t = int(rng.integers(0, 5000))
    ref = float(x[t]) - float(np.max(x)) - math.log(np.sum(np.exp(x.astype(np.float64) - float(np.max(x)))))
    got = O.token_logprob(x, t)
    assert abs(got - ref) <= 1e-4 * max(1.0, abs(ref))


def test_candidate_distribution():
    # frequencies of a 4-candidate draw match softmax(v / T) (T = 0.7) within 5 sigma
    vals, ids = [2.0, 1.5, 0.5, -1.0], [10, 11, 12, 13]
    T = 0.7
    w = np.exp((np.array(vals) - vals[0]) / T)
    p = w / w.sum()
    st = O.seed_rng(99)
    n = 20000
    counts = np.zeros(4)
    for _ in range(n):
        tok, st = O.sample_candidates(st, vals, ids, T)
        counts[tok - 10] += 1
    sd = np.sqrt(n * p * (1 - p))
    assert np.all(np.abs(counts - n * p) < 5 * sd)


def test_top_p_cut_and_errors():
    # top_p keeps the shortest prefix reaching the mass: with p = [.5,.3,.2] and top_p .75 the third never appears
    vals = [0.0, math.log(0.6), math.log(0.4)]
    st = O.seed_rng(5)
    seen = set()
    for _ in range(400):
        tok, st = O.sample_candidates(st, vals, [1, 2, 3], 1.0, top_p=0.75)
        seen.add(tok)
    assert seen == {1, 2}
    with pytest.raises(RuntimeError, match="empty or mismatched"):
        O.sample_candidates(O.seed_rng(1), [], [], 1.0)


def test_softcap_closed_form():
    x = (np.random.default_rng(3).standard_normal(10000) * 10).astype(F)
    out = np.zeros_like(x)
    O.lib().orc_finish_logits(O.fp(x), len(x), 1.0, 30.0, O.fp(out))
    assert np.max(np.abs(out - 30 * np.tanh(x.astype(np.float64) / 30))) < 1e-5
    O.lib().orc_finish_logits(O.fp(x), len(x), 1.0, 0.0, O.fp(out))
    assert np.array_equal(out, x)
