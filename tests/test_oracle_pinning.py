"""Pins the oracle parts that no reference vector fixes, against independent library routines, and shows
that each check fails against an oracle with a planted mistake (oracle/Makefile `mutants`).

  heap rank order among equal values (all_candidates_sorted, src/sampling.br:301-365): numpy's heapsort
      (the same bottom-up max-heap with strict-greater child choice and extraction of the root), reversed;
  the index-order normaliser (logprob_normalizer, src/sampling.br:254-266): np.cumsum over float32 terms
      (a sequential float32 sum, checked here against a plain loop) of glibc's expf, called through ctypes;
  the rank-order sums of sample_candidates_with_probs (src/sampling.br:506-598): sum_exp, the top-p running
      probability, the min-p cut, the tempered sum and the draw's running sum, the same way, with the RNG
      draw from the xorshift closed form.
  top_n_sigma_logits (src/sampling.br:376-407): the count, sum and sum of squares of the values above -1e29
      as sequential float64 sums (np.cumsum over float64), then mean, variance, the square root rounded to
      float32 and the threshold max - n * sigma in float32.
  sample_mirostat_v1's fit (src/sampling.br:683-699): the sequential float32 loop over the first 100 ranked
      probabilities with glibc's logf and powf through ctypes, and on exact Zipf probabilities the fitted
      exponent and the closed-form cutoff.
  sample_adaptive_p (src/sampling.br:705-740): the row's normaliser, the transformed values, their
      normaliser and the draw's running sum in index order, with numpy sequential sums and glibc's expf/logf.
The planted mistakes: ties sent to the right child in the sift (1), a pairwise normaliser sum (2), the
softmax sum in reverse rank order (3), the tempered sum as two halves (4), top-n-sigma's value sum in
float32 (5), the mirostat v1 fit's last pair dropped (6), adaptive-p's distance scaled by 0.25 (8); the
JSON classifier's mistake (7) is caught in test_oracle_json.py.
"""
import ctypes
from fractions import Fraction

import numpy as np
import pytest

import _oracle as O

F = np.float32
MASK = (1 << 64) - 1
_m = ctypes.CDLL("libm.so.6")
_m.expf.restype = ctypes.c_float
_m.expf.argtypes = [ctypes.c_float]
_m.logf.restype = ctypes.c_float
_m.logf.argtypes = [ctypes.c_float]
_vexpf = np.frompyfunc(_m.expf, 1, 1)


def gexpf(a):
    """glibc expf elementwise (float32 in, float32 out)."""
    return np.asarray(_vexpf(np.asarray(a, F)), dtype=F)


def seq_sum(a):
    """Sequential float32 sum, left to right."""
    return F(np.cumsum(np.asarray(a, F), dtype=F)[-1]) if len(a) else F(0.0)


def test_cumsum_is_a_sequential_float32_sum():
    x = (np.random.default_rng(1).standard_normal(4000) * 3).astype(F)
    s = F(0.0)
    run = []
    for v in x:
        s = F(s + v)
        run.append(s)
    assert np.array_equal(np.cumsum(x, dtype=F), np.array(run, F))
    assert np.sum(x) != s  # numpy's sum is pairwise, the reason it is not used here


# ---------------------------------------------------------------- heap rank order

def tied_arrays(seed, n_arrays):
    rng = np.random.default_rng(seed)
    for _ in range(n_arrays):
        n = int(rng.integers(2, 700))
        kind = int(rng.integers(0, 3))
        if kind == 0:
            yield rng.integers(0, int(rng.integers(1, 8)), n).astype(F)
        elif kind == 1:
            yield (rng.integers(-12, 12, n) * 0.25).astype(F)
        else:  # bfloat16-rounded normals
            x = (rng.standard_normal(n) * 3).astype(F)
            yield (x.view(np.uint32) & 0xFFFF0000).view(F)


def heap_mismatches(L, arrays):
    bad = 0
    for x in arrays:
        v = np.zeros(len(x), F)
        i = np.zeros(len(x), np.int32)
        L.orc_all_candidates_sorted(O.fp(x), len(x), O.fp(v), O.ip(i))
        bad += not np.array_equal(i, np.argsort(x, kind="heapsort")[::-1])
    return bad


def test_heap_tie_order_equals_numpy_heapsort():
    assert heap_mismatches(O.lib(), tied_arrays(7, 1200)) == 0


def test_heap_tie_order_full_vocabulary():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(151936) * 3).astype(F)
    x = (x.view(np.uint32) & 0xFFFF0000).view(F)  # bfloat16: thousands of equal values
    assert heap_mismatches(O.lib(), [x]) == 0


def test_heap_check_fails_on_planted_mistake():
    assert heap_mismatches(O.mutant(1), tied_arrays(7, 200)) > 0


# ---------------------------------------------------------------- index-order normaliser

def normaliser_rows():
    rng = np.random.default_rng(21)
    rows = [(rng.standard_normal(151936) * s).astype(F) for s in (3.0, 4.0)]
    rows.append((rng.standard_normal(262144) * 10).astype(F))
    for _ in range(30):
        n = int(rng.integers(1, 6000))
        rows.append((rng.standard_normal(n) * float(rng.uniform(0.1, 12))).astype(F))
    rows.append((np.arange(5000) % 7).astype(F))  # ties and exact crossings
    return rows


def normaliser_mismatches(L, rows):
    bad = 0
    for x in rows:
        mx = x.max()
        want = seq_sum(gexpf(x - mx))
        bad += L.orc_logprob_sum(O.fp(x), len(x)) != want
        m, lse = ctypes.c_float(), ctypes.c_float()
        L.orc_logprob_normalizer(O.fp(x), len(x), ctypes.byref(m), ctypes.byref(lse))
        bad += m.value != mx or lse.value != _m.logf(float(want))
    return bad


def test_normaliser_is_the_sequential_glibc_sum():
    assert normaliser_mismatches(O.lib(), normaliser_rows()) == 0


def test_normaliser_check_fails_on_planted_mistake():
    assert normaliser_mismatches(O.mutant(2), normaliser_rows()) > 0


# ---------------------------------------------------------------- rank-order sums of the draw

def xorshift(x):
    x ^= (x << 13) & MASK
    x ^= x >> 7
    x ^= (x << 17) & MASK
    return x


def u64_to_f32(x):
    if x == 0:
        return 0.0
    e = x.bit_length() - 1
    sh = max(e - 23, 0)
    m = Fraction(x, 1 << sh)
    q = m.numerator // m.denominator
    r = m - q
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and q & 1):
        q += 1
    return float(F(q * (1 << sh)))


def draw_trace(state, v, T, top_p, min_p, min_keep):
    """sample_candidates_with_probs' float32 sums for a ranked list v (no typical, XTC or dynatemp),
    restated with numpy sequential sums and glibc expf."""
    n = len(v)
    keep = min(max(min_keep, 1), n)
    e = gexpf(v - v[0])
    sum_exp = seq_sum(e)
    p = (e / sum_exp).astype(F)
    cutoff = n
    if top_p < 1.0:
        cum = np.cumsum(p, dtype=F)
        hit = np.nonzero((cum >= F(top_p)) & (np.arange(1, n + 1) >= keep))[0]
        if len(hit):
            cutoff = int(hit[0]) + 1
    if min_p > 0.0:
        thr = F(p[0] * F(min_p))
        mc = keep
        while mc < cutoff and p[mc] >= thr:
            mc += 1
        cutoff = mc
    r = gexpf(((v[:cutoff] - v[0]).astype(F) / F(T)).astype(F))
    renorm = seq_sum(r)
    r01 = F(u64_to_f32(xorshift(state)) / 2.0 ** 64)
    target = F(r01 * renorm)
    run = np.cumsum(r, dtype=F)
    hit = np.nonzero(run >= target)[0]
    chosen = int(hit[0]) if len(hit) else cutoff - 1
    return [sum_exp, F(T), renorm, target], [cutoff, 0, chosen]


def ranked_cases():
    rng = np.random.default_rng(31)
    cases = []
    for s, T, tp, mp in ((4.0, 0.7, 0.9, 0.0), (3.0, 1.0, 1.0, 0.0), (4.0, 0.8, 0.95, 0.05)):
        x = (rng.standard_normal(151936) * s).astype(F)
        cases.append((np.sort(x)[::-1].copy(), T, tp, mp, 1, int(rng.integers(1, 1 << 62))))
    for _ in range(150):
        n = int(rng.integers(1, 600))
        x = np.sort((rng.standard_normal(n) * float(rng.uniform(0.2, 6))).astype(F))[::-1].copy()
        cases.append((x, float(rng.choice([0.3, 0.7, 1.0, 1.5])), float(rng.choice([1.0, 0.9, 0.5])),
                      float(rng.choice([0.0, 0.05, 0.2])), int(rng.integers(0, 4)), int(rng.integers(1, 1 << 62))))
    return cases


def trace_mismatches(L, cases):
    bad = 0
    for v, T, tp, mp, mk, st in cases:
        ids = np.arange(len(v), dtype=np.int32)
        of = np.zeros(4, F)
        oi = (ctypes.c_int64 * 3)()
        tok = L.orc_sample_candidates_trace(st, O.fp(v), O.ip(ids), len(v), T, tp, mp, mk, O.fp(of), oi)
        wf, wi = draw_trace(st, v, T, tp, mp, mk)
        bad += (not np.array_equal(of, np.array(wf, F))) or list(oi) != wi or tok != wi[2]
    return bad


def test_rank_order_sums_are_sequential_glibc_sums():
    assert trace_mismatches(O.lib(), ranked_cases()) == 0


@pytest.mark.parametrize("k", [3, 4])
def test_rank_order_check_fails_on_planted_mistake(k):
    assert trace_mismatches(O.mutant(k), ranked_cases()) > 0


# ---------------------------------------------------------------- top-n-sigma statistics

def tns_rows():
    rng = np.random.default_rng(41)
    rows = []
    for k in range(60):
        n = int(rng.integers(2, 3000)) if k % 3 else 151936
        x = (rng.standard_normal(n) * float(rng.uniform(0.5, 8.0)) + float(rng.uniform(-3, 3))).astype(F)
        x[rng.integers(0, n, max(1, n // 500))] = F(-1e30)  # excluded from the statistics
        rows.append((x, float(rng.choice([0.5, 1.0, 1.7, 3.0]))))
    return rows


def tns_threshold(x, n):
    """max - n * sigma, or None when the row is kept whole"""
    v = x[x > F(-1e29)].astype(np.float64)
    cnt = len(v)
    if n <= 0.0 or cnt <= 1:
        return None
    s = np.cumsum(v)[-1]
    q = np.cumsum(v * v)[-1]
    mean = s / cnt
    var = q / cnt - mean * mean
    if var <= 0.0:
        return None
    sigma = F(np.sqrt(var))
    return F(x[x > F(-1e29)].max() - F(F(n) * sigma))


def tns_mismatches(L, rows):
    bad = 0
    for x, n in rows:
        want = tns_threshold(x, n)
        thr = ctypes.c_float()
        kept = L.orc_top_n_sigma_threshold(O.fp(x), len(x), n, ctypes.byref(thr))
        bad += (want is None) != (kept == 0) or (want is not None and thr.value != want)
        o = np.zeros_like(x)
        L.orc_top_n_sigma(O.fp(x), len(x), n, O.fp(o))
        bad += not np.array_equal(o, x if want is None else np.where(x >= want, x, F(-1e30)).astype(F))
    return bad


def test_top_n_sigma_is_the_sequential_float64_statistics():
    assert tns_mismatches(O.lib(), tns_rows()) == 0


def test_top_n_sigma_check_fails_on_planted_mistake():
    assert tns_mismatches(O.mutant(5), tns_rows()) > 0


# ---------------------------------------------------------------- mirostat v1's Zipf fit

_m.powf.restype = ctypes.c_float
_m.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def miro_v1_cutoff(x, T, mu):
    """(cutoff, s_hat) of sample_mirostat_v1 (src/sampling.br:676-699) from numpy's sort and glibc's expf,
    logf and powf: the ranked values divided by T, their softmax with a sequential float32 sum, the fit
    over the first min(V, 100), the estimate cast as Rust `as int` does (saturating, NaN to 0), clamped."""
    V = len(x)
    v = (np.sort(np.asarray(x, F))[::-1] / F(T)).astype(F)
    terms = gexpf(v - v[0])
    probs = (terms / seq_sum(terms)).astype(F)
    sa, sb = F(0.0), F(0.0)
    with np.errstate(all="ignore"):
        for i in range(min(V, 100) - 1):
            t_i = F(_m.logf(F(F(i + 2) / F(i + 1))))
            b_i = F(_m.logf(F(probs[i] / probs[i + 1])))
            sa = F(sa + F(t_i * b_i))
            sb = F(sb + F(t_i * t_i))
        s_hat = F(sa / sb)
        eps = F(s_hat - F(1.0))
        num = F(eps * F(_m.powf(2.0, mu)))
        den = F(F(1.0) - F(_m.powf(F(V), -eps)))
        est = F(_m.powf(F(num / den), F(F(1.0) / s_hat)))
    if est != est:
        e = 0
    elif est >= F(2.0 ** 63):
        e = 2 ** 63 - 1
    elif est <= F(-2.0 ** 63):
        e = -2 ** 63
    else:
        e = int(est)
    return min(max(e, 1), V), s_hat


def miro_rows():
    rng = np.random.default_rng(53)
    rows = []
    for k in range(40):
        V = int(rng.choice([3, 50, 101, 1000, 5003, 40000]))
        if k % 4 == 0:  # Zipf: p_i proportional to (i + 1)^-s, shuffled
            s = float(rng.uniform(1.05, 2.5))
            x = (-s * np.log(np.arange(1, V + 1))).astype(F)
            rng.shuffle(x)
            T = 1.0
        elif k % 4 == 1:  # wide spread: tail probabilities underflow to zero (NaN fit, cutoff 1)
            x = (rng.standard_normal(V) * 60.0).astype(F)
            T = float(rng.choice([0.5, 1.0]))
        else:
            x = (rng.standard_normal(V) * float(rng.uniform(0.5, 4.0))).astype(F)
            x[rng.integers(0, V, max(1, V // 50))] = x[int(rng.integers(0, V))]  # equal values
            T = float(rng.choice([0.5, 0.9, 1.0, 1.7]))
        rows.append((x, T, float(rng.choice([3.0, 6.0, 10.0, 16.0]))))
    return rows


def miro_mismatches(L, rows):
    L.orc_mirostat_v1_cutoff.restype = ctypes.c_int64
    L.orc_mirostat_v1_cutoff.argtypes = [O.f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_float,
                                         ctypes.POINTER(ctypes.c_float)]
    bad = 0
    for x, T, mu in rows:
        want, ws = miro_v1_cutoff(x, T, mu)
        s = ctypes.c_float()
        got = L.orc_mirostat_v1_cutoff(O.fp(x), len(x), T, mu, ctypes.byref(s))
        bad += got != want or not (np.float32(s.value).view(np.uint32) == ws.view(np.uint32) or (ws != ws and s.value != s.value))
    return bad


def test_mirostat_v1_fit_is_the_sequential_float32_loop():
    assert miro_mismatches(O.lib(), miro_rows()) == 0


def test_mirostat_v1_fit_recovers_a_zipf_exponent():
    """On exact Zipf probabilities the fit returns the exponent s and the cutoff follows the closed form
    ((s - 1) 2^mu / (1 - V^(1 - s)))^(1/s) (float64, here)."""
    L = O.lib()
    L.orc_mirostat_v1_cutoff.restype = ctypes.c_int64
    L.orc_mirostat_v1_cutoff.argtypes = [O.f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_float,
                                         ctypes.POINTER(ctypes.c_float)]
    rng = np.random.default_rng(5)
    for s, V, mu in ((1.1, 5003, 10.0), (1.5, 40000, 6.0), (2.0, 1000, 10.0), (1.3, 151936, 8.0)):
        x = (-s * np.log(np.arange(1, V + 1))).astype(F)
        rng.shuffle(x)
        sh = ctypes.c_float()
        got = L.orc_mirostat_v1_cutoff(O.fp(x), V, 1.0, mu, ctypes.byref(sh))
        assert abs(sh.value - s) < 2e-3 * s, (s, sh.value)
        est = ((s - 1) * 2.0 ** mu / (1 - V ** (1 - s))) ** (1 / s)
        want = min(max(int(est), 1), V)
        assert abs(got - want) <= max(2, 0.02 * want), (s, V, mu, got, want)


def test_mirostat_v1_check_fails_on_planted_mistake():
    assert miro_mismatches(O.mutant(6), miro_rows()) > 0


# ---------------------------------------------------------------- adaptive-p

def adaptive_trace(state, x, target, decay, ws, tw):
    """sample_adaptive_p (src/sampling.br:705-740) from numpy's sequential float32 sums and glibc's expf/logf:
    the normaliser of the row, the transformed values, their normaliser, the draw's running sum in index
    order (the RNG's first draw from its closed form); returns (token, state, weighted sum, total weight)."""
    x = np.asarray(x, F)
    M = x.max()
    lse = F(_m.logf(seq_sum(gexpf(x - M))))
    p = gexpf((x - M) - lse)
    avg = target if tw == F(0.0) else F(ws / tw)
    at = F(F(2.0) * target - avg)
    at = min(max(at, F(0.0)), F(1.0))
    dist = (np.abs(p - at) / F(0.3)).astype(F)
    num = ((F(10.0) * dist).astype(F) * dist).astype(F)
    t = np.where(x <= F(-1e29), x, (F(5.0) - (num / (F(1.0) + dist)).astype(F)).astype(F)).astype(F)
    tmax = t.max()
    tsum = F(_m.logf(seq_sum(gexpf(t - tmax))))
    s1 = xorshift(state)
    draw = F(F(u64_to_f32(s1)) / F(2.0 ** 64))
    run = np.cumsum(gexpf((t - tmax) - tsum), dtype=F)
    hit = np.nonzero(run >= draw)[0]
    sel = int(hit[0]) if len(hit) else len(x) - 1
    return sel, s1, F(p[sel] + F(decay * ws)), F(F(1.0) + F(decay * tw))


def adaptive_rows():
    rng = np.random.default_rng(29)
    rows = []
    for k in range(24):
        V = int(rng.choice([3, 40, 777, 3000]))
        x = (rng.standard_normal(V) * float(rng.uniform(0.5, 5.0))).astype(F)
        if k % 5 == 0:
            x[rng.integers(0, V, max(1, V // 30))] = F(-1e30)  # excluded from the transform
        target, decay = F(rng.choice([0.05, 0.3, 0.6, 0.95])), F(rng.choice([0.0, 0.5, 0.9, 0.99]))
        ws, tw = (F(0.0), F(0.0)) if k % 7 == 0 else (F(target / F(F(1.0) - decay)), F(F(1.0) / F(F(1.0) - decay)))
        rows.append((int(rng.integers(1, 2 ** 63)), x, target, decay, ws, tw))
    return rows


def adaptive_mismatches(L):
    bad = 0
    for state, x, target, decay, ws, tw in adaptive_rows():
        want = adaptive_trace(state, x, target, decay, ws, tw)
        s = ctypes.c_uint64(state)
        w, tt = ctypes.c_float(ws), ctypes.c_float(tw)
        tok = L.orc_adaptive_p(ctypes.byref(s), O.fp(x), len(x), float(target), float(decay), ctypes.byref(w),
                               ctypes.byref(tt))
        bad += (tok, s.value) != want[:2] or F(w.value) != want[2] or F(tt.value) != want[3]
    return bad


def test_adaptive_p_is_the_sequential_loop():
    assert adaptive_mismatches(O.lib()) == 0


def test_adaptive_p_check_fails_on_planted_mistake():
    assert adaptive_mismatches(O.mutant(8)) > 0
