"""Parity of the library's kernels, run on the CPU SIMT emulator, against the oracle (test infrastructure).

The emulator build (tests/cpu/simt/Makefile) compiles the same kernel and C-ABI sources as the HIP
library, with every GPU thread a fiber; device pointers are host pointers. This script loads a private
copy of the Python binding pointed at that build (the product module and its library path are left
alone) and checks the workloads the GPU parity tests check, at reduced step counts:

    python run_parity.py --lib _build/libbl_simt.so small:0-10:25 w2:2 w4:1:8 w5:1 async:2

Items: small:<cases>:<steps>, w2:<steps>, w3:<steps>, w4:<steps>:<rows>, w5:<steps>, async:<steps>,
grammar:<cases>:<steps>, bigk:<steps>, pair:<case>:<case>:<steps>.
Prints one line per item ("ok ..." / "FAIL ...") and exits 1 if any failed.
"""
import argparse
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(HERE, "..", "..", ".."))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import _oracle as O  # noqa: E402
from _cases import CASES, EOGS, EOS, SMALL_V, small_case_inputs, small_case_logits  # noqa: E402



class HostMem:
    """Device buffers of the emulator: host memory (numpy)."""

    class Buf:
        def __init__(self, n, dtype):
            self.a = np.zeros(n, dtype)
            self.ptr = self.a.ctypes.data

        def upload(self, x):
            self.a[:] = x

        def host(self):
            return self.a.copy()

    def zeros(self, n, dtype):
        return self.Buf(n, dtype)


# where the harness allocates "device" buffers; the GPU tests replace it with torch device memory
MEM = HostMem()


def load_binding(lib_path):
    spec = importlib.util.spec_from_file_location("bl_select_simt", os.path.join(ROOT, "boring-llm_amd", "bl_select.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    m.LIB_PATH = os.path.abspath(lib_path)
    m._lib = None
    return m


def lp_close(a, b):
    """logprobs and probabilities are bit-identical (NaN equal to NaN)"""
    a, b = np.float32(a), np.float32(b)
    return (a != a and b != b) or a.view(np.uint32) == b.view(np.uint32)


def quantize(x, mode):
    """Logits with ties: `bf16` rounds to bfloat16 (nearest even), as the output of a bf16 LM head
    converted to float32; `q4` rounds to multiples of 0.25."""
    if mode == "bf16":
        u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
        u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
        return u.astype(np.uint32).view(np.float32)
    return (np.round(x * np.float32(4.0)) / np.float32(4.0)).astype(np.float32)


def run_small(BL, case, steps, coarse=False, ramp=False, quant=None):
    """A small case against the oracle; `coarse` floors the logits to a few integers, so that thousands of
    values tie at the chunk top-K bound (the radix fallback with an index-order cut of the ties); `ramp`
    adds a slope of ln 2 per 63 tokens, so that the index-order sum crosses a power of two in nearly every
    64-term group (more critical groups than the normaliser precomputes)."""
    kw = CASES[case]
    rng, hist, reply, bias = small_case_inputs(case)
    ctx = BL.Context(SMALL_V, 2, 2)
    ctx.set_eog(EOS, EOGS)
    ctx.slot_reset(1, BL.Params(**kw), BL.seed_rng(100 + case), history=hist, reply=reply, bias=bias)
    op = O.params(**kw)
    L = O.lib()
    L.orc_set_eog_tokens(O.ip(O.i32([EOS] + EOGS)), 1 + len(EOGS), -1)
    hh, rr = O.i32(hist), O.i32(reply)
    bi, bv = O.i32(list(bias.keys())), O.f32(list(bias.values()))
    h = L.orc_slot_new(O.C.byref(op), BL.seed_rng(100 + case), O.ip(hh), len(hist), O.ip(rr), len(reply),
                       O.ip(bi), O.fp(bv), len(bias))
    wants = 1 if kw.get("logprobs") else 0
    n_probs = kw.get("n_probs", 0)
    buf = MEM.zeros(SMALL_V, np.float32)
    try:
        for t in range(steps):
            x = small_case_logits(rng)
            if coarse:
                x = np.floor(x / np.float32(5.0)).astype(np.float32)
            if ramp:
                x = (x * np.float32(0.05) + np.arange(SMALL_V, dtype=np.float32) * np.float32(0.011)).astype(np.float32)
            if quant:
                x = quantize(x, quant)
            buf.upload(x)
            tok, lp, ti, tl = ctx.sample_step([1], buf.ptr, SMALL_V, top_stride=max(n_probs, 1))
            ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
            oti, otl = np.full(max(n_probs, 1), -1, np.int32), np.zeros(max(n_probs, 1), np.float32)
            eog = O.C.c_int()
            assert L.orc_slot_step(h, O.fp(x), SMALL_V, wants, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl),
                                   O.C.byref(eog)) == 0
            if tok[0] != ot[0]:
                return f"step {t}: token {tok[0]} vs {ot[0]}"
            if wants and not eog.value:
                if not lp_close(lp[0], olp[0]):
                    return f"step {t}: logprob {lp[0]} vs {olp[0]}"
                if ti[0][:n_probs] != list(oti[:n_probs]) or not all(lp_close(tl[0][q], otl[q]) for q in range(n_probs)):
                    return f"step {t}: alternatives differ"
        if ctx.slot_rng(1) != L.orc_slot_rng(h):
            return "final RNG state differs"
    finally:
        L.orc_slot_free(h)
        L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
        ctx.close()
    return None


DRY_CASES = [
    # (params, breakers over the alphabet's indices: 0-19 form the phrases, 20-23 are sparse inserts)
    (dict(temperature=0.0, dry_multiplier=0.8, dry_base=1.75, dry_allowed_length=2, dry_penalty_last_n=64,
          logprobs=1, n_probs=5), [[20], [21, 22], [4]]),
    (dict(temperature=0.9, top_k=0, min_p=0.05, dry_multiplier=1.5, dry_base=2.0, dry_allowed_length=1,
          dry_penalty_last_n=200, repeat_penalty=1.2, repeat_last_n=32, frequency_penalty=0.3), []),
    (dict(temperature=0.7, top_k=40, dry_multiplier=0.5, dry_base=1.1, dry_allowed_length=3,
          dry_penalty_last_n=2048, ignore_eos=1, logprobs=1, n_probs=3), [[21], [22, 23], [20], [23, 20, 21]]),
    (dict(temperature=1.0, top_k=10, dry_multiplier=3.0, dry_base=1.0000005, dry_allowed_length=0,
          dry_penalty_last_n=16), [[0]]),
    (dict(temperature=0.0, dry_multiplier=1e-30, dry_base=10.0, dry_allowed_length=0, dry_penalty_last_n=300,
          logprobs=1, n_probs=2), [[20, 21]]),
    # a two-token breaker inside a long repeat: the suffix starts after it
    (dict(temperature=0.0, dry_multiplier=1e-3, dry_base=1.05, dry_allowed_length=2, dry_penalty_last_n=300,
          logprobs=1, n_probs=8), [[20, 21]]),
    (dict(temperature=0.0, dry_multiplier=1e-3, dry_base=1.05, dry_allowed_length=2, dry_penalty_last_n=300,
          logprobs=1, n_probs=8), [[20], [20, 21]]),
    # phrases holding the pair 20, 21: listing the pair before or after the single 20 moves the start by one
    # token (cases 7 and 8)
    (dict(temperature=0.0, dry_multiplier=0.05, dry_base=1.5, dry_allowed_length=0, dry_penalty_last_n=300,
          logprobs=1, n_probs=8), [[20, 21], [20]]),
    (dict(temperature=0.0, dry_multiplier=0.05, dry_base=1.5, dry_allowed_length=0, dry_penalty_last_n=300,
          logprobs=1, n_probs=8), [[20], [20, 21]]),
]


def dry_inputs(case):
    """A history of 400 tokens of repeated phrases over alphabet tokens 0-19 (so that suffixes recur), with
    sparse inserts of tokens 20-23 (the breakers' material); the logits favour the phrase tokens, so that the
    reply keeps repeating. Returns (rng, alphabet, history, reply)."""
    rng = np.random.default_rng(900 + case)
    alpha = [int(x) for x in rng.choice(np.arange(20, SMALL_V), 24, replace=False)]
    phrases = [[alpha[int(i)] for i in rng.integers(0, 20, int(rng.integers(3, 9)))] for _ in range(6)]
    hist = []
    while len(hist) < 400:
        hist += phrases[int(rng.integers(0, 6))]
        if rng.random() < 0.12:
            hist += [alpha[20 + int(rng.integers(0, 4))] for _ in range(int(rng.integers(1, 3)))]
    if case == 4:  # a long exact repeat: maximum repeats past the exponent cap (38 for base 10)
        hist = (phrases[0] * 80)[:300]
    if case in (5, 6):  # a phrase repeated, the breaker pair 20, 21 three phrases from the end
        ph = alpha[:7]
        hist = ph * 37 + [alpha[20], alpha[21]] + ph * 3
    if case in (7, 8):
        hist = [alpha[0], alpha[20], alpha[21], alpha[1], alpha[2], alpha[3]] * 50
    return rng, alpha, hist[:400], hist[-30:]


def run_dry(BL, case, steps):
    """DRY rows (src/sampling.br:114-171) against the oracle's decode step: the penalty map recomputed on the
    device after every commit (and after an explicit bl_slot_commit at step steps // 2), breakers in list
    order (single and multi-token), the exponent cap, logprobs of the penalised logits."""
    kw, br_idx = DRY_CASES[case]
    rng, alpha, hist, reply = dry_inputs(case)
    breakers = [[alpha[i] for i in b] for b in br_idx]
    ctx = BL.Context(SMALL_V, 2, 2)
    ctx.set_eog(EOS, EOGS)
    ctx.slot_reset(1, BL.Params(**kw), BL.seed_rng(950 + case), history=hist, reply=reply)
    ctx.slot_dry_breakers(1, breakers)
    op = O.params(**kw)
    L = O.lib()
    L.orc_set_eog_tokens(O.ip(O.i32([EOS] + EOGS)), 1 + len(EOGS), -1)
    hh, rr = O.i32(hist), O.i32(reply)
    h = L.orc_slot_new(O.C.byref(op), BL.seed_rng(950 + case), O.ip(hh), len(hist), O.ip(rr), len(reply),
                       O.ip(O.i32([0])), O.fp(O.f32([0.0])), 0)
    flat = O.i32([t for b in breakers for t in b] or [0])
    L.orc_slot_set_breakers(h, O.ip(flat), O.ip(O.i32([len(b) for b in breakers] or [0])), len(breakers))
    wants = 1 if kw.get("logprobs") else 0
    n_probs = kw.get("n_probs", 0)
    buf = MEM.zeros(SMALL_V, np.float32)
    try:
        for t in range(steps):
            if t == steps // 2:
                extra = alpha[t % 24]
                ctx.commit(1, [extra])
                L.orc_slot_push(h, extra, EOS)
            x = (rng.standard_normal(SMALL_V) * 2.0).astype(np.float32)
            x[alpha[:20]] += np.float32(7.0)
            buf.upload(x)
            tok, lp, ti, tl = ctx.sample_step([1], buf.ptr, SMALL_V, top_stride=max(n_probs, 1))
            ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
            oti, otl = np.full(max(n_probs, 1), -1, np.int32), np.zeros(max(n_probs, 1), np.float32)
            eog = O.C.c_int()
            assert L.orc_slot_step(h, O.fp(x), SMALL_V, wants, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl),
                                   O.C.byref(eog)) == 0
            if tok[0] != ot[0]:
                return f"step {t}: token {tok[0]} vs {ot[0]}"
            if wants and not eog.value:
                if not lp_close(lp[0], olp[0]):
                    return f"step {t}: logprob {lp[0]} vs {olp[0]}"
                if ti[0][:n_probs] != list(oti[:n_probs]) or not all(lp_close(tl[0][q], otl[q]) for q in range(n_probs)):
                    return f"step {t}: alternatives differ"
        if ctx.slot_rng(1) != L.orc_slot_rng(h):
            return "final RNG state differs"
    finally:
        L.orc_slot_free(h)
        L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
        ctx.close()
    return None


def run_bigties(BL, steps):
    """Two full-vocabulary rows (T 1.0 with min-p 0.05; T 0.7 with top-p 0.95 and min-p 0.02) at V=151936 on
    N(0, 3^2) logits rounded to bfloat16 (several tokens share each bfloat16 value within 4 of the maximum,
    where min-p keeps the draws), so that draws land on runs of equal values: the heap simulation against
    the oracle's heap sort."""
    V = 151936
    rng = np.random.default_rng(11)
    kws = [dict(temperature=1.0, min_p=0.05), dict(temperature=0.7, top_p=0.95, min_p=0.02)]
    ctx = BL.Context(V, 2, 2)
    L = O.lib()
    hs = []
    for r, kw in enumerate(kws):
        ctx.slot_reset(r, BL.Params(**kw), BL.seed_rng(700 + r))
        op = O.params(**kw)
        hs.append(L.orc_slot_new(O.C.byref(op), BL.seed_rng(700 + r), None, 0, None, 0, None, None, 0))
    buf = MEM.zeros(2 * V, np.float32)
    try:
        for t in range(steps):
            x = quantize((rng.standard_normal(2 * V) * 3.0).astype(np.float32), "bf16")
            buf.upload(x)
            tok = ctx.sample_step([0, 1], buf.ptr, V)[0]
            for r in range(2):
                ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
                oti, otl = np.zeros(1, np.int32), np.zeros(1, np.float32)
                eog = O.C.c_int()
                row = np.ascontiguousarray(x[r * V:(r + 1) * V])
                assert L.orc_slot_step(hs[r], O.fp(row), V, 0, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl),
                                       O.C.byref(eog)) == 0
                if tok[r] != ot[0]:
                    return f"step {t} row {r}: token {tok[r]} vs {ot[0]}"
    finally:
        for h in hs:
            L.orc_slot_free(h)
        ctx.close()
    return None


UNFILT_ROWS = [(0.7, 3.0, None), (0.3, 3.0, None), (1.5, 2.0, None), (0.7, 3.0, "bf16"), (1.0, 0.5, None),
               (0.05, 3.0, None)]


def distinct(x):
    """x with equal values moved apart by ulps (float32 rows whose draws reach far down the ranking, past
    the device's heap simulation of equal values)"""
    x = x.copy()
    for _ in range(16):
        u, inv, cnt = np.unique(x, return_inverse=True, return_counts=True)
        if len(u) == len(x):
            return x
        for v in np.nonzero(cnt > 1)[0]:
            idx = np.nonzero(inv == v)[0]
            for j, i in enumerate(idx[1:]):
                for _ in range(j + 1):
                    x[i] = np.nextafter(x[i], np.float32(np.inf))
    raise AssertionError("could not make the values distinct")


def run_unfiltered(BL, steps, rows=None):
    """Full-vocabulary rows without top-p or min-p at V=151936 (temperature, N(0, sigma^2) logits, rounding):
    the draw sees only the tempered sum, and the selection drops the candidates whose terms fall below half
    an ulp of every running sum that can precede them (bounded from the exponent blocks' sums). Large and
    small sums, a bfloat16 row (draws on equal values near the top) and a near-greedy temperature; the
    float32 rows hold distinct values."""
    V = 151936
    spec = [UNFILT_ROWS[i] for i in (rows if rows is not None else range(len(UNFILT_ROWS)))]
    R = len(spec)
    rng = np.random.default_rng(23)
    ctx = BL.Context(V, R, R)
    L = O.lib()
    hs = []
    for r, (T, _, _) in enumerate(spec):
        ctx.slot_reset(r, BL.Params(temperature=T), BL.seed_rng(900 + r))
        op = O.params(temperature=T)
        hs.append(L.orc_slot_new(O.C.byref(op), BL.seed_rng(900 + r), None, 0, None, 0, None, None, 0))
    buf = MEM.zeros(R * V, np.float32)
    try:
        for t in range(steps):
            x = np.concatenate([quantize((rng.standard_normal(V) * sg).astype(np.float32), q) if q else
                                distinct((rng.standard_normal(V) * sg).astype(np.float32)) for (_, sg, q) in spec])
            buf.upload(x)
            tok = ctx.sample_step(list(range(R)), buf.ptr, V)[0]
            for r in range(R):
                ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
                oti, otl = np.zeros(1, np.int32), np.zeros(1, np.float32)
                eog = O.C.c_int()
                row = np.ascontiguousarray(x[r * V:(r + 1) * V])
                assert L.orc_slot_step(hs[r], O.fp(row), V, 0, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl),
                                       O.C.byref(eog)) == 0
                if tok[r] != ot[0]:
                    return f"step {t} row {r} {spec[r]}: token {tok[r]} vs {ot[0]}"
    finally:
        for h in hs:
            L.orc_slot_free(h)
        ctx.close()
    return None


def halfway_rows(copies=(3, 20), V=151936):
    """Plain full-vocabulary rows (T 1) whose ranked list has a long tail holding `copies` tokens of one value
    whose term expf(v - 0) lies exactly halfway between two multiples of u = 2^(K-23), K the binade of the
    row's float32 sum: the maximum 0 at token 0, 6000 values evenly spread over [-9, -0.5], the copies near
    -6, every other token at -100. Each such term's rounding follows the parity of the running sum before it;
    past eight of them the device ranks the whole list. Returns the rows (float32, len(copies) x V)."""
    import ctypes
    expf = ctypes.CDLL("libm.so.6").expf
    expf.restype, expf.argtypes = ctypes.c_float, [ctypes.c_float]
    bulk = np.linspace(-9.0, -0.5, 6000, dtype=np.float32)
    pos = np.random.default_rng(41).permutation(np.arange(1, V))
    out = []
    for n in copies:
        def fsum(vh):
            vals = np.sort(np.concatenate([[np.float32(0.0)], bulk, np.full(n, vh, np.float32)]))[::-1]
            s = np.float32(0.0)
            for v in vals:
                s = np.float32(s + np.float32(expf(float(v))))
            return s
        S = fsum(np.float32(-6.0))
        K = int(np.floor(np.log2(float(S))))
        u = 2.0 ** (K - 23)
        vh = np.float32(-6.0)
        while True:
            y = float(np.float32(expf(float(vh)))) / u
            if y - np.floor(y) == 0.5:
                break
            vh = np.nextafter(vh, np.float32(-np.inf))
        S2 = fsum(vh)
        assert int(np.floor(np.log2(float(S2)))) == K and 1.05 < float(S2) / 2.0 ** K < 1.95, (S2, K)
        x = np.full(V, -100.0, np.float32)
        x[0] = 0.0
        x[pos[:6000]] = bulk
        x[pos[6000:6000 + n]] = vh
        out.append(x)
    return np.stack(out)


def run_halfway(BL, steps):
    """halfway_rows' draws against the oracle's slot step, `steps` steps (the RNG moves the target)."""
    X = halfway_rows()
    R, V = X.shape
    ctx = BL.Context(V, R, R)
    L = O.lib()
    hs = []
    for r in range(R):
        ctx.slot_reset(r, BL.Params(temperature=1.0), BL.seed_rng(950 + r))
        op = O.params(temperature=1.0)
        hs.append(L.orc_slot_new(O.C.byref(op), BL.seed_rng(950 + r), None, 0, None, 0, None, None, 0))
    buf = MEM.zeros(R * V, np.float32)
    try:
        buf.upload(X.reshape(-1))
        for t in range(steps):
            tok = ctx.sample_step(list(range(R)), buf.ptr, V)[0]
            for r in range(R):
                ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
                oti, otl = np.zeros(1, np.int32), np.zeros(1, np.float32)
                eog = O.C.c_int()
                assert L.orc_slot_step(hs[r], O.fp(np.ascontiguousarray(X[r])), V, 0, 1, O.ip(ot), O.fp(olp),
                                       O.ip(oti), O.fp(otl), O.C.byref(eog)) == 0
                if tok[r] != ot[0]:
                    return f"step {t} row {r}: token {tok[r]} vs {ot[0]}"
    finally:
        for h in hs:
            L.orc_slot_free(h)
        ctx.close()
    return None


TYPICAL_ROWS = [(dict(temperature=0.8, typical_p=0.9), 3.0),
                (dict(temperature=1.0, typical_p=0.5, min_keep=3), 2.0),
                (dict(temperature=0.7, typical_p=0.95, top_p=0.9, min_p=0.02), 3.0),
                (dict(temperature=1.2, typical_p=0.8, dynatemp_range=0.5), 1.5),
                (dict(temperature=0.9, typical_p=0.3), 4.0)]


def run_typical(BL, steps, V):
    """typical_p over full-vocabulary lists (every token a candidate) at vocabulary V: entropy, the selection
    order by distance |-ln p - H| (the two monotone runs of the ranked list merged), the walk to typical_p and
    min_keep, then top-p / min-p / dynamic temperature and the draw over the kept entries, against the oracle's
    slot step (whose selection loop is quadratic: V stays small). Distinct float32 values (no heap ties)."""
    R = len(TYPICAL_ROWS)
    rng = np.random.default_rng(61 + V)
    ctx = BL.Context(V, R, R)
    L = O.lib()
    hs = []
    for r, (kw, _) in enumerate(TYPICAL_ROWS):
        ctx.slot_reset(r, BL.Params(**kw), BL.seed_rng(990 + r))
        op = O.params(**kw)
        hs.append(L.orc_slot_new(O.C.byref(op), BL.seed_rng(990 + r), None, 0, None, 0, None, None, 0))
    buf = MEM.zeros(R * V, np.float32)
    try:
        for t in range(steps):
            x = np.concatenate([distinct((rng.standard_normal(V) * sg).astype(np.float32)) for (_, sg) in TYPICAL_ROWS])
            buf.upload(x)
            tok = ctx.sample_step(list(range(R)), buf.ptr, V)[0]
            for r in range(R):
                ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
                oti, otl = np.zeros(1, np.int32), np.zeros(1, np.float32)
                eog = O.C.c_int()
                row = np.ascontiguousarray(x[r * V:(r + 1) * V])
                assert L.orc_slot_step(hs[r], O.fp(row), V, 0, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl),
                                       O.C.byref(eog)) == 0
                if tok[r] != ot[0]:
                    return f"step {t} row {r} {TYPICAL_ROWS[r][0]}: token {tok[r]} vs {ot[0]}"
    finally:
        for h in hs:
            L.orc_slot_free(h)
        ctx.close()
    return None


TNS_ROWS = [dict(temperature=0.8, top_k=0, top_n_sigma=1.0),
            dict(temperature=1.0, top_k=64, top_n_sigma=0.5, logprobs=1, n_probs=5),
            dict(temperature=0.7, top_k=0, top_n_sigma=2.0, top_p=0.9),
            dict(temperature=1.2, top_k=0, top_n_sigma=1.5, min_p=0.01)]


def run_tns(BL, steps):
    """Top-n-sigma rows at V=151936 on N(0, 4^2) logits with 300 bumped ids (the sigma from the row pass's
    double-double statistics against the reference's sequential float64 sums): each step's token and the
    logprob against the oracle's slot step. A row whose sigma is undecided reports BL_ETIE, and then the
    oracle's sigma must lie at a float32 rounding boundary of the device's interval (never seen so far)."""
    V = 151936
    R = len(TNS_ROWS)
    rng = np.random.default_rng(31)
    ctx = BL.Context(V, R, R)
    L = O.lib()
    hs = []
    for r, kw in enumerate(TNS_ROWS):
        ctx.slot_reset(r, BL.Params(**kw), BL.seed_rng(700 + r))
        op = O.params(**kw)
        hs.append(L.orc_slot_new(O.C.byref(op), BL.seed_rng(700 + r), None, 0, None, 0, None, None, 0))
    buf = MEM.zeros(R * V, np.float32)
    try:
        for t in range(steps):
            x = (rng.standard_normal(R * V) * 4.0).astype(np.float32)
            x[rng.integers(0, R * V, 300)] += 12.0
            buf.upload(x)
            tok, lp = ctx.sample_step(list(range(R)), buf.ptr, V, top_stride=5)[:2]
            for r in range(R):
                ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
                oti, otl = np.zeros(5, np.int32), np.zeros(5, np.float32)
                eog = O.C.c_int()
                row = np.ascontiguousarray(x[r * V:(r + 1) * V])
                assert L.orc_slot_step(hs[r], O.fp(row), V, 5, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl),
                                       O.C.byref(eog)) == 0
                if tok[r] != ot[0]:
                    return f"step {t} row {r} {TNS_ROWS[r]}: token {tok[r]} vs {ot[0]}"
                if TNS_ROWS[r].get("logprobs") and not lp_close(lp[r], olp[0]):
                    return f"step {t} row {r}: logprob {lp[r]} vs {olp[0]}"
    finally:
        for h in hs:
            L.orc_slot_free(h)
        ctx.close()
    return None


MIRO_ROWS = [(1.0, 5.0, 0.1), (0.7, 3.0, 0.5), (1.5, 8.0, 0.2)]


def miro_logits(rng, V):
    """N(0, 2.5^2) logits with 30 bumped ids and 5 planted equal values (the small cases' shape at any V)."""
    if V == SMALL_V:
        return small_case_logits(rng)
    x = (rng.standard_normal(V) * 2.5).astype(np.float32)
    x[rng.integers(0, V, 30)] += 6.0
    x[rng.integers(0, V, 5)] = x[int(rng.integers(0, V))]
    return x


def run_mirostat(BL, steps, version=2, V=SMALL_V):
    """Mirostat rows (temperature, tau, eta) of one version on logits with planted ties (the heap's order)
    against the oracle's sample_mirostat_v1 / v2, the running mu carried by both; the final RNG states."""
    L = O.lib()
    L.orc_mirostat.restype = O.C.c_int32
    L.orc_mirostat.argtypes = [O.C.c_int, O.C.POINTER(O.C.c_uint64), O.C.POINTER(O.C.c_float), O.C.c_int64,
                               O.C.c_float, O.C.c_float, O.C.c_float, O.C.POINTER(O.C.c_float)]
    R = len(MIRO_ROWS)
    ctx = BL.Context(V, R, R)
    rng = np.random.default_rng(77 + version)
    states, mus = [], []
    for r, (T, tau, eta) in enumerate(MIRO_ROWS):
        ctx.slot_reset(r, BL.Params(temperature=T, mirostat=version, mirostat_tau=tau, mirostat_eta=eta),
                       BL.seed_rng(300 + r))
        states.append(O.C.c_uint64(BL.seed_rng(300 + r)))
        mus.append(O.C.c_float(2.0 * tau))
    buf = MEM.zeros(R * V, np.float32)
    try:
        for t in range(steps):
            xs = [miro_logits(rng, V) for _ in range(R)]
            buf.upload(np.concatenate(xs))
            tok = ctx.sample_step(list(range(R)), buf.ptr, V)[0]
            for r, (T, tau, eta) in enumerate(MIRO_ROWS):
                x = np.ascontiguousarray(xs[r])
                ot = L.orc_mirostat(version, O.C.byref(states[r]), x.ctypes.data_as(O.C.POINTER(O.C.c_float)), V,
                                    T, tau, eta, O.C.byref(mus[r]))
                if tok[r] != ot:
                    return f"step {t} row {r}: token {tok[r]} vs {ot} (mu {mus[r].value})"
        for r in range(R):
            if ctx.slot_rng(r) != states[r].value:
                return f"row {r}: final RNG state differs"
    finally:
        ctx.close()
    return None


ADAPT_ROWS = [(0.3, 0.9, 1.0), (0.05, 0.5, 0.0), (0.8, 0.99, 0.7), (0.0, 0.0, 1.2)]  # target, decay, temperature


def run_adaptive(BL, steps, V=SMALL_V):
    """Adaptive-p rows (target, decay, temperature: the sampler ignores it) on logits with planted ties and
    excluded (-1e30) values against the oracle's sample_adaptive_p, the running weighted sum and total weight
    carried by both; the final RNG states."""
    L = O.lib()
    L.orc_adaptive_p.restype = O.C.c_int32
    L.orc_adaptive_p.argtypes = [O.C.POINTER(O.C.c_uint64), O.C.POINTER(O.C.c_float), O.C.c_int64, O.C.c_float,
                                 O.C.c_float, O.C.POINTER(O.C.c_float), O.C.POINTER(O.C.c_float)]
    R = len(ADAPT_ROWS)
    ctx = BL.Context(V, R, R)
    rng = np.random.default_rng(91)
    states, wss, tws = [], [], []
    for r, (tg, dc, T) in enumerate(ADAPT_ROWS):
        ctx.slot_reset(r, BL.Params(temperature=T, adaptive_target=tg, adaptive_decay=dc), BL.seed_rng(400 + r))
        states.append(O.C.c_uint64(BL.seed_rng(400 + r)))
        one = np.float32(1.0) - np.float32(dc)
        wss.append(O.C.c_float(np.float32(tg) / one))
        tws.append(O.C.c_float(np.float32(1.0) / one))
    buf = MEM.zeros(R * V, np.float32)
    try:
        for t in range(steps):
            xs = [miro_logits(rng, V) for _ in range(R)]
            xs[t % R][rng.integers(0, V, 20)] = np.float32(-1e30)
            buf.upload(np.concatenate(xs))
            tok = ctx.sample_step(list(range(R)), buf.ptr, V)[0]
            for r, (tg, dc, T) in enumerate(ADAPT_ROWS):
                x = np.ascontiguousarray(xs[r])
                ot = L.orc_adaptive_p(O.C.byref(states[r]), x.ctypes.data_as(O.C.POINTER(O.C.c_float)), V, tg, dc,
                                      O.C.byref(wss[r]), O.C.byref(tws[r]))
                if tok[r] != ot:
                    return f"step {t} row {r}: token {tok[r]} vs {ot}"
        for r in range(R):
            if ctx.slot_rng(r) != states[r].value:
                return f"row {r}: final RNG state differs"
    finally:
        ctx.close()
    return None


def run_pair(BL, ca, cb, steps):
    """Two small cases stepped together in one call (rows 0 and 1 of an odd-length vocabulary: row 1 starts
    at a 4-byte but not 16-byte aligned address)."""
    L = O.lib()
    L.orc_set_eog_tokens(O.ip(O.i32([EOS] + EOGS)), 1 + len(EOGS), -1)
    ctx = BL.Context(SMALL_V, 2, 2)
    ctx.set_eog(EOS, EOGS)
    hs, rngs, wants = [], [], []
    for slot, case in enumerate((ca, cb)):
        kw = CASES[case]
        rng, hist, reply, bias = small_case_inputs(case)
        ctx.slot_reset(slot, BL.Params(**kw), BL.seed_rng(100 + case), history=hist, reply=reply, bias=bias)
        op = O.params(**kw)
        hh, rr = O.i32(hist), O.i32(reply)
        bi, bv = O.i32(list(bias.keys())), O.f32(list(bias.values()))
        hs.append(L.orc_slot_new(O.C.byref(op), BL.seed_rng(100 + case), O.ip(hh), len(hist), O.ip(rr), len(reply),
                                 O.ip(bi), O.fp(bv), len(bias)))
        rngs.append(rng)
        wants.append((1 if kw.get("logprobs") else 0, kw.get("n_probs", 0)))
    buf = MEM.zeros(2 * SMALL_V, np.float32)
    stride = max(max(w[1] for w in wants), 1)
    try:
        for t in range(steps):
            xs = [small_case_logits(r) for r in rngs]
            buf.upload(np.concatenate(xs))
            tok, lp, ti, tl = ctx.sample_step([0, 1], buf.ptr, SMALL_V, top_stride=stride)
            for r in range(2):
                ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
                oti, otl = np.full(stride, -1, np.int32), np.zeros(stride, np.float32)
                eg = O.C.c_int()
                assert L.orc_slot_step(hs[r], O.fp(xs[r]), SMALL_V, wants[r][0], 1, O.ip(ot), O.fp(olp), O.ip(oti),
                                       O.fp(otl), O.C.byref(eg)) == 0
                if tok[r] != ot[0]:
                    return f"step {t} row {r}: token {tok[r]} vs {ot[0]}"
                if wants[r][0] and not eg.value:
                    n = wants[r][1]
                    if not lp_close(lp[r], olp[0]) or ti[r][:n] != list(oti[:n]):
                        return f"step {t} row {r}: logprob {lp[r]} vs {olp[0]} or alternatives differ"
    finally:
        for h in hs:
            L.orc_slot_free(h)
        L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
        ctx.close()
    return None


def c2_context(BL, V, seed):
    ctx = BL.Context(V, 8, 8)
    for r in range(8):
        p = BL.Params(temperature=[0.0, 0.7, 1.0][r % 3], top_k=[0, 20, 64][r // 3], top_p=[1.0, 0.9][r % 2],
                      frequency_penalty=0.5, presence_penalty=0.3, logprobs=1, n_probs=10)
        reply = BL.workload_ids(1, 2, seed, r, 4096, V)
        ctx.slot_reset(r, p, BL.seed_rng(seed + r), history=reply, reply=reply,
                       bias=BL.workload_bias(2, seed, r, 300, V, -100.0, 100.0))
    return ctx


def run_w2(BL, steps):
    V, seed, B = 151936, 2, 8
    wt, wl = np.zeros(steps * B, np.int32), np.zeros(steps * B, np.float32)
    wi, wp = np.zeros(steps * B * 10, np.int32), np.zeros(steps * B * 10, np.float32)
    assert O.lib().orc_run_c2(seed, steps, B, O.ip(wt), O.fp(wl), O.ip(wi), O.fp(wp), None) == 0
    ctx = c2_context(BL, V, seed)
    buf = MEM.zeros(B * V, np.float32)
    try:
        for t in range(steps):
            ctx.synth_logits(buf.ptr, V, 2, seed, t, B, V)
            tok, lp, ti, tl = ctx.sample_step(list(range(B)), buf.ptr, V, top_stride=10)
            for r in range(B):
                a = t * B + r
                if tok[r] != wt[a] or not lp_close(lp[r], wl[a]) or ti[r] != list(wi[a * 10:(a + 1) * 10]):
                    return f"step {t} row {r}: token {tok[r]} vs {wt[a]}, logprob {lp[r]} vs {wl[a]}"
                if not all(lp_close(tl[r][q], wp[a * 10 + q]) for q in range(10)):
                    return f"step {t} row {r}: alternative logprobs differ"
    finally:
        ctx.close()
    return None


def run_w4(BL, steps, rows):
    V, seed, B = 262144, 7, 32
    wt, wl = np.zeros(steps * B, np.int32), np.zeros(steps * B, np.float32)
    wi, wp = np.zeros(steps * B * 20, np.int32), np.zeros(steps * B * 20, np.float32)
    assert O.lib().orc_run_c4(seed, steps, B, O.ip(wt), O.fp(wl), O.ip(wi), O.fp(wp), None) == 0
    ctx = BL.Context(V, rows, rows)
    for r in range(rows):
        ctx.slot_reset(r, BL.Params(temperature=1.0, top_k=64, top_p=0.95, logprobs=1, n_probs=20, final_softcap=30.0),
                       BL.seed_rng(seed + r))
    buf = MEM.zeros(rows * V, np.float32)
    try:
        for t in range(steps):
            ctx.synth_logits(buf.ptr, V, 4, seed, t, rows, V)
            tok, lp, ti, tl = ctx.sample_step(list(range(rows)), buf.ptr, V, top_stride=20)
            for r in range(rows):
                a = t * B + r
                if tok[r] != wt[a] or not lp_close(lp[r], wl[a]) or ti[r] != list(wi[a * 20:(a + 1) * 20]):
                    return f"step {t} row {r}: token {tok[r]} vs {wt[a]}, logprob {lp[r]} vs {wl[a]}"
                if not all(lp_close(tl[r][q], wp[a * 20 + q]) for q in range(20)):
                    return f"step {t} row {r}: alternative logprobs differ"
    finally:
        ctx.close()
    return None


def run_w5(BL, steps):
    S, K, V, seed = 16, 8, 151936, 5
    R = S * (K + 1)
    wgt, wga = np.zeros(steps * R, np.int32), np.zeros(steps * S, np.int32)
    wst, wsa = np.zeros(steps * R, np.int32), np.zeros(steps * S, np.int32)
    assert O.lib().orc_run_c5(seed, steps, S, O.ip(wgt), O.ip(wga), O.ip(wst), O.ip(wsa), None) == 0
    g, s = BL.Context(V, S, R), BL.Context(V, S, R)
    for b in range(S):
        g.slot_reset(b, BL.Params(), BL.seed_rng(seed + b))
        s.slot_reset(b, BL.Params(temperature=0.7), BL.seed_rng(seed + b))
    buf = MEM.zeros(R * V, np.float32)
    try:
        for t in range(steps):
            g.synth_logits(buf.ptr, V, 5, seed, t, R, V)
            am = np.argmax(buf.host().reshape(R, V), axis=1)
            drafts = []
            for b in range(S):
                drafts += BL.workload_drafts(seed, t, b, [int(x) for x in am[b * (K + 1):b * (K + 1) + K]], V)
            gt, ga = g.spec_verify(list(range(S)), K, buf.ptr, V, drafts)
            st, sa = s.spec_verify(list(range(S)), K, buf.ptr, V, drafts)
            if gt != list(wgt[t * R:(t + 1) * R]) or ga != list(wga[t * S:(t + 1) * S]):
                return f"greedy step {t}"
            if st != list(wst[t * R:(t + 1) * R]) or sa != list(wsa[t * S:(t + 1) * S]):
                return f"sampled step {t}"
    finally:
        g.close()
        s.close()
    return None


def run_spec_penalties(BL, rounds, K=6):
    """Speculative verification of rows with frequency/presence/repeat penalties (row i sees the drafts before
    it in its history and reply): every row's token, the accepted length and, at the end, the RNG state equal
    the oracle's spec_verify over the same rows, round after round (the device commits in between). Drafts
    repeat a few hot tokens so that the penalties decide rows; a 3-token window makes drafts leave it. K drafts
    per sequence (row K holds up to 2 K count corrections)."""
    V = 997
    confs = [dict(temperature=0.0, repeat_penalty=1.3, repeat_last_n=3, frequency_penalty=0.4, presence_penalty=0.2),
             dict(temperature=0.8, top_k=0, repeat_penalty=1.2, repeat_last_n=8, frequency_penalty=0.3,
                  presence_penalty=0.1),
             dict(temperature=0.0, repeat_penalty=1.5, repeat_last_n=-1),
             dict(temperature=0.7, top_k=20, frequency_penalty=0.8, presence_penalty=0.5)]
    S = len(confs)
    rng = np.random.default_rng(21)
    hot = [int(x) for x in rng.choice(V, 6, replace=False)]
    L = O.lib()
    L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
    ctx = BL.Context(V, S, S * (K + 1))
    hs = []
    buf = MEM.zeros(S * (K + 1) * V, np.float32)
    try:
        for b, kw in enumerate(confs):
            hist = [int(x) for x in rng.choice(hot + [int(y) for y in rng.integers(0, V, 6)], 12)]
            ctx.slot_reset(b, BL.Params(**kw), BL.seed_rng(300 + b), history=hist, reply=hist)
            op = O.params(**kw)
            hh = O.i32(hist)
            hs.append(L.orc_slot_new(O.C.byref(op), BL.seed_rng(300 + b), O.ip(hh), len(hist), O.ip(hh), len(hist),
                                     None, None, 0))
        for t in range(rounds):
            rows = (rng.standard_normal((S * (K + 1), V)) * 2.0).astype(np.float32)
            rows[:, hot] += np.float32(5.0)
            drafts = []
            for b in range(S):
                for i in range(K):
                    r = rows[b * (K + 1) + i]
                    drafts.append(int(np.argmax(r)) if rng.random() < 0.7 else hot[int(rng.integers(0, len(hot)))])
            buf.upload(rows.reshape(-1))
            toks, acc = ctx.spec_verify(list(range(S)), K, buf.ptr, V, drafts)
            for b in range(S):
                ot = np.zeros(K + 1, np.int32)
                oa = O.C.c_int32()
                assert L.orc_slot_spec_verify(hs[b], O.fp(rows[b * (K + 1):(b + 1) * (K + 1)].reshape(-1)), V,
                                              O.ip(O.i32(drafts[b * K:(b + 1) * K])), K, O.ip(ot), O.C.byref(oa)) == 0
                if toks[b * (K + 1):(b + 1) * (K + 1)] != list(ot) or acc[b] != oa.value:
                    return (f"round {t} sequence {b} ({confs[b]}): tokens {toks[b * (K + 1):(b + 1) * (K + 1)]} "
                            f"vs {list(ot)}, accepted {acc[b]} vs {oa.value}")
        for b in range(S):
            if ctx.slot_rng(b) != L.orc_slot_rng(hs[b]):
                return f"sequence {b}: final RNG state differs"
    finally:
        for h in hs:
            L.orc_slot_free(h)
        ctx.close()
    return None


def run_async(BL, steps):
    """bl_bind_rows + bl_sample_step_async into caller buffers equals the synchronous step."""
    V, seed, B = 151936, 2, 8
    pool = [MEM.zeros(B * V, np.float32) for _ in range(steps)]
    eager = c2_context(BL, V, seed)
    for t in range(steps):
        eager.synth_logits(pool[t].ptr, V, 2, seed, t, B, V)
    want = [eager.sample_step(list(range(B)), pool[t].ptr, V, top_stride=10)[:2] for t in range(steps)]
    eager.close()
    ctx = c2_context(BL, V, seed)
    ctx.bind_rows(list(range(B)))
    tok, lp = MEM.zeros(B, np.int32), MEM.zeros(B, np.float32)
    ti, tl = MEM.zeros(B * 10, np.int32), MEM.zeros(B * 10, np.float32)
    try:
        for t in range(steps):
            ctx.sample_step_async(B, pool[t].ptr, V, tok.ptr, lp.ptr, ti.ptr, tl.ptr, 10)
            if tok.host().tolist() != list(want[t][0]) or lp.host().tolist() != list(want[t][1]):
                return f"step {t}: asynchronous step differs from the synchronous one"
    finally:
        ctx.close()
    return None


NOALLOC_ROWS = [
    dict(temperature=0.0, logprobs=1, n_probs=10),
    dict(temperature=0.7, top_k=20, frequency_penalty=0.5, presence_penalty=0.3, logprobs=1, n_probs=10),
    dict(temperature=1.0, top_p=0.9, logprobs=1, n_probs=10),
    dict(temperature=0.8, top_k=64, min_p=0.05, repeat_penalty=1.1),
    dict(temperature=1.0, mirostat=2, mirostat_tau=5.0, mirostat_eta=0.1),
    dict(temperature=0.9, top_p=0.95, logprobs=1, n_probs=5, post_sampling_probs=1),
    dict(temperature=1.0, top_k=40, xtc_probability=0.5, xtc_threshold=0.1),
    dict(temperature=0.6, logprobs=1, n_probs=3, frequency_penalty=0.2),
]


def run_noalloc(BL):
    """bl_sample_rows_noalloc, twice in a row (the second call smaller), equals bl_sample_step over fresh
    slots with the same parameters and RNG states."""
    seed = 5
    for B, V, ld, step in ((8, 151936, 151936, 0), (3, 50000, 50048, 1)):
        buf = MEM.zeros(B * ld, np.float32)
        gen = BL.Context(V, 1, 1)
        gen.synth_logits(buf.ptr, ld, 2, seed, step, B, V)
        gen.close()
        params = [BL.Params(**NOALLOC_ROWS[(r + step) % len(NOALLOC_ROWS)]) for r in range(B)]
        rngs = [BL.seed_rng(seed * 100 + 10 * step + r) for r in range(B)]
        got = BL.sample_rows_noalloc(params, rngs, buf.ptr, ld, V, top_stride=10)
        ctx = BL.Context(V, B, B)
        for r in range(B):
            ctx.slot_reset(r, params[r], rngs[r])
        want = list(ctx.sample_step(list(range(B)), buf.ptr, ld, top_stride=10)) + [[ctx.slot_rng(r) for r in range(B)]]
        ctx.close()
        if got[0] != want[0]:
            return f"B={B} V={V}: tokens {got[0]} vs {want[0]}"
        if not all(lp_close(a, b) for a, b in zip(got[1], want[1])):
            return f"B={B} V={V}: logprobs differ"
        if got[2] != want[2] or not all(lp_close(a, b) for x, y in zip(got[3], want[3]) for a, b in zip(x, y)):
            return f"B={B} V={V}: alternatives differ"
        if got[4] != want[4]:
            return f"B={B} V={V}: RNG states differ"
    return None


def run_bigk(BL, steps):
    """top_k 250 and 256 logprob alternatives at V=151936: 38 chunks x 256 candidates per row."""
    V, seed = 151936, 11
    kw = dict(temperature=0.9, top_k=250, top_p=0.95, logprobs=1, n_probs=256, frequency_penalty=0.2)
    L = O.lib()
    L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
    reply = [int(x) for x in np.random.default_rng(seed).integers(0, V, 64)]
    op = O.params(**kw)
    rr = O.i32(reply)
    h = L.orc_slot_new(O.C.byref(op), BL.seed_rng(seed), O.ip(rr), len(reply), O.ip(rr), len(reply), None, None, 0)
    ctx = BL.Context(V, 1, 1)
    ctx.slot_reset(0, BL.Params(**kw), BL.seed_rng(seed), history=reply, reply=reply)
    buf = MEM.zeros(V, np.float32)
    try:
        for t in range(steps):
            ctx.synth_logits(buf.ptr, V, 2, seed, t, 1, V)
            x = buf.host()
            tok, lp, ti, tl = ctx.sample_step([0], buf.ptr, V, top_stride=256)
            ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
            oti, otl = np.zeros(256, np.int32), np.zeros(256, np.float32)
            eg = O.C.c_int()
            assert L.orc_slot_step(h, O.fp(x), V, 1, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl), O.C.byref(eg)) == 0
            if tok[0] != ot[0] or not lp_close(lp[0], olp[0]):
                return f"step {t}: token {tok[0]} vs {ot[0]}, logprob {lp[0]} vs {olp[0]}"
            if ti[0] != list(oti) or not all(lp_close(tl[0][q], otl[q]) for q in range(256)):
                return f"step {t}: alternatives differ"
    finally:
        L.orc_slot_free(h)
        ctx.close()
    return None


GOLDEN = os.path.join(ROOT, "tests", "golden")


def run_w3(BL, steps, check_masks=True, schema=None):
    """Workload 3: greedy decode under the config-3 JSON-Schema grammar, masks and tokens per step. With
    `schema` (the schema's JSON text) the slot is constrained through bl_slot_schema instead of the
    committed GBNF text."""
    V, seed = 151936, 3
    L = O.lib()
    L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
    wt, wc, wf = np.zeros(steps, np.int32), np.zeros(steps, np.uint32), np.zeros(steps, np.int32)
    assert L.orc_run_c3(seed, steps, 1, O.ip(wt), wc.ctypes.data_as(O.C.POINTER(O.C.c_uint32)), O.ip(wf), None) == 0, \
        O.last_error()
    blob, off, eos = BL.workload_c3_vocab(seed, V)
    with open(os.path.join(GOLDEN, "c3_schema.gbnf")) as f:
        gbnf = f.read()
    ctx = BL.Context(V, 1, 1)
    ctx.set_eog(eos, [])
    ctx.set_vocab(blob, off)

    def restart():
        ctx.slot_reset(0, BL.Params(), BL.seed_rng(seed))
        if schema is None:
            ctx.slot_grammar(0, gbnf)
        else:
            ctx.slot_schema(0, schema)

    restart()
    buf = MEM.zeros(V, np.float32)
    mask = MEM.zeros((V + 31) // 32, np.uint32)
    try:
        for t in range(steps):
            ctx.synth_logits(buf.ptr, V, 3, seed, t, 1, V)
            if check_masks:
                forced = ctx.grammar_mask(0, mask.ptr)
                m = mask.host()
                crc = L.orc_crc32(m.ctypes.data, m.nbytes)
                if crc != wc[t] or int(forced) != wf[t]:
                    return f"step {t}: mask crc {crc:#x} vs {int(wc[t]):#x}, forced {forced} vs {wf[t]}"
            tok = ctx.sample_step([0], buf.ptr, V)[0][0]
            if tok != wt[t]:
                return f"step {t}: token {tok} vs {wt[t]}"
            if tok == eos:
                restart()
    finally:
        ctx.close()
    return None


# byte-level vocabulary with every lone byte, UTF-8 fragments and whole characters, and a grammar whose
# classes see non-ASCII text: exercises the carry of unfinished sequences and the trailing U+FFFD rule
GRAMMAR_CASES = [
    'root ::= "{" [^"}]* "}" "x"?\n',
    'root ::= ([a-c] | [\\u00e0-\\u00ff] | "\\u20ac")+ ";"\n',
    'root ::= "\\"" ( [^"\\\\] | "\\\\" ["\\\\n] )* "\\"" [ ]{0,3}\n',
    'root ::= ("ab" | "a" [^b])* "!" | [0-9]{2,4}\n',
    None,  # the workload-3 schema grammar (tests/golden/c3_schema.gbnf)
    'root ::= [^\\x00-\\x7f]{1,6} ("." [^\\x00-\\x7f])* ";"\n',
    'root ::= ("\\u00e9\\u20ac" | "\\U0001F600" | "a")+ "."\n',
    'root ::= "x" [0-9]+ ";"\n',  # few allowed tokens: sampled top-k rows widen past the merged list
]


def grammar_vocab(rng, n_extra):
    pieces = [bytes([b]) for b in range(256)]
    chars = ["a", "b", "c", "{", "}", '"', "\\", "!", ";", "x", " ", "é", "ÿ", "€", "\U0001F600", "�",
             "n", "0", "7"]
    for _ in range(n_extra):
        k = int(rng.integers(1, 5))
        s = "".join(chars[int(i)] for i in rng.integers(0, len(chars), k)).encode()
        if rng.random() < 0.3:  # a fragment: cut inside a multi-byte sequence
            cut = int(rng.integers(0, len(s) + 1))
            s = s[cut:] if rng.random() < 0.5 else s[:cut]
        if not s:
            s = bytes([int(rng.integers(0, 256))])
        pieces.append(s)
    pieces.append(b"<|eos|>")
    off = [0]
    for pc in pieces:
        off.append(off[-1] + len(pc))
    return b"".join(pieces), off, len(pieces) - 1


# sampled grammar rows (src/server.br:323-362): (grammar case, parameters, logit sigma)
GRAMMAR_SAMPLED = [
    (0, dict(temperature=0.8, top_k=40), 3.0),
    (3, dict(temperature=0.8, top_k=40, top_p=0.9, logprobs=1, n_probs=4), 3.0),
    (4, dict(temperature=1.0, top_k=0, min_p=0.05), 3.0),
    (2, dict(temperature=0.7, top_k=0, repeat_penalty=1.2, repeat_last_n=16, logprobs=1, n_probs=3,
             post_sampling_probs=1), 3.0),
    (6, dict(temperature=1.2, top_k=200, xtc_probability=0.5, xtc_threshold=0.1), 3.0),
    (1, dict(temperature=0.9, top_k=5), 3.0),
    # widening past the merged top-256 list (levels 640 and the whole vocabulary)
    (7, dict(temperature=0.9, top_k=40), 3.0),
    (7, dict(temperature=0.8, top_k=10, logprobs=1, n_probs=2), 2.0),
    # full-vocabulary rows whose allowed maximum lies far below the row maximum
    (4, dict(temperature=1.0, top_k=0), 12.0),
    (7, dict(temperature=0.8, top_k=0, top_p=0.95), 12.0),
]


def run_grammar_case(BL, case, steps, kw=None, sigma=3.0, quant=0.0):
    """Masks and tokens of a small grammar against the oracle's slot on random rows: greedy, or sampled with
    the parameters `kw` (the RNG carried across the replies that end or die); logits N(0, sigma^2), rounded to
    multiples of `quant` when given (equal allowed maxima)."""
    kw = kw or {}
    seed = 77 if kw else 1
    rng = np.random.default_rng(500 + case)
    blob, off, eos = grammar_vocab(rng, 700)
    V = len(off) - 1
    gbnf = GRAMMAR_CASES[case]
    if gbnf is None:
        with open(os.path.join(GOLDEN, "c3_schema.gbnf")) as f:
            gbnf = f.read()
    L = O.lib()
    L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
    op = O.params(**kw)
    rs = BL.seed_rng(seed) if kw else 1
    h = L.orc_slot_new(O.C.byref(op), rs, None, 0, None, 0, None, None, 0)
    oo = np.array(off, np.uint32)
    assert L.orc_slot_set_grammar(h, gbnf.encode(), blob, oo.ctypes.data_as(O.C.POINTER(O.C.c_uint32)), V,
                                  eos) == 0, O.last_error()
    ctx = BL.Context(V, 1, 1)
    ctx.set_eog(eos, [])
    ctx.set_vocab(blob, off)
    ctx.slot_reset(0, BL.Params(**kw), rs)
    ctx.slot_grammar(0, gbnf)
    wants = 1 if kw.get("logprobs") else 0
    n_probs = kw.get("n_probs", 0)

    def restart():
        L.orc_slot_restart(h)
        ctx.slot_reset(0, BL.Params(**kw), ctx.slot_rng(0))
        ctx.slot_grammar(0, gbnf)
    words = (V + 31) // 32
    mask, want = MEM.zeros(words, np.uint32), np.zeros(words, np.uint32)
    buf = MEM.zeros(V, np.float32)
    try:
        for t in range(steps):
            of = O.C.c_int()
            ok = L.orc_slot_grammar_mask(h, V, want.ctypes.data_as(O.C.POINTER(O.C.c_uint32)), O.C.byref(of), 1)
            try:
                forced = ctx.grammar_mask(0, mask.ptr)
            except BL.BLError as e:
                if e.code != BL.BL_EGRAMMAR_DEAD or ok != 0:
                    return f"step {t}: device '{e}', oracle mask status {ok}"
                # both find the reply dead (a piece can be allowed and the re-decoded reply still fail,
                # src/server.br:311-318): start a new reply
                restart()
                continue
            if ok != 1:
                return f"step {t}: the oracle's reply is dead ({ok}) but the device's is not"
            got = mask.host()
            if not np.array_equal(got, want) or bool(of.value) != forced:
                bad = np.nonzero(got != want)[0]
                return f"step {t}: mask differs in {len(bad)} words (first {bad[:4]}), forced {forced} vs {of.value}"
            x = (rng.standard_normal(V) * sigma).astype(np.float32)
            if quant:
                x = (np.round(x / quant) * quant).astype(np.float32)
            buf.upload(x)
            ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
            oti, otl = np.full(max(n_probs, 1), -1, np.int32), np.zeros(max(n_probs, 1), np.float32)
            eg = O.C.c_int()
            orc = L.orc_slot_step(h, O.fp(x), V, wants, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl), O.C.byref(eg))
            try:
                tok, lp, ti, tl = ctx.sample_step([0], buf.ptr, V, top_stride=max(n_probs, 1))
                tok = tok[0]
            except BL.BLError as e:
                # the reference's errors (dead reply, every token rejected) must be the same errors
                if orc == 0 or O.last_error() not in str(e):
                    return f"step {t}: device error '{e}', oracle {'token ' + str(ot[0]) if orc == 0 else O.last_error()}"
                return None
            if orc != 0:
                return f"step {t}: oracle error '{O.last_error()}', device token {tok}"
            if tok != ot[0]:
                return f"step {t}: token {tok} vs {ot[0]}"
            if wants and not eg.value:
                if not lp_close(lp[0], olp[0]):
                    return f"step {t}: logprob {lp[0]} vs {olp[0]}"
                if ti[0][:n_probs] != list(oti[:n_probs]) or not all(lp_close(tl[0][q], otl[q]) for q in range(n_probs)):
                    return f"step {t}: alternatives differ"
            if kw and ctx.slot_rng(0) != L.orc_slot_rng(h):
                return f"step {t}: RNG state differs"
            if tok == eos:
                restart()
    finally:
        L.orc_slot_free(h)
        ctx.close()
    return None


JSON_CASES = [
    # response_format json_object (src/server.br:261-304): (parameters, logit sigma)
    (dict(temperature=0.0), 3.0),
    (dict(temperature=0.8, top_k=40), 3.0),
    (dict(temperature=1.0, top_k=0, min_p=0.02, logprobs=1, n_probs=3), 4.0),
    (dict(temperature=0.7, top_k=10, repeat_penalty=1.3, repeat_last_n=8, ignore_eos=1), 3.0),
]


def json_vocab(rng, n_extra):
    """Byte tokens plus pieces of JSON syntax, literals, numbers and multi-byte characters (some cut inside a
    UTF-8 sequence), and an end-of-sequence token."""
    pieces = [bytes([b]) for b in range(256)]
    chars = ["{", "}", "[", "]", ":", ",", '"', "\\", " ", "\n", "t", "r", "u", "e", "f", "a", "l", "s", "n",
             "0", "1", "9", "-", ".", "E", "+", "é", "€", "\U0001F600", "x", "k"]
    for _ in range(n_extra):
        k = int(rng.integers(1, 6))
        s = "".join(chars[int(i)] for i in rng.integers(0, len(chars), k)).encode()
        if rng.random() < 0.2:
            cut = int(rng.integers(0, len(s) + 1))
            s = s[cut:] if rng.random() < 0.5 else s[:cut]
        if not s:
            s = bytes([int(rng.integers(0, 256))])
        pieces.append(s)
    for w in (b'{"', b'":', b'",', b'"}', b"true", b"null", b"false", b"12", b"-0.5", b"1e+3", b"[]", b"{}", b"  "):
        pieces.append(w)
    pieces.append(b"<|eos|>")
    off = [0]
    for pc in pieces:
        off.append(off[-1] + len(pc))
    return b"".join(pieces), off, len(pieces) - 1


def run_json_case(BL, case, steps):
    """Masks and tokens of a response_format json_object slot against the oracle's sample_json_token: the
    classifier over the re-decoded reply, forced end of sequence on a complete object, rank-order widening,
    the sampling chain over the allowed candidates; a new reply after each end of sequence."""
    kw, sigma = JSON_CASES[case]
    rng = np.random.default_rng(800 + case)
    blob, off, eos = json_vocab(rng, 900)
    V = len(off) - 1
    L = O.lib()
    L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
    L.orc_slot_set_json_object.argtypes = [O.C.c_void_p, O.C.c_char_p, O.C.POINTER(O.C.c_uint32), O.C.c_int64,
                                           O.C.c_int32]
    op = O.params(**kw)
    rs = BL.seed_rng(60 + case)
    h = L.orc_slot_new(O.C.byref(op), rs, None, 0, None, 0, None, None, 0)
    oo = np.array(off, np.uint32)
    L.orc_slot_set_json_object(h, blob, oo.ctypes.data_as(O.C.POINTER(O.C.c_uint32)), V, eos)
    ctx = BL.Context(V, 1, 1)
    ctx.set_eog(eos, [])
    ctx.set_vocab(blob, off)
    ctx.slot_reset(0, BL.Params(**kw), rs)
    ctx.slot_json_object(0)
    wants = 1 if kw.get("logprobs") else 0
    n_probs = kw.get("n_probs", 0)

    def restart():
        L.orc_slot_restart(h)
        ctx.slot_reset(0, BL.Params(**kw), ctx.slot_rng(0))
        ctx.slot_json_object(0)
    words = (V + 31) // 32
    mask, want = MEM.zeros(words, np.uint32), np.zeros(words, np.uint32)
    buf = MEM.zeros(V, np.float32)
    # closing pieces favoured, so that replies complete (and the end of sequence is forced) now and then
    closing = np.array([b"}" in blob[off[i]:off[i + 1]] or b'"' in blob[off[i]:off[i + 1]] for i in range(V)])
    ends = 0
    try:
        for t in range(steps):
            of = O.C.c_int()
            L.orc_slot_grammar_mask(h, V, want.ctypes.data_as(O.C.POINTER(O.C.c_uint32)), O.C.byref(of), 1)
            forced = ctx.grammar_mask(0, mask.ptr)
            got = mask.host()
            if not np.array_equal(got, want) or bool(of.value) != forced:
                bad = np.nonzero(got != want)[0]
                return f"step {t}: mask differs in {len(bad)} words (first {bad[:4]}), forced {forced} vs {of.value}"
            x = (rng.standard_normal(V) * sigma).astype(np.float32)
            x[closing] += np.float32(3.0 * sigma)
            buf.upload(x)
            ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
            oti, otl = np.full(max(n_probs, 1), -1, np.int32), np.zeros(max(n_probs, 1), np.float32)
            eg = O.C.c_int()
            orc = L.orc_slot_step(h, O.fp(x), V, wants, 1, O.ip(ot), O.fp(olp), O.ip(oti), O.fp(otl), O.C.byref(eg))
            try:
                tok, lp, ti, tl = ctx.sample_step([0], buf.ptr, V, top_stride=max(n_probs, 1))
                tok = tok[0]
            except BL.BLError as e:
                if orc == 0 or O.last_error() not in str(e):
                    return f"step {t}: device error '{e}', oracle {'token ' + str(ot[0]) if orc == 0 else O.last_error()}"
                return None
            if orc != 0:
                return f"step {t}: oracle error '{O.last_error()}', device token {tok}"
            if tok != ot[0]:
                return f"step {t}: token {tok} vs {ot[0]}"
            if wants and not eg.value:
                if not lp_close(lp[0], olp[0]):
                    return f"step {t}: logprob {lp[0]} vs {olp[0]}"
                if ti[0][:n_probs] != list(oti[:n_probs]) or not all(lp_close(tl[0][q], otl[q]) for q in range(n_probs)):
                    return f"step {t}: alternatives differ"
            if ctx.slot_rng(0) != L.orc_slot_rng(h):
                return f"step {t}: RNG state differs"
            if tok == eos:
                ends += 1
                restart()
    finally:
        L.orc_slot_free(h)
        ctx.close()
    return None


def parse_range(s):
    out = []
    for part in s.split(","):
        if "-" in part:
            a, b = part.split("-")
            out += list(range(int(a), int(b) + 1))
        else:
            out.append(int(part))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib", required=True)
    ap.add_argument("items", nargs="+")
    a = ap.parse_args()
    BL = load_binding(a.lib)
    failed = 0
    for item in a.items:
        f = item.split(":")
        kind = f[0]
        results = []
        if kind == "small":
            for c in parse_range(f[1]):
                results.append((f"small case {c}", run_small(BL, c, int(f[2]) if len(f) > 2 else 25)))
        elif kind == "coarse":
            for c in parse_range(f[1]):
                results.append((f"coarse case {c}", run_small(BL, c, int(f[2]) if len(f) > 2 else 25, coarse=True)))
        elif kind in ("bf16", "q4"):
            for c in parse_range(f[1]):
                results.append((f"{kind} case {c}", run_small(BL, c, int(f[2]) if len(f) > 2 else 25, quant=kind)))
        elif kind == "ramp":
            for c in parse_range(f[1]):
                results.append((f"ramp case {c}", run_small(BL, c, int(f[2]) if len(f) > 2 else 25, ramp=True)))
        elif kind == "w2":
            results.append(("workload 2", run_w2(BL, int(f[1]))))
        elif kind == "w4":
            results.append(("workload 4", run_w4(BL, int(f[1]), int(f[2]) if len(f) > 2 else 32)))
        elif kind == "w5":
            results.append(("workload 5", run_w5(BL, int(f[1]))))
        elif kind == "specpen":  # specpen:rounds[:K]
            K = int(f[2]) if len(f) > 2 else 6
            results.append((f"speculative rows with penalties, {K} drafts", run_spec_penalties(BL, int(f[1]), K)))
        elif kind == "async":
            results.append(("asynchronous step", run_async(BL, int(f[1]))))
        elif kind == "pair":
            results.append((f"rows {f[1]} + {f[2]}", run_pair(BL, int(f[1]), int(f[2]), int(f[3]) if len(f) > 3 else 10)))
        elif kind == "bigties":
            results.append(("bf16 ties at V=151936", run_bigties(BL, int(f[1]))))
        elif kind == "tns":
            results.append(("top-n-sigma rows at V=151936", run_tns(BL, int(f[1]))))
        elif kind == "miro":
            results.append(("mirostat v2 rows", run_mirostat(BL, int(f[1]))))
        elif kind == "dry":  # dry:cases[:steps]
            for c in parse_range(f[1]):
                results.append((f"DRY case {c}", run_dry(BL, c, int(f[2]) if len(f) > 2 else 20)))
        elif kind == "adapt":  # adapt:steps[:V]
            V = int(f[2]) if len(f) > 2 else SMALL_V
            results.append((f"adaptive-p rows at V={V}", run_adaptive(BL, int(f[1]), V)))
        elif kind == "miro1":  # miro1:steps[:V]
            V = int(f[2]) if len(f) > 2 else SMALL_V
            results.append((f"mirostat v1 rows at V={V}", run_mirostat(BL, int(f[1]), 1, V)))
        elif kind == "unfilt":
            rows = [int(v) for v in f[2].split(",")] if len(f) > 2 else None
            results.append(("unfiltered rows at V=151936", run_unfiltered(BL, int(f[1]), rows)))
        elif kind == "gtie":  # gtie:cases[:steps]: greedy grammar rows on logits in steps of 0.5
            for c in parse_range(f[1]):
                for kw in ({}, {"top_k": 40}):
                    results.append((f"grammar ties case {c} top_k {kw.get('top_k', 0)}",
                                    run_grammar_case(BL, c, int(f[2]) if len(f) > 2 else 30, kw, quant=0.5)))
        elif kind == "gstie":  # gstie:cases[:steps]: sampled grammar rows (T 0.8) on logits in steps of 0.5
            for c in parse_range(f[1]):
                for kw in ({"temperature": 0.8}, {"temperature": 0.8, "top_k": 40}):
                    results.append((f"sampled grammar ties case {c} top_k {kw.get('top_k', 0)}",
                                    run_grammar_case(BL, c, int(f[2]) if len(f) > 2 else 30, kw, quant=0.5)))
        elif kind == "typical":  # typical:steps:V
            V = int(f[2]) if len(f) > 2 else SMALL_V
            results.append((f"typical rows at V={V}", run_typical(BL, int(f[1]), V)))
        elif kind == "halfway":
            results.append(("halfway tail terms", run_halfway(BL, int(f[1]))))
        elif kind == "noalloc":
            results.append(("allocation-free step", run_noalloc(BL)))
        elif kind == "bigk":
            results.append(("large top-k / n_probs", run_bigk(BL, int(f[1]))))
        elif kind == "w3":
            results.append(("workload 3", run_w3(BL, int(f[1]))))
        elif kind == "w3schema":  # the same decode with the slot constrained through bl_slot_schema
            schema = ('{"type":"object","properties":{"name":{"type":"string","pattern":"^[a-z_]+$"},'
                      '"count":{"type":"integer"},"tags":{"type":"array","items":{"type":"string"}}},'
                      '"required":["name","count","tags"]}')
            results.append(("workload 3 via the schema entry point", run_w3(BL, int(f[1]), schema=schema)))
        elif kind == "gsamp":  # sampled grammar rows: gsamp:indices[:steps]
            for c in parse_range(f[1]):
                gc, gkw, gsig = GRAMMAR_SAMPLED[c]
                results.append((f"sampled grammar {c}",
                                 run_grammar_case(BL, gc, int(f[2]) if len(f) > 2 else 30, gkw, gsig)))
        elif kind == "json":  # json:cases[:steps]
            for c in parse_range(f[1]):
                results.append((f"JSON-object case {c}", run_json_case(BL, c, int(f[2]) if len(f) > 2 else 40)))
        elif kind == "grammar":
            for c in parse_range(f[1]):
                results.append((f"grammar case {c}", run_grammar_case(BL, c, int(f[2]) if len(f) > 2 else 30)))
        else:
            raise SystemExit(f"unknown item {item}")
        for name, err in results:
            failed += err is not None
            print(f"ok   {name}" if err is None else f"FAIL {name}: {err}", flush=True)
    sys.exit(1 if failed else 0)


if __name__ == "__main__":
    main()
