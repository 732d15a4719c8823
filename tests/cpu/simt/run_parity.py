"""Parity of the library's kernels, run on the CPU SIMT emulator, against the oracle (test infrastructure).

The emulator build (tests/cpu/simt/Makefile) compiles the same kernel and C-ABI sources as the HIP
library, with every GPU thread a fiber; device pointers are host pointers. This script loads a private
copy of the Python binding pointed at that build (the product module and its library path are left
alone) and checks the workloads the GPU parity tests check, at reduced step counts:

    python run_parity.py --lib _build/libbl_simt.so small:0-10:25 w2:2 w4:1:8 w5:1 async:2

Items: small:<cases>:<steps>, w2:<steps>, w4:<steps>:<rows>, w5:<steps>, async:<steps>.
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

LP_RTOL = 1e-5


def load_binding(lib_path):
    spec = importlib.util.spec_from_file_location("bl_select_simt", os.path.join(ROOT, "boring-llm_amd", "bl_select.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    m.LIB_PATH = os.path.abspath(lib_path)
    m._lib = None
    return m


def lp_close(a, b):
    a, b = np.float32(a), np.float32(b)
    return abs(a - b) <= LP_RTOL * max(abs(a), abs(b)) or abs(a - b) <= 1e-7


def run_small(BL, case, steps):
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
    buf = np.zeros(SMALL_V, np.float32)
    try:
        for t in range(steps):
            x = small_case_logits(rng)
            buf[:] = x
            tok, lp, ti, tl = ctx.sample_step([1], buf.ctypes.data, SMALL_V, top_stride=max(n_probs, 1))
            ot, olp = np.zeros(1, np.int32), np.zeros(1, np.float32)
            oti, otl = np.zeros(max(n_probs, 1), np.int32), np.zeros(max(n_probs, 1), np.float32)
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
    buf = np.zeros(B * V, np.float32)
    try:
        for t in range(steps):
            ctx.synth_logits(buf.ctypes.data, V, 2, seed, t, B, V)
            tok, lp, ti, tl = ctx.sample_step(list(range(B)), buf.ctypes.data, V, top_stride=10)
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
    buf = np.zeros(rows * V, np.float32)
    try:
        for t in range(steps):
            ctx.synth_logits(buf.ctypes.data, V, 4, seed, t, rows, V)
            tok, lp, ti, tl = ctx.sample_step(list(range(rows)), buf.ctypes.data, V, top_stride=20)
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
    buf = np.zeros(R * V, np.float32)
    try:
        for t in range(steps):
            g.synth_logits(buf.ctypes.data, V, 5, seed, t, R, V)
            am = np.argmax(buf.reshape(R, V), axis=1)
            drafts = []
            for b in range(S):
                drafts += BL.workload_drafts(seed, t, b, [int(x) for x in am[b * (K + 1):b * (K + 1) + K]], V)
            gt, ga = g.spec_verify(list(range(S)), K, buf.ctypes.data, V, drafts)
            st, sa = s.spec_verify(list(range(S)), K, buf.ctypes.data, V, drafts)
            if gt != list(wgt[t * R:(t + 1) * R]) or ga != list(wga[t * S:(t + 1) * S]):
                return f"greedy step {t}"
            if st != list(wst[t * R:(t + 1) * R]) or sa != list(wsa[t * S:(t + 1) * S]):
                return f"sampled step {t}"
    finally:
        g.close()
        s.close()
    return None


def run_async(BL, steps):
    """bl_bind_rows + bl_sample_step_async into caller buffers equals the synchronous step."""
    V, seed, B = 151936, 2, 8
    pool = np.zeros((steps, B * V), np.float32)
    eager = c2_context(BL, V, seed)
    for t in range(steps):
        eager.synth_logits(pool[t].ctypes.data, V, 2, seed, t, B, V)
    want = [eager.sample_step(list(range(B)), pool[t].ctypes.data, V, top_stride=10)[:2] for t in range(steps)]
    eager.close()
    ctx = c2_context(BL, V, seed)
    ctx.bind_rows(list(range(B)))
    tok, lp = np.zeros(B, np.int32), np.zeros(B, np.float32)
    ti, tl = np.zeros(B * 10, np.int32), np.zeros(B * 10, np.float32)
    try:
        for t in range(steps):
            ctx.sample_step_async(B, pool[t].ctypes.data, V, tok.ctypes.data, lp.ctypes.data, ti.ctypes.data,
                                  tl.ctypes.data, 10)
            if tok.tolist() != list(want[t][0]) or lp.tolist() != list(want[t][1]):
                return f"step {t}: asynchronous step differs from the synchronous one"
    finally:
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
        elif kind == "w2":
            results.append(("workload 2", run_w2(BL, int(f[1]))))
        elif kind == "w4":
            results.append(("workload 4", run_w4(BL, int(f[1]), int(f[2]) if len(f) > 2 else 32)))
        elif kind == "w5":
            results.append(("workload 5", run_w5(BL, int(f[1]))))
        elif kind == "async":
            results.append(("asynchronous step", run_async(BL, int(f[1]))))
        else:
            raise SystemExit(f"unknown item {item}")
        for name, err in results:
            failed += err is not None
            print(f"ok   {name}" if err is None else f"FAIL {name}: {err}", flush=True)
    sys.exit(1 if failed else 0)


if __name__ == "__main__":
    main()
