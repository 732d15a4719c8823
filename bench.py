"""Benchmark of boring-llm's per-step token selection on one MI355X.

Workload: B=8 slots, V=151936, per-row temperature {0,0.7,1.0} x top_k
{0,20,64} x top_p {1.0,0.9}, frequency 0.5 / presence 0.3 over 4096 Zipf(1.1) reply ids, 300 logit_bias
ids in [-100,100], n_probs=10 logprobs, logits ~N(0,4^2). A step is one decode-loop sampling block for
the 8 rows (transform, rank, exact draw, logprobs, history commit) through the C ABI. Inputs are
resident in HBM: the logits of up to 512 distinct workload steps (at least 64 of them, 311 MB, more than
the 256 MB Infinity Cache) are generated on the device beforehand; step t reads those of step t mod P.

Prints one JSON line. `value` is steps/s of back-to-back direct launches of the step, each writing its
tokens and logprobs to its own row of a device log; after the timed region the logged warmup and timed
steps (up to --check-steps of them) are compared with the oracle's stream of the same workload, and a
mismatch fails the run. p50 is one step + stream synchronisation (direct launches, and HIP-graph replays).
`roofline` is the step's: the 4*B*V logits a step must read over the summed durations of its three kernels,
each timed by the start and end events of an extended launch (the kernel's own execution); a second entry
does the same for the row pass, the kernel that reads the logits. `traffic` is FETCH_SIZE + WRITE_SIZE per
launch from the committed counter summary. The CPU baseline times the oracle (the reference's algorithms
restated in C++: per-stage row copies, insertion top-k, heap sort, hash maps, sequential sums) on one host
core over a bounded sample of the same workload.
"""
import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "boring-llm_amd"))

METRIC = "sampling steps/s + p50 µs/step at B=8,V=151936; HBM GB/s vs peak"
V, B, SEED, POOL_MAX, TOPN = 151936, 8, 2, 512, 10
HBM_PEAK_GBS = 8000.0


def setup_slots(BL, ctx):
    for r in range(B):
        p = BL.Params(temperature=[0.0, 0.7, 1.0][r % 3], top_k=[0, 20, 64][r // 3], top_p=[1.0, 0.9][r % 2],
                      frequency_penalty=0.5, presence_penalty=0.3, logprobs=1, n_probs=TOPN)
        reply = BL.workload_ids(1, 2, SEED, r, 4096, V)
        ctx.slot_reset(r, p, BL.seed_rng(SEED + r), history=reply, reply=reply,
                       bias=BL.workload_bias(2, SEED, r, 300, V, -100.0, 100.0))


def cpu_baseline(target_s):
    """The oracle on one core over the first steps of the workload (all 8 rows per step)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import ctypes
    import _oracle as O
    L = O.lib()
    steps = 4
    while True:
        t = np.zeros(steps * B, np.int32)
        lp = np.zeros(steps * B, np.float32)
        ti = np.zeros(steps * B * TOPN, np.int32)
        tl = np.zeros(steps * B * TOPN, np.float32)
        us = ctypes.c_double()
        assert L.orc_run_c2(SEED, steps, B, O.ip(t), O.fp(lp), O.ip(ti), O.fp(tl), ctypes.byref(us)) == 0
        sec = us.value / 1e6
        if sec >= target_s or steps >= 4096:
            break
        steps = min(4096, steps * 4, max(steps * 2, int(steps * target_s / max(sec, 1e-3)) + 1))
    return {"value": steps / sec, "unit": "steps/s", "cores": 1, "kind": "port",
            "sample": f"first {steps} steps of the workload, 8 rows each, oracle (oracle/liboracle.so) on one "
                      f"host core ({platform.processor() or platform.machine()}, nproc {os.cpu_count()}); "
                      f"{sec:.1f} s of sampling time excluding input generation",
            "ms_per_step": 1e3 * sec / steps}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_step_b8_v151936.json")


def measured_traffic():
    """HBM bytes per launch of each step kernel (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration),
    from the committed hardware-counter summary; None when it is absent."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        t = json.load(f)
    return {k: v["bytes_per_launch"] for k, v in t["kernels"].items()}


def cpu_sample(run, target_s, unit_steps=1):
    """Grows the oracle's step count (at most 4x per run: a step's cost can grow with the history, as the
    grammar path's whole-reply re-decode does) until its own timer passes target_s; returns (steps, seconds)."""
    import ctypes
    steps = 2
    while True:
        us = ctypes.c_double()
        run(steps, ctypes.byref(us))
        sec = us.value / 1e6
        if sec >= target_s or steps >= 4096:
            return steps, sec
        steps = min(4096, steps * 4, max(steps * 2, int(steps * target_s / max(sec, 1e-3)) + 1))


def bench_workload(args, wl):
    """Configs 1, 3, 4 and 5 of BASELINE.json (parity-tested elsewhere; timed here on request)."""
    import torch
    import bl_select as BL
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _oracle as O
    L = O.lib()
    dev = torch.device("cuda:0")
    out = {"metric": f"workload {wl} steps/s + p50 us/step", "unit": "steps/s", "n_gpus": 1, "higher_is_better": True,
           "dtype": "f32", "data": f"synthetic (seeded integer-hash inputs, BASELINE configs[{wl - 1}])", "vs_baseline": None}
    lat, elapsed, steps = [], 0.0, args.steps
    if wl in (1, 4):
        if wl == 1:
            V, B, seed, pool_n, cfg = 151936, 1, 1234, 512, 1
            params = [BL.Params(temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64)]
            desc = "B=1, V=151936, T 0.8, top_k 40, top_p 0.95, min_p 0.05, repeat 1.1 over the last 64 of 512 ids"
        else:
            V, B, seed, pool_n, cfg = 262144, 32, 7, 16, 4
            params = [BL.Params(temperature=1.0, top_k=64, top_p=0.95, logprobs=1, n_probs=20, final_softcap=30.0)] * B
            desc = "B=32, V=262144, soft-cap 30, T 1.0, top_k 64, top_p 0.95, 20 logprobs"
        ctx = BL.Context(V, B, B)
        for r in range(B):
            hist = BL.workload_ids(0, 1, seed, 0, 512, V) if wl == 1 else []
            ctx.slot_reset(r, params[r], BL.seed_rng(seed + r), history=hist)
        ctx.bind_rows(list(range(B)))
        pool = torch.empty((pool_n, B, V), dtype=torch.float32, device=dev)
        for p in range(pool_n):
            ctx.synth_logits(pool[p].data_ptr(), V, cfg, seed, p, B, V)
        topn = 20 if wl == 4 else 0
        d_tok = torch.zeros(B, dtype=torch.int32, device=dev)
        d_lp = torch.zeros(B, dtype=torch.float32, device=dev)
        d_ti = torch.zeros(max(B * topn, 1), dtype=torch.int32, device=dev)
        d_tl = torch.zeros(max(B * topn, 1), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        graphs = [ctx.step_graph(B, pool[p].data_ptr(), V, d_tok.data_ptr(), d_lp.data_ptr(), d_ti.data_ptr(),
                                 d_tl.data_ptr(), topn) for p in range(pool_n)]
        for i in range(args.warmup):
            ctx.graph_launch(graphs[i % pool_n])
        ctx.sync()
        t0 = time.perf_counter()
        for i in range(steps):
            ctx.graph_launch(graphs[i % pool_n])
        ctx.sync()
        elapsed = time.perf_counter() - t0
        for i in range(min(steps, 500)):
            a = time.perf_counter()
            ctx.graph_launch(graphs[i % pool_n])
            ctx.sync()
            lat.append(time.perf_counter() - a)
        for g in graphs:
            BL.Context.graph_destroy(g)
        ctx.close()
        out["config"] = {"workload": desc, "batch": B, "vocab": V, "hip_graph": True,
                         "logits_pool_MB": pool_n * B * V * 4 / 1e6}
        if not args.no_cpu:
            if wl == 1:
                n, sec = cpu_sample(lambda k, us: L.orc_run_c1(seed, k, O.ip(np.zeros(k, np.int32)), us), args.cpu_seconds)
            else:
                def run4(k, us):
                    z = lambda m, t: np.zeros(m, t)
                    L.orc_run_c4(seed, k, B, O.ip(z(k * B, np.int32)), O.fp(z(k * B, np.float32)),
                                 O.ip(z(k * B * 20, np.int32)), O.fp(z(k * B * 20, np.float32)), us)
                n, sec = cpu_sample(run4, args.cpu_seconds)
    elif wl == 3:
        V, seed = 151936, 3
        blob, off, eos = BL.workload_c3_vocab(seed, V)
        with open(os.path.join(ROOT, "tests", "golden", "c3_schema.gbnf")) as f:
            gbnf = f.read()
        ctx = BL.Context(V, 1, 1)
        ctx.set_eog(eos, [])
        ctx.set_vocab(blob, off)

        def restart():
            ctx.slot_reset(0, BL.Params(), BL.seed_rng(seed))
            ctx.slot_grammar(0, gbnf)

        restart()
        pool_n = 256
        pool = torch.empty((pool_n, V), dtype=torch.float32, device=dev)
        for p in range(pool_n):
            ctx.synth_logits(pool[p].data_ptr(), V, 3, seed, p, 1, V)
        torch.cuda.synchronize()
        steps = min(steps, 256)
        for i in range(steps + args.warmup):
            a = time.perf_counter()
            tok = ctx.sample_step([0], pool[i % pool_n].data_ptr(), V)[0][0]
            dt = time.perf_counter() - a
            if i >= args.warmup:
                lat.append(dt)
                elapsed += dt
            if tok == eos:
                restart()  # the forced EOS ends the reply; the next request starts over (not timed)
        ctx.close()
        out["config"] = {"workload": "B=1 grammar-constrained greedy, V=151936 synthetic vocabulary, the config-3 "
                                     "JSON-Schema GBNF; synchronous bl_sample_step (host outputs)", "batch": 1,
                         "vocab": V, "hip_graph": False}
        if not args.no_cpu:
            L.orc_set_eog_tokens(O.ip(O.i32([0])), 0, -1)
            n, sec = cpu_sample(lambda k, us: L.orc_run_c3(seed, k, 0, O.ip(np.zeros(k, np.int32)),
                                                            np.zeros(k, np.uint32).ctypes.data_as(
                                                                O.C.POINTER(O.C.c_uint32)),
                                                            O.ip(np.zeros(k, np.int32)), us), args.cpu_seconds)
    elif wl == 5:
        S, K, V, seed = 16, 8, 151936, 5
        R = S * (K + 1)
        pool_n = 4
        g, sm = BL.Context(V, S, R), BL.Context(V, S, R)
        for b in range(S):
            g.slot_reset(b, BL.Params(), BL.seed_rng(seed + b))
            sm.slot_reset(b, BL.Params(temperature=0.7), BL.seed_rng(seed + b))
        pool = torch.empty((pool_n, R, V), dtype=torch.float32, device=dev)
        drafts = []
        for p in range(pool_n):
            g.synth_logits(pool[p].data_ptr(), V, 5, seed, p, R, V)
            am = pool[p].argmax(dim=1).cpu().numpy()
            dp = []
            for b in range(S):
                dp += BL.workload_drafts(seed, p, b, [int(x) for x in am[b * (K + 1):b * (K + 1) + K]], V)
            drafts.append(dp)
        torch.cuda.synchronize()
        steps = min(steps, 200)
        per = {}
        for name, ctx in (("greedy", g), ("sampled_T0.7", sm)):
            for i in range(args.warmup):
                ctx.spec_verify(list(range(S)), K, pool[i % pool_n].data_ptr(), V, drafts[i % pool_n])
            ts = []
            for i in range(steps):
                a = time.perf_counter()
                ctx.spec_verify(list(range(S)), K, pool[i % pool_n].data_ptr(), V, drafts[i % pool_n])
                ts.append(time.perf_counter() - a)
            per[name] = {"steps_per_s": len(ts) / sum(ts), "p50_us": 1e6 * float(np.median(ts))}
            lat += ts
            elapsed += sum(ts)
        g.close()
        sm.close()
        steps = len(lat)
        out["config"] = {"workload": "speculative verification, 16 sequences x 9 rows, V=151936, greedy and "
                                     "sampled (T 0.7, top_k 0) contexts; synchronous bl_spec_verify", "batch": R,
                         "vocab": V, "hip_graph": False, "per_mode": per}
        if not args.no_cpu:
            def run5(k, us):
                z = lambda m: np.zeros(m, np.int32)
                L.orc_run_c5(seed, k, S, O.ip(z(k * R)), O.ip(z(k * S)), O.ip(z(k * R)), O.ip(z(k * S)), us)
            n, sec = cpu_sample(run5, args.cpu_seconds)
    else:
        raise SystemExit(f"bench.py: unknown workload {wl}")
    out.update({"value": steps / elapsed, "steps": steps, "warmup": args.warmup, "ms_per_step": 1e3 * elapsed / steps,
                "p50_us_per_step": 1e6 * float(np.median(lat)), "scaling": "weak"})
    if not args.no_cpu:
        out["cpu_baseline"] = {"value": n / sec, "unit": "steps/s", "cores": 1, "kind": "port",
                               "sample": f"first {n} steps of workload {wl}, oracle on one host core; {sec:.1f} s"}
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph latency leg (hardware-counter runs)")
    ap.add_argument("--check-steps", type=int, default=256,
                    help="leading steps of the logged stream compared with the oracle after the timed region")
    ap.add_argument("--copy-calib", action="store_true",
                    help="run only a plain 256 MiB device-to-device copy (calibrates FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--workload", type=int, default=2,
                    help="BASELINE.json config (1-5); 2, the headline workload, is the default")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; the path shards by slot with no exchange "
              "(see DESIGN.md), and no multi-GPU figure is produced", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calib:
        n = 64 << 20  # 256 MiB of float32 each way
        a = torch.ones(n, dtype=torch.float32, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_read": 4 * n, "copy_calib_bytes_written": 4 * n, "launches": 5}))
        return

    if args.workload != 2:
        bench_workload(args, args.workload)
        return

    import bl_select as BL

    dev = torch.device("cuda:0")
    ctx = BL.Context(V, B, B)
    setup_slots(BL, ctx)
    ctx.bind_rows(list(range(B)))
    W, K = args.warmup, args.steps
    n_stream = W + K  # the warmup and timed steps: their tokens and logprobs are logged
    # step t reads the logits of workload step t % P (P distinct steps, 64 of them already larger than the
    # 256 MB Infinity Cache); the checked steps are all distinct, so their stream is the oracle's
    P = max(64, min(n_stream, POOL_MAX))
    pool = torch.empty((P, B, V), dtype=torch.float32, device=dev)
    for p in range(P):
        ctx.synth_logits(pool[p].data_ptr(), V, 2, SEED, p, B, V)
    log_tok = torch.full((n_stream, B), -2, dtype=torch.int32, device=dev)
    log_lp = torch.zeros((n_stream, B), dtype=torch.float32, device=dev)
    d_tok = torch.zeros(B, dtype=torch.int32, device=dev)
    d_lp = torch.zeros(B, dtype=torch.float32, device=dev)
    d_ti = torch.zeros(B * TOPN, dtype=torch.int32, device=dev)
    d_tl = torch.zeros(B * TOPN, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def launch(i, tok, lp):
        ctx.sample_step_async(B, pool[i % P].data_ptr(), V, tok, lp, d_ti.data_ptr(), d_tl.data_ptr(), TOPN)

    def logged(i):
        launch(i, log_tok[i].data_ptr(), log_lp[i].data_ptr())

    for i in range(W):
        logged(i)
    ctx.sync()
    # throughput: K back-to-back steps (direct launches; each step's outputs go to its own log row)
    t0 = time.perf_counter()
    for i in range(W, W + K):
        logged(i)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    checked = check_tokens(log_tok.cpu().numpy(), log_lp.cpu().numpy(), min(n_stream, args.check_steps, P))

    # latency: one step + stream synchronisation, continuing the stream
    nxt = n_stream
    lat_d = []
    for i in range(min(K, 1000)):
        a = time.perf_counter()
        launch(nxt, d_tok.data_ptr(), d_lp.data_ptr())
        ctx.sync()
        lat_d.append(time.perf_counter() - a)
        nxt += 1
    p50_direct = 1e6 * float(np.median(lat_d))
    # the same with the step captured in a HIP graph (bl_step_graph_create: no allocation, no host work)
    p50_graph = None
    if not args.no_graph:
        graphs = [ctx.step_graph(B, pool[(nxt + g) % P].data_ptr(), V, d_tok.data_ptr(), d_lp.data_ptr(),
                                 d_ti.data_ptr(), d_tl.data_ptr(), TOPN) for g in range(16)]
        lat_g = []
        for i in range(min(K, 500)):
            a = time.perf_counter()
            ctx.graph_launch(graphs[i % 16])
            ctx.sync()
            lat_g.append(time.perf_counter() - a)
        for g in graphs:
            BL.Context.graph_destroy(g)
        p50_graph = 1e6 * float(np.median(lat_g))
        nxt += len(lat_g)
    p50_us = min(p50_direct, p50_graph) if p50_graph is not None else p50_direct

    # each kernel's own duration (start and end events of an extended launch, on the launch stream)
    ctx.set_timing(True)
    n_t = min(K, 400)
    for i in range(n_t):
        launch(nxt + i, d_tok.data_ptr(), d_lp.data_ptr())
    kms, nsteps = ctx.get_timing()
    ctx.set_timing(False)
    ctx.sync()

    names = ["bl_k_rowpass", "bl_k_exppass", "bl_k_select"]
    kus = {names[k]: 1e3 * kms[k] for k in range(3)}
    step_us = sum(kus.values())
    alg_bytes = 4.0 * B * V  # the logits a step must read (the path's algorithmic traffic)
    traffic = measured_traffic()
    step_traffic = sum(traffic.values()) if traffic else None
    achieved = alg_bytes / (step_us * 1e-6) / 1e9
    k1 = kus["bl_k_rowpass"]
    out = {
        "metric": METRIC,
        "value": K / elapsed,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": 1e3 * elapsed / K,
        "p50_us_per_step": p50_us,
        "p50_us_by_launch": {"direct_launches": p50_direct, "graph_replay": p50_graph},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded integer-hash logits, Zipf histories, bias lists; BASELINE configs[1])",
        "config": {"workload": "B=8 slots, V=151936, per-row T/top_k/top_p table, freq 0.5 / presence 0.3 over "
                               "4096 Zipf(1.1) ids, 300 bias ids in [-100,100], n_probs 10",
                   "batch": B, "vocab": V, "launch": "direct", "logits_pool_MB": P * B * V * 4 / 1e6},
        "kernels_us": kus,
        "kernels_timed_steps": nsteps,
        "step_kernels_us": step_us,
        # the step: the logits it must read over its three kernels' summed durations
        "roofline": {"bound": "hbm", "kernel": "step: bl_k_rowpass + bl_k_exppass + bl_k_select",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": step_traffic, "algorithmic_bytes_per_launch": alg_bytes},
        # the kernel that reads the logits first (the row pass)
        "roofline_logits_kernel": {"bound": "hbm", "kernel": "bl_k_rowpass", "achieved": alg_bytes / (k1 * 1e-6) / 1e9,
                                   "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                   "frac": alg_bytes / (k1 * 1e-6) / 1e9 / HBM_PEAK_GBS,
                                   "traffic": traffic.get("bl_k_rowpass") if traffic else None,
                                   "algorithmic_bytes_per_launch": alg_bytes},
        "traffic_bytes_per_launch": traffic,
        "traffic_vs_algorithmic": step_traffic / alg_bytes if traffic else None,
        "tokens_checked": checked,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out))
    if not checked["tokens_match"] or not checked["logprobs_within_tolerance"]:
        print(f"bench.py: the timed steps differ from the oracle's stream: {checked}", file=sys.stderr)
        sys.exit(1)


def check_tokens(tok, lp, n):
    """The first n logged steps against the oracle's stream of the workload (tokens bit-exact, logprobs within
    the 1e-5 relative tolerance of the north star)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import ctypes
    import _oracle as O
    wt = np.zeros(n * B, np.int32)
    wl = np.zeros(n * B, np.float32)
    wi = np.zeros(n * B * TOPN, np.int32)
    wp = np.zeros(n * B * TOPN, np.float32)
    assert O.lib().orc_run_c2(SEED, n, B, O.ip(wt), O.fp(wl), O.ip(wi), O.fp(wp), ctypes.byref(ctypes.c_double())) == 0
    got_t = tok[:n].reshape(-1)
    got_l = lp[:n].reshape(-1).astype(np.float64)
    bad = np.nonzero(got_t != wt)[0]
    rel = np.abs(got_l - wl) / np.maximum(np.maximum(np.abs(got_l), np.abs(wl)), 1e-30)
    return {"steps": int(n), "rows": B, "first_step": 0, "tokens_match": bool(len(bad) == 0),
            "first_mismatch": None if len(bad) == 0 else [int(bad[0] // B), int(bad[0] % B)],
            "logprob_max_rel_err": float(rel.max()) if n else 0.0,
            "logprobs_within_tolerance": bool((rel <= 1e-5).all())}


if __name__ == "__main__":
    main()
