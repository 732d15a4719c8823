"""Benchmark of boring-llm's per-step token selection on one MI355X.

Workload: B=8 slots, V=151936, per-row temperature {0,0.7,1.0} x top_k
{0,20,64} x top_p {1.0,0.9}, frequency 0.5 / presence 0.3 over 4096 Zipf(1.1) reply ids, 300 logit_bias
ids in [-100,100], n_probs=10 logprobs, logits ~N(0,4^2). A step is one decode-loop sampling block for
the 8 rows (transform, rank, exact draw, logprobs, history commit) through the C ABI. Inputs are
resident in HBM: a pool of 64 steps of logits (311 MB, more than the 256 MB Infinity Cache) is
generated on the device beforehand and the steps cycle through it.

Prints one JSON line. `value` is steps/s of back-to-back HIP-graph replays; p50 is one replay + sync.
The roofline object reports the dominant kernel's algorithmic HBM bytes (the 4*B*V logits it must read)
over its event-timed average duration against 8 TB/s. The CPU baseline times the oracle (the
reference's algorithms restated in C++: per-stage row copies, insertion top-k, heap sort, hash maps,
sequential sums) on one host core over a bounded sample of the same workload.
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
V, B, SEED, POOL, TOPN = 151936, 8, 2, 64, 10
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
        steps = min(4096, max(steps * 2, int(steps * target_s / max(sec, 1e-3)) + 1))
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="direct launches (hardware-counter runs)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="run only a plain 256 MiB device-to-device copy (calibrates FETCH_SIZE/WRITE_SIZE)")
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

    import bl_select as BL

    dev = torch.device("cuda:0")
    ctx = BL.Context(V, B, B)
    setup_slots(BL, ctx)
    ctx.bind_rows(list(range(B)))
    pool = torch.empty((POOL, B, V), dtype=torch.float32, device=dev)
    for p in range(POOL):
        ctx.synth_logits(pool[p].data_ptr(), V, 2, SEED, p, B, V)
    d_tok = torch.zeros(B, dtype=torch.int32, device=dev)
    d_lp = torch.zeros(B, dtype=torch.float32, device=dev)
    d_ti = torch.zeros(B * TOPN, dtype=torch.int32, device=dev)
    d_tl = torch.zeros(B * TOPN, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def launch(p):
        ctx.sample_step_async(B, pool[p].data_ptr(), V, d_tok.data_ptr(), d_lp.data_ptr(), d_ti.data_ptr(),
                              d_tl.data_ptr(), TOPN)

    # one HIP graph per pool entry, captured by the library on its own stream (bl_step_graph_create): no
    # allocation and no host synchronisation inside a step
    graphs = []
    if not args.no_graph:
        graphs = [ctx.step_graph(B, pool[p].data_ptr(), V, d_tok.data_ptr(), d_lp.data_ptr(), d_ti.data_ptr(),
                                 d_tl.data_ptr(), TOPN) for p in range(POOL)]
    use_graph = bool(graphs)

    def step(i):
        if use_graph:
            ctx.graph_launch(graphs[i % POOL])
        else:
            launch(i % POOL)

    for i in range(args.warmup):
        step(i)
    ctx.sync()

    # throughput: K back-to-back steps
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    ctx.sync()
    elapsed = time.perf_counter() - t0

    # latency: one step + stream synchronisation
    lat = []
    base = args.warmup + args.steps
    for i in range(min(args.steps, 1000)):
        a = time.perf_counter()
        step(base + i)
        ctx.sync()
        lat.append(time.perf_counter() - a)
    p50_us = 1e6 * float(np.median(lat))

    # per-kernel durations (events around each kernel on the launch stream)
    ctx.set_timing(True)
    n_t = min(args.steps, 400)
    for i in range(n_t):
        launch((base + i) % POOL)
    kms, nsteps = ctx.get_timing()
    ctx.set_timing(False)
    ctx.sync()
    for g in graphs:
        BL.Context.graph_destroy(g)

    names = ["bl_k_rowpass", "bl_k_exppass", "bl_k_select"]
    dom = int(np.argmax(kms))
    alg_bytes = 4.0 * B * V  # logits each step must read (the path's algorithmic traffic)
    achieved = alg_bytes / (kms[dom] * 1e-3) / 1e9
    traffic = measured_traffic()
    out = {
        "metric": METRIC,
        "value": args.steps / elapsed,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * elapsed / args.steps,
        "p50_us_per_step": p50_us,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded integer-hash logits, Zipf histories, bias lists; BASELINE configs[1])",
        "config": {"workload": "B=8 slots, V=151936, per-row T/top_k/top_p table, freq 0.5 / presence 0.3 over "
                               "4096 Zipf(1.1) ids, 300 bias ids in [-100,100], n_probs 10",
                   "batch": B, "vocab": V, "hip_graph": use_graph, "logits_pool_MB": POOL * B * V * 4 / 1e6},
        "kernels_us": {names[k]: 1e3 * kms[k] for k in range(3)},
        "roofline": {"bound": "hbm", "kernel": names[dom], "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic.get(names[dom]) if traffic else None,
                     "algorithmic_bytes_per_launch": alg_bytes},
        "traffic_bytes_per_launch": traffic,
        # each kernel's measured HBM bytes (counters) over its event-timed duration
        "kernel_hbm_GBs": ({names[k]: traffic[names[k]] / (kms[k] * 1e-3) / 1e9 for k in range(3)}
                           if traffic else None),
        "hbm_GBs_step": alg_bytes / (1e-3 * sum(kms)) / 1e9,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
