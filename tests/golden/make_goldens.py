"""Regenerates the oracle's golden vectors under tests/golden/ (run from the repo root:
python tests/golden/make_goldens.py). The vectors are the CPU oracle's outputs on the seeded
workloads; the tests check that the oracle still produces them and that the device matches them."""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import _oracle as O  # noqa: E402

L = O.lib()


def rng_streams():
    out = {}
    for seed in (0, 1, 7, 42, 1234):
        st = O.seed_rng(seed)
        u, f = [], []
        s = st
        for _ in range(64):
            v, s2 = O.rng_next_u64(s)
            ff, _ = O.rng_next_f32(s)
            u.append(str(v))
            f.append(float(ff).hex())
            s = s2
        out[str(seed)] = {"state": str(st), "u64": u, "f32": f}
    return out


def main():
    with open(os.path.join(HERE, "rng_streams.json"), "w") as fh:
        json.dump(rng_streams(), fh, indent=1)
    n = 64
    t = np.zeros(n, np.int32)
    assert L.orc_run_c1(1234, n, O.ip(t), None) == 0
    np.savetxt(os.path.join(HERE, "c1_tokens.txt"), t, fmt="%d")
    steps, B = 12, 8
    wt, wl = np.zeros(steps * B, np.int32), np.zeros(steps * B, np.float32)
    wi, wp = np.zeros(steps * B * 10, np.int32), np.zeros(steps * B * 10, np.float32)
    assert L.orc_run_c2(2, steps, B, O.ip(wt), O.fp(wl), O.ip(wi), O.fp(wp), None) == 0
    np.savez(os.path.join(HERE, "c2_golden.npz"), tokens=wt, logprobs=wl, top_ids=wi, top_logprobs=wp)


if __name__ == "__main__":
    main()
