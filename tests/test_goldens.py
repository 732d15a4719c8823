"""The committed golden vectors (tests/golden/, written by make_goldens.py from the oracle): the RNG streams
against the xorshift64 closed form computed with Python integers, and the oracle's workload-1/2 outputs
against the files (a regression check: the device tests compare against the same files)."""
import json
import os

import numpy as np

import _oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MASK = (1 << 64) - 1


def test_rng_streams_closed_form():
    # src/sampling.br:35-54: seed fold, xorshift64 (13, 7, 17), u64 -> f32 / 2^64
    from test_oracle_pinning import u64_to_f32, xorshift
    streams = json.load(open(os.path.join(HERE, "rng_streams.json")))
    assert set(streams) == {"0", "1", "7", "42", "1234"}
    for seed, s in streams.items():
        seed = int(seed)
        st = 88172645463325252 if seed == 0 else (seed & MASK) ^ 88172645463325252
        assert int(s["state"]) == st == O.seed_rng(seed)
        for u, f in zip(s["u64"], s["f32"]):
            x = xorshift(st)
            assert int(u) == x
            assert float.fromhex(f) == u64_to_f32(x) / 2.0 ** 64
            st = x


def test_oracle_reproduces_c2_golden():
    g = np.load(os.path.join(HERE, "c2_golden.npz"))
    steps, B = 12, 8
    wt, wl = np.zeros(steps * B, np.int32), np.zeros(steps * B, np.float32)
    wi, wp = np.zeros(steps * B * 10, np.int32), np.zeros(steps * B * 10, np.float32)
    assert O.lib().orc_run_c2(2, steps, B, O.ip(wt), O.fp(wl), O.ip(wi), O.fp(wp), None) == 0
    assert np.array_equal(wt, g["tokens"]) and np.array_equal(wl, g["logprobs"])
    assert np.array_equal(wi, g["top_ids"]) and np.array_equal(wp, g["top_logprobs"])


def test_oracle_reproduces_c1_golden():
    want = np.loadtxt(os.path.join(HERE, "c1_tokens.txt"), dtype=np.int32)
    t = np.zeros(len(want), np.int32)
    assert O.lib().orc_run_c1(1234, len(want), O.ip(t), None) == 0
    assert np.array_equal(t, want)
