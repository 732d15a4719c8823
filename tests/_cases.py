"""Parameter sets of the small-vocabulary parity cases, shared by the GPU tests and the CPU emulator runs.

Each case is one bl_params / oracle Params configuration; the inputs (history, reply, logit_bias, planted
ties) are drawn from numpy's default_rng(case) in `small_case_inputs`.
"""
import numpy as np

CASES = [
    dict(temperature=0.0),
    dict(temperature=0.9, top_k=5),
    dict(temperature=1.3, top_k=0),
    dict(temperature=0.5, top_k=0, top_p=0.8, min_p=0.02),
    dict(temperature=0.7, top_k=50, top_p=0.9, min_p=0.1, min_keep=3),
    dict(temperature=1.0, top_k=200, repeat_penalty=1.3, repeat_last_n=16),
    dict(temperature=0.8, top_k=0, repeat_penalty=0.9, repeat_last_n=-1, frequency_penalty=0.4, presence_penalty=-0.2),
    dict(temperature=0.0, repeat_penalty=1.5, repeat_last_n=8, logprobs=1, n_probs=5),
    dict(temperature=1.0, top_k=10, logprobs=1, n_probs=12, ignore_eos=1),
    dict(temperature=2.0, top_k=0, logprobs=1, n_probs=3, final_softcap=5.0),
    dict(temperature=0.6, top_k=30, logit_mul=0.5, logprobs=1, n_probs=1),
    # XTC (src/sampling.br:552-572) and post-sampling probabilities (src/server.br:1015-1025)
    dict(temperature=0.9, top_k=40, xtc_probability=0.6, xtc_threshold=0.1, logprobs=1, n_probs=6,
         post_sampling_probs=1),
    dict(temperature=1.1, top_k=0, top_p=0.95, xtc_probability=0.5, xtc_threshold=0.05),
    dict(temperature=0.8, top_k=0, xtc_probability=0.7, xtc_threshold=0.2, min_keep=2, logprobs=1, n_probs=4,
         post_sampling_probs=1),
    dict(temperature=0.0, logprobs=1, n_probs=3, post_sampling_probs=1),
    dict(temperature=1.2, top_k=0, min_p=0.05, logprobs=1, n_probs=8, post_sampling_probs=1),
    # dynamic temperature, exponent 1 (src/sampling.br:467-488)
    dict(temperature=0.9, top_k=30, dynatemp_range=0.5, logprobs=1, n_probs=4, post_sampling_probs=1),
    dict(temperature=1.0, top_k=0, min_p=0.05, dynatemp_range=0.8),
    dict(temperature=0.4, top_k=0, dynatemp_range=0.6, xtc_probability=0.5, xtc_threshold=0.15),
    # the typical filter (src/sampling.br:424-465) on top-k lists
    dict(temperature=0.9, top_k=50, typical_p=0.6, logprobs=1, n_probs=5, post_sampling_probs=1),
    dict(temperature=1.1, top_k=120, typical_p=0.9, min_keep=4, top_p=0.95, min_p=0.02, xtc_probability=0.4,
         xtc_threshold=0.1, dynatemp_range=0.3),
    # top-n-sigma (src/sampling.br:376-407) before a full-vocabulary rank and before top-k
    dict(temperature=0.9, top_k=0, top_n_sigma=1.5, logprobs=1, n_probs=4),
    dict(temperature=1.0, top_k=40, top_n_sigma=0.8, top_p=0.9, repeat_penalty=1.2, repeat_last_n=16),
    dict(temperature=1.2, top_k=0, top_n_sigma=3.0, min_p=0.02, frequency_penalty=0.3, presence_penalty=0.2),
    # dynamic temperature with exponents other than 1 (glibc powf of the normalised entropy)
    dict(temperature=1.0, top_k=0, min_p=0.05, dynatemp_range=0.8, dynatemp_exponent=0.5),
    dict(temperature=0.9, top_k=30, dynatemp_range=0.5, dynatemp_exponent=2.3, logprobs=1, n_probs=4,
         post_sampling_probs=1),
]
SMALL_V = 5003
EOS, EOGS = 7, [11, 13]


def small_case_inputs(case):
    """(rng, history, reply, bias) of a small case; the rng then draws the per-step logits."""
    rng = np.random.default_rng(case)
    hist = [int(x) for x in rng.integers(0, SMALL_V, 40)]
    reply = hist[-15:]
    bias = {int(i): float(np.float32(v)) for i, v in zip(rng.integers(0, SMALL_V, 20), rng.uniform(-5, 5, 20))}
    return rng, hist, reply, bias


def small_case_logits(rng):
    """One step's logits: N(0, 2.5^2), 30 bumped ids and 5 planted equal values."""
    x = (rng.standard_normal(SMALL_V) * 2.5).astype(np.float32)
    x[rng.integers(0, SMALL_V, 30)] += 6.0
    x[rng.integers(0, SMALL_V, 5)] = x[int(rng.integers(0, SMALL_V))]
    return x
