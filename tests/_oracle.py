"""ctypes binding of the CPU oracle (oracle/liboracle.so) for the tests and the benchmark baseline.

The oracle is the checker: it is never part of the product path.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "liboracle.so")

_lib = None

f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)
u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)
i64 = C.c_int64


class OrcParams(C.Structure):
    _fields_ = [
        ("temperature", C.c_float), ("dynatemp_range", C.c_float), ("dynatemp_exponent", C.c_float),
        ("top_n_sigma", C.c_float), ("top_k", i64), ("typical_p", C.c_float), ("top_p", C.c_float),
        ("min_p", C.c_float), ("xtc_probability", C.c_float), ("xtc_threshold", C.c_float), ("min_keep", i64),
        ("repeat_penalty", C.c_float), ("repeat_last_n", i64), ("dry_multiplier", C.c_float),
        ("dry_base", C.c_float), ("dry_allowed_length", i64), ("dry_penalty_last_n", i64),
        ("frequency_penalty", C.c_float), ("presence_penalty", C.c_float), ("n_probs", i64),
        ("post_sampling_probs", i64), ("ignore_eos", i64), ("final_softcap", C.c_float), ("logit_mul", C.c_float),
    ]


def params(**kw):
    """SamplingParams defaults of greedy_params() (src/model.br:1586-1589) plus server extras."""
    p = OrcParams(temperature=0.0, dynatemp_range=0.0, dynatemp_exponent=1.0, top_n_sigma=-1.0, top_k=0,
                  typical_p=1.0, top_p=1.0, min_p=0.0, xtc_probability=0.0, xtc_threshold=0.1, min_keep=0,
                  repeat_penalty=1.0, repeat_last_n=64, dry_multiplier=0.0, dry_base=1.75, dry_allowed_length=2,
                  dry_penalty_last_n=64, frequency_penalty=0.0, presence_penalty=0.0, n_probs=0,
                  post_sampling_probs=0, ignore_eos=0, final_softcap=0.0, logit_mul=1.0)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            subprocess.check_call(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
        _lib = _configure(C.CDLL(LIB))
    return _lib


def mutant(k):
    """The oracle built with planted mistake k (oracle/Makefile `mutants`): the checks that pin the oracle
    must fail against it."""
    path = os.path.join(ROOT, "oracle", f"liboracle_mut{k}.so")
    subprocess.check_call(["make", "-s", "-C", os.path.join(ROOT, "oracle"), f"liboracle_mut{k}.so"])
    return _configure(C.CDLL(path))


def _configure(L):
    if True:
        L.orc_last_error.restype = C.c_char_p
        L.orc_seed_rng.restype = C.c_uint64
        L.orc_seed_rng.argtypes = [i64]
        L.orc_resolve_seed.restype = i64
        L.orc_resolve_seed.argtypes = [i64, C.c_uint64, i64]
        L.orc_rng_next_u64.restype = C.c_uint64
        L.orc_rng_next_u64.argtypes = [u64p]
        L.orc_rng_next_f32.restype = C.c_float
        L.orc_rng_next_f32.argtypes = [u64p]
        L.orc_sample_greedy.restype = C.c_int32
        L.orc_sample_greedy.argtypes = [f32p, i64]
        L.orc_token_logprob.restype = C.c_float
        L.orc_token_logprob.argtypes = [f32p, i64, C.c_int32]
        L.orc_logprob_normalizer.argtypes = [f32p, i64, f32p, f32p]
        L.orc_top_k_select.argtypes = [f32p, i64, i64, f32p, i32p]
        L.orc_all_candidates_sorted.argtypes = [f32p, i64, f32p, i32p]
        L.orc_top_n_sigma.argtypes = [f32p, i64, C.c_float, f32p]
        L.orc_top_n_sigma_threshold.argtypes = [f32p, i64, C.c_float, f32p]
        L.orc_sample_candidates.restype = C.c_int32
        L.orc_sample_candidates.argtypes = [u64p, f32p, i32p, i64, C.c_float, C.c_float, C.c_float, C.c_float,
                                            C.c_float, C.c_float, C.c_float, C.c_float, i64, f32p, i32p, i64,
                                            C.POINTER(i64)]
        L.orc_typical_filter.restype = i64
        L.orc_typical_filter.argtypes = [f32p, f32p, i32p, i64, C.c_float, i64, f32p, f32p, i32p]
        L.orc_dynamic_temperature.restype = C.c_float
        L.orc_dynamic_temperature.argtypes = [f32p, i64, i64, i64, C.c_float, C.c_float, C.c_float]
        L.orc_mirostat.restype = C.c_int32
        L.orc_mirostat.argtypes = [C.c_int, u64p, f32p, i64, C.c_float, C.c_float, C.c_float, f32p]
        L.orc_adaptive_p.restype = C.c_int32
        L.orc_adaptive_p.argtypes = [u64p, f32p, i64, C.c_float, C.c_float, f32p, f32p]
        L.orc_sample.restype = C.c_int32
        L.orc_sample.argtypes = [u64p, f32p, i64, C.POINTER(OrcParams), i32p, i64]
        L.orc_apply_repeat_penalty.argtypes = [f32p, i64, i32p, i64, C.c_float, i64, f32p]
        L.orc_apply_presence_frequency.argtypes = [f32p, i64, i32p, i64, C.c_float, C.c_float, f32p]
        L.orc_apply_dry.argtypes = [f32p, i64, i32p, i64, C.c_float, C.c_float, i64, i64, i32p, i32p, i64, f32p]
        L.orc_apply_logit_bias.argtypes = [f32p, i64, i32p, f32p, i64, f32p]
        L.orc_set_eog_tokens.argtypes = [i32p, i64, C.c_int32]
        L.orc_is_eog_token.argtypes = [C.c_int32, C.c_int32]
        L.orc_turn_close_token.restype = C.c_int32
        L.orc_turn_close_token.argtypes = [C.c_int32]
        L.orc_suppress_eog_tokens.argtypes = [f32p, i64, C.c_int32, f32p]
        L.orc_suppress_token.argtypes = [f32p, i64, C.c_int32, f32p]
        L.orc_finish_logits.argtypes = [f32p, i64, C.c_float, C.c_float, f32p]
        L.orc_bytes_to_cps.restype = i64
        L.orc_bytes_to_cps.argtypes = [C.c_char_p, i64, u32p, i64]
        L.orc_is_valid_utf8.argtypes = [C.c_char_p, i64]
        L.orc_grammar_new.restype = C.c_void_p
        L.orc_grammar_new.argtypes = [C.c_char_p]
        L.orc_grammar_free.argtypes = [C.c_void_p]
        L.orc_grammar_accepts.argtypes = [C.c_void_p, C.c_char_p]
        L.orc_grammar_viable.argtypes = [C.c_void_p, C.c_char_p]
        L.orc_json_schema_to_gbnf.restype = i64
        L.orc_json_schema_to_gbnf.argtypes = [C.c_char_p, C.c_char_p, i64]
        L.orc_ngram_draft.restype = i64
        L.orc_ngram_draft.argtypes = [i32p, i64, i64, i64, i64, i32p]
        L.orc_slot_new.restype = C.c_void_p
        L.orc_slot_new.argtypes = [C.POINTER(OrcParams), C.c_uint64, i32p, i64, i32p, i64, i32p, f32p, i64]
        L.orc_slot_free.argtypes = [C.c_void_p]
        L.orc_slot_set_breakers.argtypes = [C.c_void_p, i32p, i32p, i64]
        L.orc_slot_push.argtypes = [C.c_void_p, C.c_int32, C.c_int32]
        L.orc_slot_rng.restype = C.c_uint64
        L.orc_slot_rng.argtypes = [C.c_void_p]
        L.orc_slot_set_grammar.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, u32p, i64, C.c_int32]
        L.orc_slot_restart.argtypes = [C.c_void_p]
        L.orc_slot_step.argtypes = [C.c_void_p, f32p, i64, C.c_int, C.c_int, i32p, f32p, i32p, f32p,
                                    C.POINTER(C.c_int)]
        L.orc_slot_grammar_mask.argtypes = [C.c_void_p, i64, u32p, C.POINTER(C.c_int), C.c_int]
        L.orc_slot_spec_verify.argtypes = [C.c_void_p, f32p, i64, i32p, i64, i32p, i32p]
        L.orc_synth_logits.argtypes = [C.c_int, i64, i64, i64, i64, f32p]
        L.orc_run_c1.argtypes = [i64, i64, i32p, C.POINTER(C.c_double)]
        L.orc_run_c2.argtypes = [i64, i64, C.c_int, i32p, f32p, i32p, f32p, C.POINTER(C.c_double)]
        L.orc_run_c3.argtypes = [i64, i64, C.c_int, i32p, u32p, i32p, C.POINTER(C.c_double)]
        L.orc_run_c4.argtypes = [i64, i64, C.c_int, i32p, f32p, i32p, f32p, C.POINTER(C.c_double)]
        L.orc_run_c5.argtypes = [i64, i64, C.c_int, i32p, i32p, i32p, i32p, C.POINTER(C.c_double)]
        L.orc_c2_row_inputs.argtypes = [i64, C.c_int, i32p, i32p, f32p]
        L.orc_c3_vocab.restype = i64
        L.orc_c3_vocab.argtypes = [i64, C.c_char_p, i64, u32p, i32p]
        L.orc_crc32.restype = C.c_uint32
        L.orc_crc32.argtypes = [C.c_void_p, C.c_size_t]
        L.orc_logprob_sum.restype = C.c_float
        L.orc_logprob_sum.argtypes = [f32p, i64]
        L.orc_sample_candidates_trace.restype = C.c_int32
        L.orc_sample_candidates_trace.argtypes = [C.c_uint64, f32p, i32p, i64, C.c_float, C.c_float, C.c_float, i64,
                                                  f32p, C.POINTER(i64)]
    return L


def fp(a):
    return a.ctypes.data_as(f32p)


def ip(a):
    return a.ctypes.data_as(i32p)


def up(a):
    return a.ctypes.data_as(u32p)


def f32(xs):
    return np.ascontiguousarray(np.asarray(xs, dtype=np.float32))


def i32(xs):
    return np.ascontiguousarray(np.asarray(xs, dtype=np.int32))


def last_error():
    return lib().orc_last_error().decode()


# ---- thin wrappers ----

def seed_rng(seed):
    return lib().orc_seed_rng(seed)


def rng_next_u64(state):
    s = C.c_uint64(state)
    v = lib().orc_rng_next_u64(C.byref(s))
    return v, s.value


def rng_next_f32(state):
    s = C.c_uint64(state)
    v = lib().orc_rng_next_f32(C.byref(s))
    return v, s.value


def sample_greedy(xs):
    a = f32(xs)
    return lib().orc_sample_greedy(fp(a), len(a))


def token_logprob(xs, tok):
    a = f32(xs)
    return lib().orc_token_logprob(fp(a), len(a), tok)


def logprob_normalizer(xs):
    a = f32(xs)
    m, s = C.c_float(), C.c_float()
    lib().orc_logprob_normalizer(fp(a), len(a), C.byref(m), C.byref(s))
    return m.value, s.value


def top_k_select(xs, k):
    a = f32(xs)
    kk = min(k, len(a))
    v = np.zeros(kk, np.float32)
    i = np.zeros(kk, np.int32)
    lib().orc_top_k_select(fp(a), len(a), k, fp(v), ip(i))
    return v, i


def all_candidates_sorted(xs):
    a = f32(xs)
    v = np.zeros(len(a), np.float32)
    i = np.zeros(len(a), np.int32)
    lib().orc_all_candidates_sorted(fp(a), len(a), fp(v), ip(i))
    return v, i


def top_n_sigma(xs, n):
    a = f32(xs)
    o = np.zeros_like(a)
    lib().orc_top_n_sigma(fp(a), len(a), n, fp(o))
    return o


def sample_candidates(state, vals, ids, temperature, dyn_range=0.0, dyn_exp=1.0, typical_p=1.0, top_p=1.0,
                      min_p=0.0, xtc_p=0.0, xtc_t=0.1, min_keep=0, with_probs=False):
    v, i = f32(vals), i32(ids)
    s = C.c_uint64(state)
    cap = max(len(v), 1)
    po = np.zeros(cap, np.float32)
    io = np.zeros(cap, np.int32)
    n = i64(0)
    tok = lib().orc_sample_candidates(C.byref(s), fp(v), ip(i), len(v), temperature, dyn_range, dyn_exp, typical_p,
                                      top_p, min_p, xtc_p, xtc_t, min_keep, fp(po), ip(io), cap, C.byref(n))
    if tok < 0:
        raise RuntimeError(last_error())
    if with_probs:
        return tok, s.value, po[:n.value], io[:n.value]
    return tok, s.value


def sample(state, xs, p, history=()):
    a, h = f32(xs), i32(list(history) or [0])
    s = C.c_uint64(state)
    tok = lib().orc_sample(C.byref(s), fp(a), len(a), C.byref(p), ip(h), len(history))
    if tok < 0:
        raise RuntimeError(last_error())
    return tok, s.value


def apply_repeat_penalty(xs, history, penalty, last_n):
    a, h = f32(xs), i32(list(history) or [0])
    o = np.zeros_like(a)
    lib().orc_apply_repeat_penalty(fp(a), len(a), ip(h), len(history), penalty, last_n, fp(o))
    return o


def apply_presence_frequency(xs, generated, freq, pres):
    a, g = f32(xs), i32(list(generated) or [0])
    o = np.zeros_like(a)
    lib().orc_apply_presence_frequency(fp(a), len(a), ip(g), len(generated), freq, pres, fp(o))
    return o


def apply_dry(xs, history, mult, base, allowed, last_n, breakers):
    a, h = f32(xs), i32(list(history) or [0])
    flat = i32([t for b in breakers for t in b] or [0])
    lens = i32([len(b) for b in breakers] or [0])
    o = np.zeros_like(a)
    lib().orc_apply_dry(fp(a), len(a), ip(h), len(history), mult, base, allowed, last_n, ip(flat), ip(lens),
                        len(breakers), fp(o))
    return o


def apply_logit_bias(xs, bias):
    a = f32(xs)
    ids, vals = i32(list(bias.keys()) or [0]), f32(list(bias.values()) or [0])
    o = np.zeros_like(a)
    lib().orc_apply_logit_bias(fp(a), len(a), ip(ids), fp(vals), len(bias), fp(o))
    return o


def bytes_to_cps(b):
    out = np.zeros(len(b) + 1, np.uint32)
    n = lib().orc_bytes_to_cps(bytes(b), len(b), up(out), len(out))
    return "".join(chr(c) for c in out[:n])


class Grammar:
    def __init__(self, gbnf):
        self.h = lib().orc_grammar_new(gbnf.encode())
        if not self.h:
            raise ValueError(last_error())

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_grammar_free(self.h)

    def accepts(self, text):
        r = lib().orc_grammar_accepts(self.h, text.encode())
        if r < 0:
            raise RuntimeError(last_error())
        return r == 1

    def viable(self, text):
        r = lib().orc_grammar_viable(self.h, text.encode())
        if r < 0:
            raise RuntimeError(last_error())
        return r == 1


def json_schema_to_gbnf(schema):
    buf = C.create_string_buffer(1 << 20)
    n = lib().orc_json_schema_to_gbnf(schema.encode(), buf, len(buf))
    if n < 0:
        raise ValueError(last_error())
    return buf.value.decode()


def ngram_draft(tokens, max_draft, nmax, nmin):
    t = i32(list(tokens) or [0])
    out = np.zeros(max(max_draft, 1), np.int32)
    n = lib().orc_ngram_draft(ip(t), len(tokens), max_draft, nmax, nmin, ip(out))
    return list(out[:n])


def synth_logits(cfg, seed, step, row, V):
    out = np.zeros(V, np.float32)
    lib().orc_synth_logits(cfg, seed, step, row, V, fp(out))
    return out
