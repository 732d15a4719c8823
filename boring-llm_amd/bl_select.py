"""Python binding of libbl_select.so (the C ABI in include/bl_select.h).

Mirrors the reference's sampler interface for one decode step (src/server.br:939-1037,
src/sampling.br sample/sample_with_probs, SamplingParams of src/model.br:1565-1589): per-request
parameters, a slot per request, and a step that returns token ids, logprobs and alternatives.
Logits are device tensors; this module never falls back to a host implementation — it raises when
the HIP library is missing.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbl_select.so")

BL_OK, BL_EPARAM, BL_EDEVICE, BL_EEMPTY = 0, -1, -2, -3
BL_EGRAMMAR, BL_EGRAMMAR_DEAD, BL_EGRAMMAR_REJECT, BL_EGRAMMAR_AMBIG = -4, -5, -6, -7
BL_EUNSUPPORTED, BL_ETIE, BL_ESCHEMA = -8, -9, -10


class BLError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{msg} (code {code})")
        self.code = code


class Params(C.Structure):
    """bl_params: SamplingParams + server extras; defaults = greedy_params() (src/model.br:1586-1589)."""
    _fields_ = [
        ("temperature", C.c_float), ("dynatemp_range", C.c_float), ("dynatemp_exponent", C.c_float),
        ("top_n_sigma", C.c_float), ("top_k", C.c_int32), ("typical_p", C.c_float), ("top_p", C.c_float),
        ("min_p", C.c_float), ("xtc_probability", C.c_float), ("xtc_threshold", C.c_float),
        ("min_keep", C.c_int32), ("repeat_penalty", C.c_float), ("repeat_last_n", C.c_int32),
        ("dry_multiplier", C.c_float), ("dry_base", C.c_float), ("dry_allowed_length", C.c_int32),
        ("dry_penalty_last_n", C.c_int32), ("frequency_penalty", C.c_float), ("presence_penalty", C.c_float),
        ("logprobs", C.c_int32), ("n_probs", C.c_int32), ("post_sampling_probs", C.c_int32),
        ("ignore_eos", C.c_int32), ("final_softcap", C.c_float), ("logit_mul", C.c_float),
        ("mirostat", C.c_int32), ("mirostat_tau", C.c_float), ("mirostat_eta", C.c_float),
        ("adaptive_target", C.c_float), ("adaptive_decay", C.c_float),
    ]

    def __init__(self, **kw):
        super().__init__()
        lib().bl_params_default(C.byref(self))
        for k, v in kw.items():
            setattr(self, k, v)


EXPORTS = [
    "bl_params_default", "bl_create", "bl_destroy", "bl_last_error", "bl_set_stream", "bl_set_eog",
    "bl_slot_reset", "bl_slot_rng", "bl_slot_commit", "bl_sample_step", "bl_bind_rows", "bl_sample_step_async",
    "bl_spec_verify", "bl_synth_logits", "bl_math_digest", "bl_workload_ids", "bl_workload_bias",
    "bl_workload_drafts", "bl_set_timing", "bl_get_timing", "bl_set_vocab", "bl_slot_grammar", "bl_grammar_mask",
    "bl_workload_c3_vocab", "bl_step_graph_create", "bl_step_graph_launch", "bl_step_graph_destroy",
    "bl_stream_sync", "bl_json_schema_to_gbnf", "bl_slot_schema", "bl_slot_status", "bl_sample_rows_noalloc",
    "bl_resolve_seed", "bl_seed_rng", "bl_slot_dry_breakers", "bl_slot_json_object",
]
NOALLOC_BYTES = 64 << 20
NOALLOC_ROWS = 16

_lib = None


def lib():
    """Load the HIP library; raises if it has not been built (no host fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with boring-llm_amd/build.sh")
        L = C.CDLL(LIB_PATH)
        i32p, f32p, u64p = C.POINTER(C.c_int32), C.POINTER(C.c_float), C.POINTER(C.c_uint64)
        L.bl_params_default.argtypes = [C.c_void_p]
        L.bl_params_default.restype = None
        L.bl_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
        L.bl_destroy.argtypes = [C.c_void_p]
        L.bl_destroy.restype = None
        L.bl_last_error.restype = C.c_char_p
        L.bl_set_stream.argtypes = [C.c_void_p, C.c_void_p]
        L.bl_set_eog.argtypes = [C.c_void_p, C.c_int32, i32p, C.c_int]
        L.bl_slot_reset.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_uint64, i32p, C.c_int, i32p, C.c_int,
                                    i32p, f32p, C.c_int]
        L.bl_slot_dry_breakers.argtypes = [C.c_void_p, C.c_int, i32p, i32p, C.c_int]
        L.bl_slot_json_object.argtypes = [C.c_void_p, C.c_int, C.c_int]
        L.bl_slot_rng.argtypes = [C.c_void_p, C.c_int, u64p]
        L.bl_slot_status.argtypes = [C.c_void_p, C.c_int]
        L.bl_slot_commit.argtypes = [C.c_void_p, C.c_int, i32p, C.c_int]
        L.bl_sample_step.argtypes = [C.c_void_p, i32p, C.c_int, C.c_void_p, C.c_int64, i32p, f32p, i32p, f32p, C.c_int]
        L.bl_bind_rows.argtypes = [C.c_void_p, i32p, C.c_int]
        L.bl_sample_step_async.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                                           C.c_void_p, C.c_void_p, C.c_int]
        L.bl_spec_verify.argtypes = [C.c_void_p, i32p, C.c_int, C.c_int, C.c_void_p, C.c_int64, i32p, i32p, i32p]
        L.bl_step_graph_create.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                                           C.c_void_p, C.c_void_p, C.c_int, C.POINTER(C.c_void_p)]
        L.bl_step_graph_launch.argtypes = [C.c_void_p, C.c_void_p]
        L.bl_step_graph_destroy.argtypes = [C.c_void_p]
        L.bl_stream_sync.argtypes = [C.c_void_p]
        L.bl_synth_logits.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int64, C.c_int64, C.c_int,
                                      C.c_int]
        L.bl_math_digest.argtypes = [C.c_void_p, C.c_int, C.c_uint32, C.c_int, u64p]
        L.bl_resolve_seed.restype = C.c_int64
        L.bl_resolve_seed.argtypes = [C.c_int64, C.c_uint64, C.c_int64]
        L.bl_seed_rng.restype = C.c_uint64
        L.bl_seed_rng.argtypes = [C.c_int64]
        L.bl_set_timing.argtypes = [C.c_void_p, C.c_int]
        L.bl_get_timing.argtypes = [C.c_void_p, C.POINTER(C.c_double), C.POINTER(C.c_int64)]
        L.bl_workload_ids.argtypes = [C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int, C.c_int, i32p]
        L.bl_workload_bias.argtypes = [C.c_int, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, i32p,
                                       f32p]
        L.bl_workload_drafts.argtypes = [C.c_int64, C.c_int64, C.c_int, i32p, C.c_int, C.c_int, i32p]
        L.bl_set_vocab.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        L.bl_slot_grammar.argtypes = [C.c_void_p, C.c_int, C.c_char_p, C.c_size_t]
        L.bl_json_schema_to_gbnf.argtypes = [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t,
                                             C.POINTER(C.c_size_t)]
        L.bl_slot_schema.argtypes = [C.c_void_p, C.c_int, C.c_char_p, C.c_size_t]
        L.bl_grammar_mask.argtypes = [C.c_void_p, C.c_int, C.c_void_p, i32p]
        L.bl_workload_c3_vocab.argtypes = [C.c_int64, C.c_int, C.c_void_p, C.c_size_t, C.c_void_p, i32p]
        L.bl_sample_rows_noalloc.argtypes = [C.c_int, C.c_void_p, C.c_void_p, u64p, C.c_int, C.c_void_p, C.c_int64,
                                             C.c_int, i32p, f32p, i32p, f32p, C.c_int]
        _lib = L
    return _lib


def _arr(ctype, xs):
    xs = list(xs)
    return (ctype * max(len(xs), 1))(*xs), len(xs)


def _check(rc):
    if rc != BL_OK:
        raise BLError(rc, lib().bl_last_error().decode())


class Context:
    """One device context (bl_create): `max_slots` requests, up to `max_rows` rows per call."""

    def __init__(self, vocab, max_slots=8, max_rows=8, device=0):
        self.vocab = vocab
        self.h = C.c_void_p()
        _check(lib().bl_create(device, max_slots, max_rows, vocab, C.byref(self.h)))

    def close(self):
        if self.h:
            lib().bl_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream_ptr):
        """Order the context's work on an existing HIP stream (0 = the context's own)."""
        _check(lib().bl_set_stream(self.h, C.c_void_p(stream_ptr)))

    def set_timing(self, enable):
        _check(lib().bl_set_timing(self.h, 1 if enable else 0))

    def get_timing(self):
        """(ms per step of the row pass, exponent pass, selection kernel; timed steps)"""
        ms = (C.c_double * 3)()
        n = C.c_int64()
        _check(lib().bl_get_timing(self.h, ms, C.byref(n)))
        k = max(n.value, 1)
        return [ms[i] / k for i in range(3)], n.value

    def set_eog(self, eos_id, eog_ids=()):
        a, n = _arr(C.c_int32, eog_ids)
        _check(lib().bl_set_eog(self.h, eos_id, a, n))

    def slot_reset(self, slot, params, rng_state, history=(), reply=(), bias=None):
        h, nh = _arr(C.c_int32, history)
        r, nr = _arr(C.c_int32, reply)
        bias = bias or {}
        bi, nb = _arr(C.c_int32, bias.keys())
        bv, _ = _arr(C.c_float, bias.values())
        _check(lib().bl_slot_reset(self.h, slot, C.byref(params), C.c_uint64(rng_state), h, nh, r, nr, bi, bv, nb))

    def slot_dry_breakers(self, slot, breakers):
        """The request's tokenised DRY sequence breakers, in order (bl_slot_dry_breakers)."""
        flat = [t for b in breakers for t in b]
        a, _ = _arr(C.c_int32, flat)
        ln, n = _arr(C.c_int32, [len(b) for b in breakers])
        _check(lib().bl_slot_dry_breakers(self.h, slot, a, ln, n))

    def slot_json_object(self, slot, on=True):
        """response_format json_object on the slot (bl_slot_json_object)."""
        _check(lib().bl_slot_json_object(self.h, slot, 1 if on else 0))

    def slot_rng(self, slot):
        s = C.c_uint64()
        _check(lib().bl_slot_rng(self.h, slot, C.byref(s)))
        return s.value

    def slot_status(self, slot):
        """Raises BLError with the failure of the slot's rows since the last call (bl_slot_status)."""
        _check(lib().bl_slot_status(self.h, slot))

    def commit(self, slot, toks):
        a, n = _arr(C.c_int32, toks)
        _check(lib().bl_slot_commit(self.h, slot, a, n))

    def sample_step(self, slots, d_logits_ptr, ld, top_stride=0):
        """Synchronous step; returns (tokens, logprobs, top_ids, top_logprobs) as Python lists."""
        B = len(slots)
        s, _ = _arr(C.c_int32, slots)
        tok = (C.c_int32 * B)()
        lp = (C.c_float * B)()
        ti = (C.c_int32 * max(B * top_stride, 1))()
        tl = (C.c_float * max(B * top_stride, 1))()
        _check(lib().bl_sample_step(self.h, s, B, C.c_void_p(d_logits_ptr), ld, tok, lp, ti, tl, top_stride))
        tops = [list(ti[b * top_stride:(b + 1) * top_stride]) for b in range(B)]
        tlps = [list(tl[b * top_stride:(b + 1) * top_stride]) for b in range(B)]
        return list(tok), list(lp), tops, tlps

    def bind_rows(self, slots):
        s, n = _arr(C.c_int32, slots)
        _check(lib().bl_bind_rows(self.h, s, n))

    def sample_step_async(self, B, d_logits_ptr, ld, d_tok, d_lp=0, d_top_ids=0, d_top_lp=0, top_stride=0):
        _check(lib().bl_sample_step_async(self.h, B, C.c_void_p(d_logits_ptr), ld, C.c_void_p(d_tok),
                                          C.c_void_p(d_lp), C.c_void_p(d_top_ids), C.c_void_p(d_top_lp), top_stride))

    def step_graph(self, B, d_logits_ptr, ld, d_tok, d_lp=0, d_top_ids=0, d_top_lp=0, top_stride=0):
        """One bound-rows step captured into a HIP graph; returns its handle (bl_step_graph_create)."""
        g = C.c_void_p()
        _check(lib().bl_step_graph_create(self.h, B, C.c_void_p(d_logits_ptr), ld, C.c_void_p(d_tok), C.c_void_p(d_lp),
                                          C.c_void_p(d_top_ids), C.c_void_p(d_top_lp), top_stride, C.byref(g)))
        return g

    def graph_launch(self, g):
        _check(lib().bl_step_graph_launch(self.h, g))

    @staticmethod
    def graph_destroy(g):
        _check(lib().bl_step_graph_destroy(g))

    def sync(self):
        _check(lib().bl_stream_sync(self.h))

    def spec_verify(self, slots, k, d_rows_ptr, ld, drafts):
        B = len(slots)
        s, _ = _arr(C.c_int32, slots)
        d, _ = _arr(C.c_int32, drafts)
        tok = (C.c_int32 * (B * (k + 1)))()
        acc = (C.c_int32 * B)()
        _check(lib().bl_spec_verify(self.h, s, B, k, C.c_void_p(d_rows_ptr), ld, d, tok, acc))
        return list(tok), list(acc)

    def set_vocab(self, blob, offsets):
        """Token pieces: `blob` (bytes or uint8 array) and `offsets` (len vocab + 1, uint32)."""
        b = bytes(blob)
        o = (C.c_uint32 * len(offsets))(*[int(x) for x in offsets])
        bb = C.create_string_buffer(b, max(len(b), 1))
        _check(lib().bl_set_vocab(self.h, bb, o, len(offsets) - 1))

    def slot_grammar(self, slot, gbnf):
        """Attach a GBNF grammar to `slot` (None detaches)."""
        if gbnf is None:
            _check(lib().bl_slot_grammar(self.h, slot, None, 0))
        else:
            t = gbnf.encode() if isinstance(gbnf, str) else bytes(gbnf)
            _check(lib().bl_slot_grammar(self.h, slot, t, len(t)))

    def slot_schema(self, slot, schema):
        """Attach the grammar of a JSON schema (its JSON text) to `slot` (None detaches)."""
        if schema is None:
            _check(lib().bl_slot_schema(self.h, slot, None, 0))
        else:
            t = schema.encode() if isinstance(schema, str) else bytes(schema)
            _check(lib().bl_slot_schema(self.h, slot, t, len(t)))

    def grammar_mask(self, slot, d_mask_ptr):
        """Writes ceil(V/32) mask words to device memory; returns forced_eos."""
        f = C.c_int32()
        _check(lib().bl_grammar_mask(self.h, slot, C.c_void_p(d_mask_ptr), C.byref(f)))
        return bool(f.value)

    def synth_logits(self, d_out_ptr, ld, cfg, seed, step, rows, vocab):
        _check(lib().bl_synth_logits(self.h, C.c_void_p(d_out_ptr), ld, cfg, seed, step, rows, vocab))

    def math_digest(self, fn, first_block, n_blocks):
        out = (C.c_uint64 * n_blocks)()
        _check(lib().bl_math_digest(self.h, fn, first_block, n_blocks, out))
        return list(out)


def sample_rows_noalloc(params, rng_states, d_logits_ptr, ld, vocab, top_stride=0, device=0, stream=0):
    """bl_sample_rows_noalloc: one stateless step of len(params) rows, no device allocation. Returns
    (tokens, logprobs, top_ids, top_logprobs, advanced RNG states) as Python lists."""
    B = len(params)
    ps = (Params * max(B, 1))(*params)
    rng = (C.c_uint64 * max(B, 1))(*rng_states)
    tok = (C.c_int32 * max(B, 1))()
    lp = (C.c_float * max(B, 1))()
    ti = (C.c_int32 * max(B * top_stride, 1))()
    tl = (C.c_float * max(B * top_stride, 1))()
    _check(lib().bl_sample_rows_noalloc(device, C.c_void_p(stream), ps, rng, B, C.c_void_p(d_logits_ptr), ld, vocab,
                                        tok, lp, ti, tl, top_stride))
    tops = [list(ti[b * top_stride:(b + 1) * top_stride]) for b in range(B)]
    tlps = [list(tl[b * top_stride:(b + 1) * top_stride]) for b in range(B)]
    return list(tok[:B]), list(lp[:B]), tops, tlps, list(rng[:B])


def workload_ids(kind, cfg, seed, row, n, vocab):
    out = (C.c_int32 * max(n, 1))()
    _check(lib().bl_workload_ids(kind, cfg, seed, row, n, vocab, out))
    return list(out[:n])


def workload_bias(cfg, seed, row, n, vocab, lo, hi):
    ids = (C.c_int32 * max(n, 1))()
    vals = (C.c_float * max(n, 1))()
    _check(lib().bl_workload_bias(cfg, seed, row, n, vocab, lo, hi, ids, vals))
    return dict(zip(ids[:n], vals[:n]))


def workload_drafts(seed, step, seq, argmax, vocab):
    k = len(argmax)
    a, _ = _arr(C.c_int32, argmax)
    out = (C.c_int32 * max(k, 1))()
    _check(lib().bl_workload_drafts(seed, step, seq, a, k, vocab, out))
    return list(out[:k])


def workload_c3_vocab(seed, vocab):
    """(blob bytes, offsets list, eos_id) of the workload-3 synthetic vocabulary."""
    cap = vocab * 64 + 4096
    blob = (C.c_uint8 * cap)()
    off = (C.c_uint32 * (vocab + 1))()
    eos = C.c_int32()
    n = lib().bl_workload_c3_vocab(seed, vocab, blob, cap, off, C.byref(eos))
    if n < 0:
        _check(n)
    return bytes(blob[:n]), list(off), eos.value


def seed_rng(seed):
    """seed_rng of src/sampling.br:35-40 (the initial xorshift state for a request seed), bl_seed_rng."""
    return int(lib().bl_seed_rng(seed))


def resolve_seed(requested, entropy, request_counter):
    """resolve_seed of src/sampling.br:21-33 (a negative request seed chosen from entropy and the request
    counter), bl_resolve_seed."""
    return int(lib().bl_resolve_seed(requested, entropy & 0xFFFFFFFFFFFFFFFF, request_counter))


def json_schema_to_gbnf(schema):
    """GBNF text of a JSON schema (json_schema_to_gbnf, src/schema_grammar.br:313-337); raises BLError
    (code BL_ESCHEMA) with the reference's message."""
    t = schema.encode() if isinstance(schema, str) else bytes(schema)
    n = C.c_size_t(0)
    _check(lib().bl_json_schema_to_gbnf(t, len(t), None, 0, C.byref(n)))
    buf = C.create_string_buffer(n.value + 1)
    _check(lib().bl_json_schema_to_gbnf(t, len(t), buf, n.value + 1, None))
    return buf.raw[:n.value].decode()
