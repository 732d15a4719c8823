"""The library's kernels on the CPU: the HIP sources built for the SIMT emulator (tests/cpu/simt) and
checked against the oracle.

No GPU is involved: every GPU thread is a fiber, workgroup barriers and wavefront shuffles/ballots are
rendezvous of those fibers, and LDS is filled with a stale-data pattern before each workgroup. The
emulator aborts on a barrier or wave operation reached from divergent code. Threads run in a random
order between barriers (SIMT_ORDER=rand), so a result that depends on the order of two threads'
unsynchronised accesses shows up as a parity failure. The AddressSanitizer/UBSan build turns any
out-of-bounds device-memory, LDS or private-array access into a failure. This runs the same code as
the GPU parity tests, on the same inputs, at reduced step counts.
"""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SIMT = os.path.join(HERE, "cpu", "simt")


def _build(target):
    r = subprocess.run(["make", "-s", "-C", SIMT, target], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.fixture(scope="module")
def simt_lib():
    _build("all")
    return os.path.join(SIMT, "_build", "libbl_simt.so")


def _run(lib, items, env_extra=None, timeout=600):
    env = dict(os.environ)
    env.update(env_extra or {})
    r = subprocess.run([sys.executable, os.path.join(SIMT, "run_parity.py"), "--lib", lib] + items,
                       capture_output=True, text=True, env=env, timeout=timeout)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    return out


def test_small_cases_random_thread_order(simt_lib):
    out = _run(simt_lib, ["small:0-20:4"], {"SIMT_ORDER": "rand"})
    assert out.count("ok   small case") == 21


def test_coarse_and_ramp_logits(simt_lib):
    """Logits floored to a few integers: greedy and top-k rows whose chunk top-K bound is reached by
    thousands of tied values (top_k 200 takes the radix fallback and cuts the ties in index order).
    Logits on a ramp: the index-order sum crosses a power of two in nearly every group, past the
    normaliser's precomputed critical groups (the rest is walked group by group)."""
    out = _run(simt_lib, ["coarse:0,1,4,5,8,10:4", "ramp:7,8,10:3"], {"SIMT_ORDER": "rand"})
    assert out.count("ok   coarse case") == 6 and out.count("ok   ramp case") == 3


def test_heap_tie_order(simt_lib):
    """Full-vocabulary rows whose draws land on equal values: logits rounded to bfloat16 or to multiples
    of 0.25, floored to a few integers, and bfloat16 N(0, 3^2) rows at V=151936. The token comes from the
    device's simulation of the reference's heap; the oracle runs the heap sort itself."""
    out = _run(simt_lib, ["bf16:2,3,6,9:8", "q4:2,3,6,9:8", "coarse:2,3,6,9:6", "bigties:2"], {"SIMT_ORDER": "rand"})
    assert out.count("ok   bf16 case") == 4 and out.count("ok   q4 case") == 4 and out.count("ok   coarse case") == 4
    assert "ok   bf16 ties at V=151936" in out


def test_mirostat_v2(simt_lib):
    """Mirostat v2 rows over the full-vocabulary rank with planted ties, the running mu carried across
    steps, against the oracle's sample_mirostat_v2."""
    out = _run(simt_lib, ["miro:12"], {"SIMT_ORDER": "rand"})
    assert "ok   mirostat v2 rows" in out


def test_adaptive_p(simt_lib):
    """Adaptive-p rows (src/sampling.br:705-740): the row's normaliser, the transformed values through the
    server stages, their index-order sums and the draw, the running weighted sum carried across steps, against
    the oracle's sample_adaptive_p (V=5003 and 20000)."""
    out = _run(simt_lib, ["adapt:8", "adapt:3:20000"], {"SIMT_ORDER": "rand"})
    assert "ok   adaptive-p rows at V=5003" in out and "ok   adaptive-p rows at V=20000" in out


def test_mirostat_v1(simt_lib):
    """Mirostat v1 rows: the Zipf fit over the merged top-100 keys and its glibc powf estimate, the draw over
    the predicted prefix and the running mu, against the oracle's sample_mirostat_v1 (V=5003 and 20000)."""
    out = _run(simt_lib, ["miro1:10", "miro1:4:20000"], {"SIMT_ORDER": "rand"})
    assert "ok   mirostat v1 rows at V=5003" in out and "ok   mirostat v1 rows at V=20000" in out


def test_unfiltered_candidate_cut(simt_lib):
    """Full-vocabulary rows without top-p or min-p at V=151936: the candidates cut at half an ulp of the
    draw's running sum (six rows, 12 steps; the bfloat16 row's draws on equal values include one whose heap
    subtree reaches past the dense LDS copy, resolved through the deep-position table). Only the head of each
    list is ranked, the tail's ulps of 2^K counted in any order, a draw past the head found through the tail
    buckets' sums; the constructed rows put terms exactly halfway between two multiples of u into the tail (3
    copies, resolved by the running sum's parity; 20 copies, past the split's limit, so the whole list is
    ranked)."""
    out = _run(simt_lib, ["unfilt:12", "halfway:3"], {"SIMT_ORDER": "rev"})
    assert "ok   unfiltered rows at V=151936" in out and "ok   halfway tail terms" in out


def test_full_vocabulary_workloads(simt_lib):
    """Workload 2 (the benchmark step), workload 4 (soft-cap, V=262144, top-64 + 20 logprobs) on 2 rows, the
    bound-rows asynchronous step against the synchronous one, two rows of an odd-length vocabulary in one
    call, and top_k 250 with 256 alternatives."""
    out = _run(simt_lib, ["w2:1", "w4:1:2", "async:1", "pair:3:8:6", "bigk:1"], {"SIMT_ORDER": "rev"})
    assert "ok   workload 2" in out and "ok   workload 4" in out and "ok   asynchronous step" in out
    assert "ok   rows 3 + 8" in out and "ok   large top-k" in out


def test_spec_verify_with_penalties(simt_lib):
    """Speculative rows whose frequency/presence/repeat penalties count the drafts before them (and the window
    entries those drafts evict) against the oracle's spec_verify, over rounds of device commits."""
    out = _run(simt_lib, ["specpen:6", "specpen:1:100"], {"SIMT_ORDER": "rand"})
    assert "ok   speculative rows with penalties, 6 drafts" in out and "ok   speculative rows with penalties, 100 drafts" in out


def test_grammar_masks_and_tokens(simt_lib):
    """The grammar path (GBNF automaton tables, per-token mask walk, masked greedy, on-device commit of
    the reply position) against the oracle's whole-reply re-decode: workload 3 and eight adversarial
    byte-level vocabularies; sampled grammar rows (top-k widening within and past the merged list,
    full-vocabulary rows whose allowed maximum lies far below the row maximum); response_format json_object
    slots (the JSON prefix classifier per candidate, forced end of sequence on complete objects)."""
    out = _run(simt_lib, ["w3:3", "w3schema:3", "grammar:0-7:40", "gsamp:0-9:30", "json:0-3:60"],
               {"SIMT_ORDER": "rand"})
    assert "ok   workload 3\n" in out and "ok   workload 3 via the schema entry point" in out
    assert out.count("ok   grammar case") == 8 and out.count("ok   sampled grammar") == 10
    assert out.count("ok   JSON-object case") == 4


def test_greedy_grammar_ties(simt_lib):
    """Greedy grammar rows whose allowed maximum is shared by several tokens (logits in steps of 0.5), top_k 0
    and 40: the lowest index while the widening levels rank by top_k_select (value desc, index asc), the
    first allowed token of the heap's extraction order (all_candidates_sorted) once a level reaches V.
    Sampled rows (T 0.8) whose draw lands on equal allowed values: the allowed token the heap puts there."""
    out = _run(simt_lib, ["gtie:0-7:20", "gstie:0-7:20"], {"SIMT_ORDER": "rand"})
    assert out.count("ok   grammar ties case") == 16 and out.count("ok   sampled grammar ties case") == 16


def test_top_n_sigma(simt_lib):
    """Top-n-sigma rows (src/sampling.br:376-407): small cases 21-23 (full-vocabulary and top-k ranks) and
    full-size rows at V=151936, the sigma from the row pass's statistics against the oracle's sequential
    float64 sums."""
    out = _run(simt_lib, ["small:21-23:12", "tns:2"], {"SIMT_ORDER": "rand"})
    assert out.count("ok   small case") == 3 and "ok   top-n-sigma rows at V=151936" in out


def test_typical_full_vocabulary(simt_lib):
    """typical_p over full-vocabulary lists at V=3000 (sorted in LDS) and V=5003 (bucket sort): the selection
    order merged from the two monotone runs of distance along the ranked list, the walk to typical_p, the
    compaction and the later stages, against the oracle's typical_filter and slot step."""
    out = _run(simt_lib, ["typical:4:3000", "typical:3:5003"], {"SIMT_ORDER": "rand"})
    assert "ok   typical rows at V=3000" in out and "ok   typical rows at V=5003" in out


def test_dynatemp_exponents(simt_lib):
    """Dynamic temperature with exponents 0.5 and 2.3 (small cases 24-25: a full-vocabulary min-p row and a
    top-k row with post-sampling probabilities), the normalised entropy raised by the device's glibc powf."""
    out = _run(simt_lib, ["small:24-25:12"], {"SIMT_ORDER": "rand"})
    assert out.count("ok   small case") == 2


def test_dry(simt_lib):
    """DRY rows (src/sampling.br:114-171): the device's penalty map, recomputed after every commit and after an
    explicit bl_slot_commit, against the oracle's decode step: one- and two-token breakers in both list orders,
    the exponent cap, a base within 1e-6 of 1, logprobs of the penalised logits (nine cases)."""
    out = _run(simt_lib, ["dry:0-8:10"], {"SIMT_ORDER": "rand"})
    assert out.count("ok   DRY case") == 9


def test_allocation_free_step(simt_lib):
    """bl_sample_rows_noalloc (slot state and workspace carved from its fixed array), twice in a row with
    the second call smaller, equals bl_sample_step over fresh slots with the same parameters and RNG states:
    tokens, logprobs, alternatives and advanced states."""
    out = _run(simt_lib, ["noalloc"], {"SIMT_ORDER": "rand"})
    assert "ok   allocation-free step" in out


def test_small_cases_address_sanitizer():
    _build("asan")
    pre = []
    for rt in ("libasan.so", "libubsan.so"):
        p = subprocess.run(["gcc", f"-print-file-name={rt}"], capture_output=True, text=True).stdout.strip()
        assert os.path.isabs(p) and os.path.exists(p), f"{rt} not found"
        pre.append(p)
    env = {"LD_PRELOAD": " ".join(pre), "ASAN_OPTIONS": "detect_leaks=0", "UBSAN_OPTIONS": "print_stacktrace=1"}
    out = _run(os.path.join(SIMT, "_build", "libbl_simt_asan.so"), ["small:0-20:3", "coarse:1,5:3", "ramp:8:2", "grammar:0-6:20", "q4:2,9:4", "dry:0-8:3",
                                                                   "halfway:1", "typical:1:3000", "gstie:0-1:10"], env)
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out


def test_unready_slot_is_rejected_without_a_launch(simt_lib):
    """bl_slot_commit, bl_slot_rng and bl_slot_status on a slot that bl_slot_reset never set up return
    BL_EPARAM before any kernel runs (slot state is zeroed at creation either way)."""
    import ctypes as C
    L = C.CDLL(simt_lib)
    L.bl_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
    L.bl_slot_commit.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_int32), C.c_int]
    L.bl_slot_rng.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_uint64)]
    L.bl_slot_status.argtypes = [C.c_void_p, C.c_int]
    L.bl_destroy.argtypes = [C.c_void_p]
    L.bl_last_error.restype = C.c_char_p
    h = C.c_void_p()
    assert L.bl_create(0, 4, 4, 4096, C.byref(h)) == 0
    toks = (C.c_int32 * 2)(5, 6)
    assert L.bl_slot_commit(h, 1, toks, 2) == -1
    assert b"not set up" in L.bl_last_error()
    st = C.c_uint64()
    assert L.bl_slot_rng(h, 1, C.byref(st)) == -1
    assert L.bl_slot_status(h, 1) == -1
    L.bl_destroy(h)
