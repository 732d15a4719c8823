"""The C-ABI library loads and exports every function include/*.h declares (no GPU needed: no
compute call is made)."""
import ctypes
import glob
import os
import re

import bl_select as BL

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(bl_\w+)\s*\(", text, flags=re.M))
    return names


def test_header_declares_the_boundary():
    names = declared()
    for must in ("bl_create", "bl_slot_reset", "bl_sample_step", "bl_spec_verify", "bl_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(BL.LIB_PATH)
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(BL.EXPORTS) <= declared()


def test_integration_extern_block_names_every_export():
    """INTEGRATION.md's Rust `extern "C"` block declares every function of include/*.h, and nothing else."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    start = text.index('extern "C" {')
    block = text[start:text.index("\n}\n", start)]
    named = set(re.findall(r"pub fn (bl_\w+)\s*\(", block))
    assert declared() - named == set(), sorted(declared() - named)
    assert named - declared() == set(), sorted(named - declared())


def test_params_layout_matches_header():
    # bl_params is 30 4-byte fields in the header's order
    assert ctypes.sizeof(BL.Params) == 30 * 4
    p = BL.Params()
    assert p.temperature == 0.0 and p.top_p == 1.0 and p.repeat_last_n == 64 and p.dynatemp_exponent == 1.0
    assert p.mirostat == 0 and p.mirostat_tau == 5.0 and abs(p.mirostat_eta - 0.1) < 1e-7
    assert p.adaptive_target == -1.0 and abs(p.adaptive_decay - 0.9) < 1e-7


def test_seed_fold():
    # seed_rng (src/sampling.br:35-40), through the library's host entry point
    assert BL.seed_rng(0) == 88172645463325252
    assert BL.seed_rng(5) == 5 ^ 88172645463325252
    assert BL.seed_rng(-3) == ((-3) & (2 ** 64 - 1)) ^ 88172645463325252


def test_resolve_seed_equals_the_oracle():
    """bl_resolve_seed against the oracle's resolve_seed (src/sampling.br:21-33) on random requests, and the
    xorshift round written out with Python integers."""
    import numpy as np
    import _oracle as O
    L = O.lib()
    L.orc_resolve_seed.restype = ctypes.c_int64
    L.orc_resolve_seed.argtypes = [ctypes.c_int64, ctypes.c_uint64, ctypes.c_int64]
    M = 2 ** 64 - 1
    rng = np.random.default_rng(3)
    for k in range(2000):
        req = int(rng.integers(-5, 5)) if k % 2 else -1
        ent = int(rng.integers(0, 2 ** 63)) * 2 + (k & 1)
        cnt = int(rng.integers(0, 2 ** 40)) if k % 3 else k
        got = BL.resolve_seed(req, ent, cnt)
        assert got == L.orc_resolve_seed(req, ent, cnt)
        if req < 0:
            x = ent ^ ((cnt << 32) & M) ^ cnt
            x ^= (x << 13) & M
            x ^= x >> 7
            x ^= (x << 17) & M
            assert got == ((x & 0x7FFFFFFF) or 1)
        else:
            assert got == req
    # the mixed value 0 maps to 1
    assert BL.resolve_seed(-1, 0, 0) == 1


def test_workload_generators_are_deterministic():
    a = BL.workload_ids(1, 2, 2, 0, 64, 151936)
    assert a == BL.workload_ids(1, 2, 2, 0, 64, 151936) and min(a) >= 0 and max(a) < 151936
    b = BL.workload_bias(2, 2, 0, 300, 151936, -100.0, 100.0)
    assert len(b) == 300 and all(-100.0 <= v < 100.0 for v in b.values())
