"""The JSON-object classifier of the device (boring-llm_amd/csrc/bl_jwalk.h, built for the host) against the
oracle's restatement of json_object_prefix_state (src/json.br:394-426): random replies of JSON fragments cut
into byte tokens at arbitrary points (inside strings, escapes, numbers, literals and UTF-8 sequences), each
candidate's allowed flag (the state after decode(reply ++ T) viable) and the committed reply's completeness."""
import ctypes
import os
import random
import subprocess

import _oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib(tmp_path):
    so = str(tmp_path / "libjwalk.so")
    subprocess.check_call(["g++", "-O1", "-std=c++17", "-shared", "-fPIC", "-o", so,
                           os.path.join(ROOT, "tests", "cpu", "jwalk_capi.cpp")])
    L = ctypes.CDLL(so)
    L.jw_check.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32), ctypes.c_int,
                           ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    return L


FRAGS = ['{', '}', '[', ']', ':', ',', ' ', '\n', '"', '"k"', '"v\\n"', '\\u00e9', '\\u12', '\\q', 'true', 'tr',
         'fals', 'null', 'nul', '-', '0', '01', '12', '3.', '.5', '1e', 'e+', '5E-2', '-0.25', 'é', '€', '\U0001F600',
         '\x01', 'x', '{"a":', '[1,2]', '{"b":{"c":[true,null,"s"]}}', '  ', '\t', '"a\x01b"', '"\x1f', '"\t"']


def test_json_walk_equals_oracle(tmp_path):
    L = _lib(tmp_path)
    Oc = O.lib()
    Oc.orc_json_prefix_state.restype = ctypes.c_int
    Oc.orc_json_prefix_state.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_int64, ctypes.c_int]
    rng = random.Random(11)
    bad, checked = [], 0

    def ostate(b):
        # bytes_to_str of the reference is the oracle's; Python's 'replace' decoder differs on some invalid
        # sequences, so the oracle decodes
        cps = (ctypes.c_uint32 * max(len(b), 1))()
        n = Oc.orc_bytes_to_cps(b, len(b), cps, len(b))
        return Oc.orc_json_prefix_state(cps, n, 1)

    Oc.orc_bytes_to_cps.restype = ctypes.c_int64
    Oc.orc_bytes_to_cps.argtypes = [ctypes.c_char_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_uint32), ctypes.c_int64]
    for case in range(400):
        if case % 3 == 0:  # mostly valid documents, cut anywhere
            text = '{"name": "café ' + rng.choice(["x", "€", "\U0001F600"]) + '", "n": [1, -2.5e+3, true, null, {"k": 0}]}'
            text = text[:rng.randrange(len(text) + 1)] + rng.choice(["", " ", "}", "]", ",", "x"])
        else:
            text = "".join(rng.choice(FRAGS) for _ in range(rng.randrange(1, 12)))
            if rng.random() < 0.7:
                text = rng.choice(["{", " {", '{"a": '] ) + text
        b = text.encode("utf-8")
        if rng.random() < 0.2 and b:  # a stray byte
            i = rng.randrange(len(b) + 1)
            b = b[:i] + bytes([rng.choice([0x80, 0xC3, 0xE2, 0xF0, 0xFF])]) + b[i:]
        cuts = sorted(rng.sample(range(1, len(b) + 1), min(len(b), rng.randrange(1, 6)))) if b else []
        toks, prev = [], 0
        for c in cuts:
            toks.append(b[prev:c])
            prev = c
        if prev < len(b):
            toks.append(b[prev:])
        for k in range(1, len(toks) + 1):
            lens = (ctypes.c_int32 * k)(*[len(t) for t in toks[:k]])
            comp, dead = ctypes.c_int(), ctypes.c_int()
            got = L.jw_check(b"".join(toks[:k]), lens, k, ctypes.byref(comp), ctypes.byref(dead))
            want = 1 if ostate(b"".join(toks[:k])) >= 0 else 0
            before = ostate(b"".join(toks[:k - 1]))
            checked += 1
            if got != want or comp.value != (1 if before == 1 else 0):
                bad.append((b, [len(t) for t in toks[:k]], got, want, comp.value, before))
    assert checked > 1000
    assert bad == [], bad[:3]
