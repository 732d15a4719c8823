"""CPU checks of the device arithmetic headers (boring-llm_amd/csrc/bl_math.h, bl_exact.h):
the exp2 table recomputed from high-precision arithmetic; the exact sequential-sum automaton and the
glibc-identical expf/tanhf (on a strided sample here; exhaustively on the GPU against
tests/golden/math_digest.bin) checked by tests/cpu/check_exact.cpp against the host glibc."""
import os
import re
import struct
import subprocess
from decimal import Decimal, getcontext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_exp2_table_is_derived():
    getcontext().prec = 60
    text = open(os.path.join(ROOT, "boring-llm_amd", "csrc", "bl_math.h")).read()
    tab = [int(x, 16) for x in re.findall(r"0x([0-9a-f]{16})ull", text)[:32]]
    ln2 = Decimal(2).ln()
    for i in range(32):
        v = float((ln2 * i / 32).exp())
        bits = struct.unpack("<Q", struct.pack("<d", v))[0]
        assert tab[i] == (bits - (i << 47)) & (2 ** 64 - 1), i


def test_exact_sum_and_math_on_cpu(tmp_path):
    exe = str(tmp_path / "check_exact")
    subprocess.check_call(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", exe,
                           os.path.join(ROOT, "tests", "cpu", "check_exact.cpp"), "-lm"])
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "exact-sum mismatches: 0" in out.stdout
