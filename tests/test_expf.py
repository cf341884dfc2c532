"""The router's expf (mgpt_amd/csrc/glibc_expf.hpp) against the C library.

The reference's softmax calls std::exp(float) = glibc expf
(/root/reference/src/main/utils/Tensor.cpp:873); bit-exact routing needs the
GPU to reproduce it.  Checked here on the host build of the same header:
  * its 2^(i/32) table equals an exact integer-arithmetic recomputation;
  * every float in [-104, 0] (all that softmax passes: l - max(l) <= 0) and
    the special values agree bit for bit with the host expf.
The GPU build is compared with the host expf in tests/test_gpu_parity.py.
"""
import concurrent.futures as cf
import os
import re
import struct
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HEADER = os.path.join(ROOT, "mgpt_amd", "csrc", "glibc_expf.hpp")


def iroot(n, k):
    lo, hi = 0, 1 << ((n.bit_length() // k) + 2)
    while lo < hi:
        mid = (lo + hi + 1) // 2
        if mid ** k <= n:
            lo = mid
        else:
            hi = mid - 1
    return lo


def test_exp2_table_is_correctly_rounded():
    text = open(HEADER).read()
    block = text[text.index("#define MGPT_EXP2_TABLE_INIT"):]
    block = block[:block.index("}") + 1]
    table = [int(v, 16) for v in re.findall(r"0x([0-9a-f]+)ull", block)]
    assert len(table) == 32
    for i in range(32):
        g = 64
        r = iroot(1 << (52 * 32 + i + 32 * g), 32)    # floor(2^(52+g+i/32))
        m = (r + (1 << (g - 1))) >> g                  # nearest double mantissa
        bits = (1023 << 52) | (m - (1 << 52))
        assert table[i] == (bits - (i << 47)) & 0xFFFFFFFFFFFFFFFF, i


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("expf") / "expf_check")
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-std=c++17", "-o", exe,
                    os.path.join(HERE, "expf_check.cpp"), "-lm"], check=True)
    return exe


def f2b(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_expf_exhaustive_negative_range(checker):
    # all floats from -0 down to -104: bit patterns 0x80000000 .. f2b(-104)
    lo, hi = 0x80000000, f2b(-104.0)
    parts = 8
    step = (hi - lo + parts) // parts
    ranges = [(lo + i * step, min(hi, lo + (i + 1) * step - 1)) for i in range(parts)]

    def run(r):
        return subprocess.run([checker, f"{r[0]:x}", f"{r[1]:x}"], capture_output=True,
                              text=True)

    with cf.ThreadPoolExecutor(max_workers=parts) as ex:
        results = list(ex.map(run, ranges))
    total = 0
    for r in results:
        assert r.returncode == 0, r.stdout
        total += int(r.stdout.split()[1])
    assert total == hi - lo + 1


def test_expf_special_values(checker):
    for lo, hi in [(f2b(0.0), f2b(0.0)), (0xFF800000, 0xFF800000),   # +0, -inf
                   (0xFFC00000, 0xFFC00010),                           # NaNs
                   (f2b(-104.0), f2b(-104.0) + 100000),                # below -104
                   (f2b(-1e30), f2b(-1e30) + 10)]:
        r = subprocess.run([checker, f"{lo:x}", f"{hi:x}"], capture_output=True, text=True)
        assert r.returncode == 0, r.stdout
