"""The router sigmoid's exp against the C library's expf, on the CPU.

The reference ranks experts on 1/(1 + std::exp(-z)) in float
(moe_router.h:19-21), i.e. on glibc's expf, which is not correctly rounded.
hummingflight_amd/csrc/hf_expf.h restates glibc's algorithm for host and
device; tests/expf_check/check (g++, the same header) compares it with the C
library's expf, and the sigmoid with 1.0f/(1.0f + expf(-x)), on every float.

Pinned independently of the C library too: the 32 table entries are 2^(i/32)
computed here to 60 digits and rounded to double, and a correctly rounded exp
planted in place of the restatement is caught by the same comparison.
"""
import os
import shutil
import struct
import subprocess
from decimal import Decimal, getcontext
from fractions import Fraction

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CHECK_DIR = os.path.join(HERE, "expf_check")
CHECK = os.path.join(CHECK_DIR, "check")


@pytest.fixture(scope="module")
def expf_driver():
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    subprocess.run(["make", "-s", "-B", "-C", CHECK_DIR], check=True)
    return CHECK


def run(expf_driver, *args):
    out = subprocess.run([expf_driver, *args], check=True, capture_output=True, text=True).stdout
    return out.split()


def test_table_is_two_to_the_i_over_32(expf_driver):
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    got = [int(h, 16) for h in run(expf_driver, "table")]
    assert len(got) == 32
    for i, entry in enumerate(got):
        exact = (ln2 * i / 32).exp()
        bits = struct.unpack("<Q", struct.pack("<d", float(Fraction(exact))))[0]
        assert entry == bits - (i << 47), f"table entry {i}"


def test_every_float_matches_the_c_library(expf_driver):
    checked, bad_exp, bad_sig, first = run(expf_driver, "exhaustive")
    assert int(checked) == (1 << 32) - 2 * ((1 << 23) - 1)  # every float but the NaNs
    assert int(bad_exp) == 0 and int(bad_sig) == 0, f"first mismatch at bits 0x{first}"


@pytest.mark.parametrize("lo,hi", [(0x3F000000, 0x3F800000), (0xC0000000, 0xC1000000)])
def test_a_correctly_rounded_exp_is_caught(expf_driver, lo, hi):
    # [0.5, 1) and [-8, -2): the correctly rounded exp and sigmoid differ from
    # glibc's on thousands of these inputs; the restatement on none.
    _, bad_exp, bad_sig, _ = run(expf_driver, "cr", hex(lo), hex(hi))
    assert int(bad_exp) > 1000 and int(bad_sig) > 1000
    _, bad_exp, bad_sig, _ = run(expf_driver, "range", hex(lo), hex(hi))
    assert int(bad_exp) == 0 and int(bad_sig) == 0
