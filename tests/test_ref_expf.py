"""The strict mode's expf (csrc/ref_expf.h) against the C library's own expf, on the CPU.

The reference's softmax (qwen.c:346-352, runq.c:409-428) and SiLU (qwen.c:558-562, runq.c:589-596) call the C
library's expf.  glibc's expf is not correctly rounded (a correctly rounded exp differs from it in about 1 of
13,000 inputs), so the strict mode restates glibc's published algorithm; these tests pin that restatement:
  - the source compiled for the host (mvh_ref_expf_host, the same header the device kernels include) against
    the oracle's or_expf, which calls the C library, bit for bit over a strided sample of all 2^32 patterns;
  - its table against 2^(i/32) computed in 60-digit decimal arithmetic (the mathematics, not a library);
  - closed forms: expf(0) = 1, -inf -> 0, +inf -> inf, nan -> nan, overflow and underflow thresholds.
The device evaluation is held to the same function in tests/test_gpu_strict.py."""
import os
import re
from decimal import Decimal, getcontext

import numpy as np

from helpers import PKG_DIR, oracle, pkg, ptr


def libc_expf(x):
    L = oracle()
    y = np.empty_like(x)
    L.or_expf(ptr(x), x.size, ptr(y))
    return y


def same_bits(a, b):
    both_nan = np.isnan(a) & np.isnan(b)
    return (a.view(np.uint32) == b.view(np.uint32)) | both_nan


def test_restatement_matches_the_c_library_over_all_bit_patterns_strided():
    P = pkg()
    stride = 263  # prime: every exponent and low-mantissa residue is visited
    bad = 0
    for start in range(0, 1 << 32, 1 << 28):
        u = np.arange(start, min(start + (1 << 28), 1 << 32), stride, dtype=np.uint64).astype(np.uint32)
        x = u.view(np.float32)
        bad += int((~same_bits(P.ref_expf(x, host=True), libc_expf(x))).sum())
    assert bad == 0


def test_restatement_matches_the_c_library_on_softmax_and_silu_ranges():
    """every float in [-24, 0] with its last 6 mantissa bits fixed, and dense samples around the special
    thresholds (the ranges softmax and SiLU arguments fall in)"""
    P = pkg()
    lo, hi = np.float32(-24.0).view(np.uint32), np.float32(-0.0).view(np.uint32)
    u = np.arange(hi, lo + 1, 61, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([u.view(np.float32), np.linspace(-104.5, -86, 200001, dtype=np.float32),
                        np.linspace(86, 89, 20001, dtype=np.float32)])
    assert same_bits(P.ref_expf(x, host=True), libc_expf(x)).all()


def test_table_is_two_to_the_i_over_32():
    src = open(os.path.join(PKG_DIR, "csrc", "ref_expf.h")).read()
    tab = [int(h, 16) for h in re.findall(r"0x([0-9a-f]{16})ull", src)]
    assert len(tab) == 32
    getcontext().prec = 60
    for i, t in enumerate(tab):
        v = float(Decimal(2) ** (Decimal(i) / Decimal(32)))  # correctly rounded from 60 digits
        assert t + (i << 47) == int(np.float64(v).view(np.uint64)), i


def test_closed_forms():
    P = pkg()
    x = np.array([0.0, -0.0, -np.inf, np.inf, np.nan, 1.0, 89.0, -104.0, 88.72283, -103.97208], np.float32)
    y = P.ref_expf(x, host=True)
    assert y[0] == 1.0 and y[1] == 1.0 and y[2] == 0.0 and y[3] == np.inf and np.isnan(y[4])
    assert y[5] == np.float32(np.e)
    assert y[6] == np.inf and y[7] == 0.0
    assert same_bits(y, libc_expf(x)).all()
