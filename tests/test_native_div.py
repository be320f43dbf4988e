"""CPU: the kernels' correctly rounded division (ns::div_rn, csrc/ns_device.h) against
IEEE float division, bit for bit.

The kernels divide by a row-uniform divisor t (the temperature, sampler.py:51, and the
repetition penalty, sampler.py:37) as q0 = RN(x * RN(1/t)), then one fma-based
correction, with IEEE division where the correction theorem's conditions fail.
tests/native/div_rn_check.c runs that formula on the CPU with C's fmaf over every binade
of the float range (a stride of mantissas in each, every mantissa in three, subnormal
bit patterns, zeros, infinities, NaN) for 28 fixed divisors (the workloads' penalties and
temperatures, the temperature clamp, divisors next to the range limits) and random ones,
both signs, and compares with x / t.  The earlier range rule, which tested |q0| alone,
must fail the same check (its remainder is inexact for |x| < 2^-100 under divisors
below 1): the check can tell the two apart.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "native", "div_rn_check.c")
BUILD = os.path.join(HERE, "native", "build")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div_rn_matches_ieee_division():
    os.makedirs(BUILD, exist_ok=True)
    exe = os.path.join(BUILD, "div_rn_check")
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-o", exe, SRC, "-lm"], check=True)
    res = subprocess.run([exe, "4"], capture_output=True, text=True, timeout=300)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches 0" in res.stdout
    old = subprocess.run([exe, "0", "old"], capture_output=True, text=True, timeout=300)
    print(old.stdout)
    assert old.returncode == 1 and "mismatch t=" in old.stdout, old.stdout + old.stderr


def test_uniform_row_probability_single_rounding():
    """The NaN guard's uniform row (sampler.py:77-80) gives every token torch's float32 1/V,
    the float64 quotient rounded to float32.  The kernels divide in float32 (ns::uniform_q):
    the two roundings agree for every vocabulary size up to the ABI's limit of 2^18."""
    import numpy as np

    v = np.arange(1, 2**18 + 1, dtype=np.float64)
    twice = (1.0 / v).astype(np.float32)
    once = np.float32(1.0) / v.astype(np.float32)
    assert np.array_equal(twice.view(np.uint32), once.view(np.uint32))


def test_fixed_point_mass_halves():
    """The wide path's masses trunc(e * 2^44) for float32 e in [0, 1] (ns::fx44): formed
    as hi = trunc(e * 2^12) and lo = trunc((e * 2^12 - hi) * 2^32) in float32, which are
    exact operations, so hi * 2^32 + lo is the float64 truncation.  Checked here on every
    257th float32 bit pattern of [0, 1] (subnormals, every binade) and on its ends; the
    whole range (about 1.07e9 patterns) gives the same result."""
    import numpy as np

    b = np.concatenate([np.arange(0, 0x3F800000, 257, dtype=np.uint32),
                        np.array([0, 1, 0x007FFFFF, 0x00800000, 0x3F7FFFFF, 0x3F800000], dtype=np.uint32)])
    e = b.view(np.float32)
    ref = np.floor(e.astype(np.float64) * 2.0**44).astype(np.uint64)
    x = (e * np.float32(4096.0)).astype(np.float32)
    hi = x.astype(np.uint32)
    lo = ((x - hi.astype(np.float32)) * np.float32(4294967296.0)).astype(np.float32).astype(np.uint64)
    got = (hi.astype(np.uint64) << np.uint64(32)) | lo
    assert np.array_equal(got, ref)
