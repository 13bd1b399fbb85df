"""Oracle pins for the linear's fused neighbours (CPU).

ModAdd y = a*(1+b)+c and AddMul y = a + b*c come from the reference's opcode
table (core/kernels/ops.cpp:80-82), compiled by NVRTC with its default
--fmad=true, which contracts each multiply-add into one fma.  The oracle
restates them as fma(a, 1+b, c) and fma(b, c, a); these tests check that
against exact rational arithmetic (one rounding of the exact value), and that
the separately rounded forms would fail the same check."""
from fractions import Fraction

import numpy as np
import pytest

import oracle


def rnd_f32(v: Fraction) -> np.float32:
    """Round an exact rational to the nearest fp32 (ties to even)."""
    f = np.float32(float(v))  # float() is correctly rounded to double
    # Correct double rounding: compare the exact value with the neighbours.
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - v),
                                     int(np.float32(c).view(np.uint32)) & 1))
    return np.float32(best)


def sample(n, seed):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(np.float32)
    b = (rng.standard_normal(n) * np.exp2(rng.integers(-24, 2, n))).astype(np.float32)
    c = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(np.float32)
    b[:8] = [-1.0, 0.0, -0.5, 1.0, np.float32(1e-8), np.float32(-1e-8), 3.0, -2.0]
    return a, b, c


def test_mod_add_is_one_rounding_of_exact():
    a, b, c = sample(3000, 1)
    rows, cols = 30, 100
    y = oracle.mod_add(a.reshape(rows, cols), b[:cols], c[:cols]).reshape(-1)
    sep_mismatch = 0
    for i in range(rows * cols):
        k = i % cols
        t = np.float32(np.float32(1.0) + b[k])  # 1 + b is rounded on its own
        want = rnd_f32(Fraction(float(a[i])) * Fraction(float(t)) + Fraction(float(c[k])))
        assert y[i].view(np.uint32) == want.view(np.uint32), i
        sep = np.float32(np.float32(a[i] * t) + c[k])
        sep_mismatch += sep.view(np.uint32) != want.view(np.uint32)
    assert sep_mismatch > 0, "the data does not tell fma from separate rounding"


def test_add_mul_is_one_rounding_of_exact():
    a, b, c = sample(3000, 2)
    rows, cols = 30, 100
    y = oracle.add_mul(a.reshape(rows, cols), b.reshape(rows, cols), c[:cols]).reshape(-1)
    sep_mismatch = 0
    for i in range(rows * cols):
        k = i % cols
        want = rnd_f32(Fraction(float(b[i])) * Fraction(float(c[k])) + Fraction(float(a[i])))
        assert y[i].view(np.uint32) == want.view(np.uint32), i
        sep = np.float32(np.float32(b[i] * c[k]) + a[i])
        sep_mismatch += sep.view(np.uint32) != want.view(np.uint32)
    assert sep_mismatch > 0


def test_mod_add_missing_operands():
    a, b, c = sample(200, 3)
    a = a.reshape(2, 100)
    assert np.array_equal(oracle.mod_add(a, None, None), a)
    # A missing shift is +0: fma(a, t, +0) is a*t rounded once, with -0 * ... + 0 = +0.
    y = oracle.mod_add(a, b[:100], None)
    prod = (a * (np.float32(1) + b[:100])).astype(np.float32)
    assert np.array_equal(y, prod)  # equal as values (+0 == -0)
    assert not np.signbit(y[prod == 0]).any()
    y = oracle.mod_add(a, None, c[:100])
    assert np.array_equal(y, (a + c[:100]).astype(np.float32))


def test_mod_add_b_minus_one_gives_shift():
    """1 + b = 0 exactly: the modulated value is the shift, whatever a is."""
    a = np.array([[3.5, -1e30, 7.0]], np.float32)
    y = oracle.mod_add(a, np.full(3, -1.0, np.float32), np.array([0.25, -2.0, 0.0], np.float32))
    assert np.array_equal(y, np.array([[0.25, -2.0, 0.0]], np.float32))
