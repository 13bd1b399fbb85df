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


# ---------------------------------------------------------------- activations
def act_sample(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    x[:12] = [0.0, -0.0, 1.0, -1.0, 10.0, -10.0, 30.0, -30.0, 1e-3, -1e-3, 5.5, -5.5]
    return x


def test_gelu_tanh_oracle_against_torch_and_float64():
    """GELU-tanh (core/kernels/ops.cpp:83-89) against torch's own tanh-GELU and
    the float64 value of the same formula."""
    torch = pytest.importorskip("torch")
    x = act_sample(20000, 3)
    y = oracle.gelu_tanh(x)
    tref = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    np.testing.assert_allclose(y, tref, rtol=1e-5, atol=1e-6)
    xd = x.astype(np.float64)
    exact = 0.5 * xd * (1 + np.tanh(np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3)))
    # 1 + tanh(t) cancels for t << 0, so the fp32 formula is good to ~1 ulp of |x|/2 there.
    np.testing.assert_allclose(y, exact, rtol=2e-6, atol=2e-7 * np.abs(xd).max())


def test_gelu_tanh_oracle_limits():
    x = np.array([0.0, 10.0, 30.0, 1e4, -10.0, -30.0, -1e4], dtype=np.float32)
    y = oracle.gelu_tanh(x)
    assert y[0] == 0.0
    # tanh(t) rounds to 1 for t > ~9: gelu(x) = 0.5 x * 2 = x exactly
    assert np.array_equal(y[1:4], x[1:4])
    # and to -1 for t < -9: 1 + tanh = 0, so gelu(x) = 0
    assert np.all(y[4:] == 0.0)
    # odd part: gelu(x) - gelu(-x) = x exactly in real arithmetic
    z = act_sample(5000, 4)
    d = oracle.gelu_tanh(z).astype(np.float64) - oracle.gelu_tanh(-z).astype(np.float64)
    np.testing.assert_allclose(d, z, rtol=1e-6, atol=1e-6)


def test_silu_gate_oracle_against_torch_and_float64():
    """silu(g) * v over [gate | value] rows (core/kernels/conv3d_causal.cpp:997-1013)."""
    torch = pytest.importorskip("torch")
    rows, cols = 40, 500
    gx = act_sample(rows * 2 * cols, 5).reshape(rows, 2 * cols)
    out = oracle.silu_gate(gx)
    g, v = gx[:, :cols], gx[:, cols:]
    tref = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(v)).numpy()
    np.testing.assert_allclose(out, tref, rtol=1e-6, atol=1e-30)
    gd, vd = g.astype(np.float64), v.astype(np.float64)
    np.testing.assert_allclose(out, gd / (1 + np.exp(-gd)) * vd, rtol=1e-6, atol=1e-30)
    # the pairing is per row: row r's value half, not the flat next block
    assert not np.allclose(out[1], (g[1] / (1 + np.exp(-g[1].astype(np.float64)))) * gx[0, cols:])


def test_silu_gate_oracle_limits():
    g = np.array([0.0, 20.0, 100.0, -100.0, -200.0], dtype=np.float32)
    v = np.array([3.0, 1.5, -2.0, 7.0, -7.0], dtype=np.float32)
    out = oracle.silu_gate(np.concatenate([g, v])[None, :])[0]
    assert out[0] == 0.0
    # exp(-g) < 2^-24: 1 + exp(-g) rounds to 1, so silu(g) * v = g * v exactly
    assert out[1] == np.float32(20.0 * 1.5) and out[2] == np.float32(-200.0)
    # exp(-g) overflows: g / inf = 0
    assert out[3] == 0.0 and out[4] == 0.0
