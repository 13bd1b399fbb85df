"""Pins for the oracle's A1 (convrot) and A2 (per-row quantiser).

A1 is pinned by its closed form: H = (J - 2R)^{(x)4} / 16 built as a dense
256x256 matrix from its definition (row d of H4 is +1 except -1 at column
3 - d), symmetric and orthonormal, so H H = I.  Integer inputs make every
butterfly step exact in fp32, so the oracle must equal H x exactly; a sign,
index-order or normalisation slip (for instance the 2I - J matrix the
reference's header names, core/host/quant.hpp:5) fails that check.
A2 is pinned by the textbook rounding rules on every near-tie fp32 value, by
crafted ties, and by the row-amax invariants.  Both are also compared bit for
bit with the reference's own core/host/quant.cpp built from its sources
(oracle/_ref), when that build is present.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle as O


def H4(kind="J-2R"):
    J = np.ones((4, 4))
    R = np.fliplr(np.eye(4))
    return J - 2 * R if kind == "J-2R" else 2 * np.eye(4) - J


def dense_H(kind="J-2R"):
    h = H4(kind)
    H = h
    for _ in range(3):
        H = np.kron(h, H)  # digit 0 (stride 1) is the fastest-varying index
    return H / 16.0


def test_dense_matrix_properties():
    H = dense_H()
    assert np.allclose(H, H.T)
    assert np.allclose(H @ H, np.eye(256))
    assert np.all(np.abs(np.abs(H) - 1 / 16) == 0)
    # the H4 factor: row d is all +1 except -1 at column 3 - d
    for d in range(4):
        row = H4()[d]
        assert row[3 - d] == -1 and np.sum(row == 1) == 3


def test_integer_inputs_are_exact_against_the_closed_form():
    rng = np.random.default_rng(0)
    x = rng.integers(-8, 9, size=(32, 512)).astype(np.float32)
    y = O.convrot(x)
    H = dense_H()
    want = np.concatenate([x[:, :256] @ H.T, x[:, 256:] @ H.T], axis=1)
    assert np.array_equal(y.astype(np.float64), want)
    # a wrong Hadamard (2I - J) is detectably different
    wrong = x[:, :256] @ dense_H("2I-J").T
    assert not np.array_equal(y[:, :256].astype(np.float64), wrong)


def test_unit_vectors_give_the_columns():
    x = np.eye(256, dtype=np.float32)
    y = O.convrot(x)
    assert np.array_equal(y.astype(np.float64), dense_H().T)


def test_random_inputs_close_to_float64_and_involution():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((16, 1024)) * 3).astype(np.float32)
    y = O.convrot(x).astype(np.float64)
    H = dense_H()
    want = np.concatenate([x[:, g:g + 256].astype(np.float64) @ H.T for g in range(0, 1024, 256)], 1)
    assert np.max(np.abs(y - want)) < 1e-5
    back = O.convrot(O.convrot(x))
    assert np.max(np.abs(back - x)) < 1e-5
    assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x.astype(np.float64), axis=1), rtol=1e-6)


@pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) absent")
def test_convrot_matches_reference_build():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((24, 1536)) * 5).astype(np.float32)
    x[:, ::97] *= 20
    assert np.array_equal(O.convrot(x).view(np.uint32), O.ref_convrot(x).view(np.uint32))


# ------------------------------------------------------------------ A2
def half_away_exact(v: np.ndarray) -> np.ndarray:
    """Nearest integer, ties away from zero, computed exactly in float64
    (every fp32 and every fp32 + 0.5 below 2^24 is a float64)."""
    d = v.astype(np.float64)
    a = np.floor(np.abs(d) + 0.5)
    return np.where(d < 0, -a, a)


def near_ties(lo=-128, hi=128, ulps=3):
    """Every half-integer in [lo, hi] and its fp32 neighbours within `ulps`."""
    centres = np.arange(lo, hi) + 0.5
    out = [centres.astype(np.float32)]
    up = dn = centres.astype(np.float32)
    for _ in range(ulps):
        up = np.nextafter(up, np.float32(np.inf))
        dn = np.nextafter(dn, np.float32(-np.inf))
        out += [up, dn]
    return np.concatenate(out)


def quantise_identity(vals: np.ndarray, round_mode):
    """Quantise a row whose amax is 127 (so scale 1, inv 1): q = round(v)."""
    K = 256 * ((vals.size + 1 + 255) // 256)
    row = np.zeros(K, np.float32)
    row[:vals.size] = vals
    row[-1] = 127.0
    q, s = O.quantize_rows(row[None], rotate=False, round_mode=round_mode)
    assert s[0] == 1.0
    return q[0, :vals.size]


def test_half_away_rounding_on_every_near_tie():
    v = near_ties()
    v = v[np.abs(v) <= 127]
    q = quantise_identity(v, O.ROUND_HALF_AWAY)
    assert np.array_equal(q.astype(np.int64), np.clip(half_away_exact(v), -127, 127).astype(np.int64))


def test_half_even_rounding_on_every_near_tie():
    v = near_ties()
    v = v[np.abs(v) <= 127]
    q = quantise_identity(v, O.ROUND_HALF_EVEN)
    assert np.array_equal(q.astype(np.int64), np.clip(np.rint(v.astype(np.float64)), -127, 127).astype(np.int64))


def test_rounding_on_a_dense_sample_of_fp32():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2 ** 31, size=200000, dtype=np.uint32)
    v = bits.view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 127)]
    q = quantise_identity(v, O.ROUND_HALF_AWAY)
    assert np.array_equal(q.astype(np.int64), half_away_exact(v).astype(np.int64))


def test_crafted_ties_distinguish_the_modes():
    v = np.array([0.5, 1.5, 2.5, -0.5, -2.5, 126.5], np.float32)
    assert list(quantise_identity(v, O.ROUND_HALF_AWAY)) == [1, 2, 3, -1, -3, 127]
    assert list(quantise_identity(v, O.ROUND_HALF_EVEN)) == [0, 2, 2, 0, -2, 126]


def test_device_floor_form_differs_from_the_host_rule_at_exactly_two_values():
    """The reference has two quantisers: the host rule rounds half away in
    double (core/host/quant.cpp:163-166); its device kernel clamps, then takes
    floorf(d + 0.5f) / ceilf(d - 0.5f) with the sum rounded to fp32
    (core/kernels/int8_gemm.cpp:777-780).  The sum is exact for every fp32 d
    except d = +-(0.5 - 2^-25): 1 - 2^-25 lies halfway between the fp32
    neighbours 1 - 2^-24 and 1 and rounds to the even one, 1.  The exhaustive
    scan over every fp32 in [-128, 128] must find exactly those two."""
    n, vals = O.round_forms_differ()
    edge = 0.5 - 2.0 ** -25
    assert n == 2
    assert sorted(float(v) for v in vals) == [-edge, edge]
    # the mechanism: the fp32 sum at the edge is 1, at its neighbours it stays below
    assert np.float32(edge) + np.float32(0.5) == np.float32(1.0)
    below = np.nextafter(np.float32(edge), np.float32(0))
    assert below + np.float32(0.5) < np.float32(1.0)


def test_device_floor_mode_in_the_quantiser():
    """The device-kernel mode gives +-1 at d = +-(0.5 - 2^-25) where the host
    rule (the library's contract) gives 0, and agrees on every other near-tie,
    the exact ties included."""
    edge = np.float32(0.5 - 2.0 ** -25)
    v = np.concatenate([[edge, -edge], near_ties(-127, 127)]).astype(np.float32)
    host = quantise_identity(v, O.ROUND_HALF_AWAY).astype(np.int64)
    dev = quantise_identity(v, O.ROUND_DEVICE_FLOOR).astype(np.int64)
    assert list(host[:2]) == [0, 0] and list(dev[:2]) == [1, -1]
    at_edge = np.abs(v) == edge  # the near-tie set holds them too (0.5 less one ulp)
    assert np.array_equal(host[~at_edge], dev[~at_edge])
    assert np.array_equal(dev[at_edge] - host[at_edge], np.sign(v[at_edge]).astype(np.int64))
    ties = np.array([0.5, -0.5, 2.5, -2.5, 126.5, -126.5], np.float32)
    assert list(quantise_identity(ties, O.ROUND_DEVICE_FLOOR)) == [1, -1, 3, -3, 127, -127]


def test_row_invariants():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((64, 768)) * rng.uniform(0.01, 100, (64, 1))).astype(np.float32)
    x[5] = 0
    q, s = O.quantize_rows(x, rotate=False)
    assert s[5] == 1.0 and not q[5].any()
    live = np.arange(64) != 5
    amax = np.abs(x[live]).max(1)
    assert np.array_equal(s[live], (amax / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(q[live]).max(1) == 127)
    am = np.abs(x[live]).argmax(1)
    assert np.all(np.abs(q[live][np.arange(live.sum()), am]) == 127)
    q7, s7 = O.quantize_rows(x, rotate=True, qmax=7.0)
    assert np.abs(q7).max() == 7


def test_scale_and_codes_against_exact_arithmetic():
    """scale = fl(amax / 127); code = half-away(fl(v * fl(1/scale))), checked with
    exact rationals on a sample (pins the operation order of quant.cpp:158-166)."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((4, 256)) * 7).astype(np.float32)
    q, s = O.quantize_rows(x, rotate=False)
    for r in range(4):
        amax = np.float32(np.abs(x[r]).max())
        scale = np.float32(amax / np.float32(127))
        assert s[r] == scale
        inv = np.float32(np.float32(1) / scale)
        for c in range(0, 256, 17):
            d = Fraction(float(np.float32(x[r, c] * inv)))
            k = int(abs(d) + Fraction(1, 2)) * (1 if d >= 0 else -1)
            assert q[r, c] == max(-127, min(127, k))


@pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("rotate", [True, False])
def test_quantiser_matches_reference_build(rotate):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((40, 2560)).astype(np.float32)
    x[:, rng.choice(2560, 24, replace=False)] *= 20
    x[7] = 0
    q, s = O.quantize_rows(x, rotate=rotate)
    qr, sr = O.ref_quantize(x, rotate=rotate)
    assert np.array_equal(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))


@pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) absent")
def test_bf16_activations_match_reference_on_their_fp32_values():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((16, 3072)).astype(np.float32)
    b = O.f32_to_bf16(x)
    q, s = O.quantize_rows(b)
    qr, sr = O.ref_quantize(O.bf16_to_f32(b))
    assert np.array_equal(q, qr) and np.array_equal(s.view(np.uint32), sr.view(np.uint32))


def nonfinite_rows():
    """Rows with a NaN, an inf of either sign, both infs, and values that
    overflow inside the rotation, beside finite rows."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((8, 768)).astype(np.float32)
    x[1, 300] = np.nan
    x[2, 5] = np.inf
    x[3, 700] = -np.inf
    x[4, 10], x[4, 600] = np.inf, -np.inf
    x[5, 256:260] = 3e38           # the group's first pass overflows to inf
    x[6, 0], x[6, 1] = 3e38, -3e38  # +inf and -inf meet in a later pass: NaN, no inf
    return x


def test_nan_products_give_the_most_negative_code():
    """A NaN product becomes -qmax (the device form's fminf(fmaxf(d, -qmax),
    qmax)); an inf amax makes every finite value's code 0."""
    x = nonfinite_rows()
    for mode in (O.ROUND_HALF_AWAY, O.ROUND_HALF_EVEN):
        q, s = O.quantize_rows(x, round_mode=mode)
        y = O.convrot(x)
        assert np.all(q[1, 256:512] == -127) and np.isfinite(s[1])
        assert np.isinf(s[2]) and np.isinf(s[3]) and np.isinf(s[4])
        for r in (2, 3, 4):
            assert np.array_equal(q[r] == -127, ~np.isfinite(y[r])) and np.all(q[r][np.isfinite(y[r])] == 0)
        assert np.array_equal(q[0], O.quantize_rows(x[:1], round_mode=mode)[0][0])


@pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) absent")
def test_nonfinite_rows_match_reference_build():
    x = nonfinite_rows()
    q, s = O.quantize_rows(x)
    qr, sr = O.ref_quantize(x)
    assert np.array_equal(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))
