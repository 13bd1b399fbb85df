"""Pins for the oracle's A4/A5 (integer product, epilogue, bf16 rounding),
the scale-table decoders and A7 (grouped 4/6-bit decode + requantise).

* A4: against a float64 BLAS product (a library routine; exact because
  |acc| <= K*127^2 < 2^53) and the row/column checksum identities;
* A5: fma(t, sb, bias) against exact rational arithmetic rounded to fp32
  (ties to even); the separately rounded form against numpy float32;
  f32 -> bf16 against torch's conversion on every kind of value;
* decoders: f16 against numpy's float16 for all 65536 patterns, e4m3 / e5m2
  against torch's float8 types for all 256 patterns;
* A7: decoded values against the reference's own dequant_codebook_int4_row /
  dequant_packed6_row built from its sources (oracle/_ref), plus hand-worked
  cases for the int8-grid ties and the requantiser.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle as O


def rand_i8(shape, seed):
    return np.random.default_rng(seed).integers(-127, 128, size=shape).astype(np.int8)


# ------------------------------------------------------------------ A4
def test_gemm_against_blas_and_checksums():
    A, B = rand_i8((37, 320), 1), rand_i8((53, 320), 2)
    acc = O.gemm_i8_i32(A, B)
    assert np.array_equal(acc, (A.astype(np.float64) @ B.astype(np.float64).T).astype(np.int32))
    assert np.array_equal(acc.astype(np.int64).sum(1), A.astype(np.int64) @ B.astype(np.int64).sum(0))
    assert np.array_equal(acc.astype(np.int64).sum(0), B.astype(np.int64) @ A.astype(np.int64).sum(0))


def test_gemm_extremes_beyond_2_24():
    K = 12288
    A = np.full((2, K), 127, np.int8)
    A[1] = -127
    B = np.full((3, K), -127, np.int8)
    B[1, ::2] = 127
    acc = O.gemm_i8_i32(A, B)
    assert acc[0, 0] == -127 * 127 * K and acc[1, 0] == 127 * 127 * K and acc[0, 1] == 0
    assert abs(int(acc[0, 0])) > 2 ** 24


# ------------------------------------------------------------------ A5
def f32_round(fr: Fraction) -> np.float32:
    """Nearest fp32 to a rational, ties to even."""
    c = np.float32(float(fr))
    cands = [np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))]
    def key(v):
        return (abs(Fraction(float(v)) - fr), int(np.array(v, np.float32).view(np.uint32)) & 1)
    return min(cands, key=key)


def test_fused_epilogue_is_exactly_rounded():
    rng = np.random.default_rng(3)
    acc = rng.integers(-2 ** 27, 2 ** 27, size=(8, 64)).astype(np.int32)
    sa = rng.uniform(1e-4, 1e-1, 8).astype(np.float32)
    sb = rng.uniform(1e-4, 1e-1, 64).astype(np.float32)
    bias = (rng.standard_normal(64) * 0.02).astype(np.float32)
    y = O.epilogue(acc, sa, sb, bias, out="f32", fused=True)
    for m in range(8):
        for n in range(0, 64, 3):
            t = np.float32(np.float32(acc[m, n]) * sa[m])  # (float)acc is RNE, then one product
            want = f32_round(Fraction(float(t)) * Fraction(float(sb[n])) + Fraction(float(bias[n])))
            assert y[m, n] == want


def test_unfused_epilogue_and_no_bias_forms():
    rng = np.random.default_rng(4)
    acc = rng.integers(-2 ** 25, 2 ** 25, size=(16, 32)).astype(np.int32)
    sa = rng.uniform(1e-4, 1e-1, 16).astype(np.float32)
    sb = rng.uniform(1e-4, 1e-1, 32).astype(np.float32)
    bias = (rng.standard_normal(32) * 0.02).astype(np.float32)
    t = acc.astype(np.float32) * sa[:, None]
    y = O.epilogue(acc, sa, sb, bias, out="f32", fused=False)
    assert np.array_equal(y, (t * sb[None]) + bias[None])
    # without bias the fused and separate forms agree: fl(t * sb)
    y0 = O.epilogue(acc, sa, sb, None, out="f32", fused=True)
    assert np.array_equal(y0, t * sb[None])
    # per-tensor scale broadcasts
    y1 = O.epilogue(acc, sa, np.array([0.002], np.float32), None, out="f32")
    assert np.array_equal(y1, t * np.float32(0.002))


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32),
        (rng.standard_normal(1000) * 1e30).astype(np.float32),
        (rng.standard_normal(1000) * 1e-39).astype(np.float32),   # subnormals
        np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.3895314e38, -3.3895314e38,
                  np.inf, -np.inf], np.float32),
    ])
    # exact ties between two bf16 values, with even and odd kept lsb
    ties = (np.arange(0, 4096, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    got = O.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(O.bf16_to_f32(got), torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float().numpy())


# ------------------------------------------------------------------ decoders
def test_f16_decoder_all_patterns():
    pats = np.arange(65536, dtype=np.uint16)
    got = O.scale_table_to_f32(pats, O.F16)
    want = pats.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


@pytest.mark.parametrize("dt,tdt", [(O.F8_E4M3, torch.float8_e4m3fn), (O.F8_E5M2, torch.float8_e5m2),
                                    (O.U8_E4M3, torch.float8_e4m3fn)])
def test_fp8_decoders_all_patterns(dt, tdt):
    pats = np.arange(256, dtype=np.uint8)
    got = O.scale_table_to_f32(pats, dt)
    want = torch.from_numpy(pats).view(tdt).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])


# ------------------------------------------------------------------ A7
def test_uniform_nibbles_hand_case():
    """code - 8 levels, s_rel = 1, s_channel = 1: row of levels -8..7; amax 8,
    scale 8/127, q = half-away(level * 127/8)."""
    codes = np.array([[0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE] * 2], np.uint8)  # 0..15 twice
    s_rel = np.ones((1, 1), np.float32)
    q, s, v = O.w4a8_expand(codes, s_rel, O.F32, np.ones(1, np.float32), k=32, group=32,
                            return_values=True)
    levels = np.tile(np.arange(16) - 8, 2).astype(np.float32)
    assert np.array_equal(v[0], levels)
    assert s[0] == np.float32(np.float32(8) / np.float32(127))
    inv = np.float32(1) / s[0]
    d = (levels * inv).astype(np.float64)  # fp32 product, widened exactly
    want = np.where(d >= 0, np.floor(d + 0.5), np.ceil(d - 0.5))
    assert np.array_equal(q[0], want.astype(np.int8))


def test_int8_grid_rounds_ties_to_even():
    """level * s_rel = 2.5 -> 2, 3.5 -> 4, -2.5 -> -2 (RNE), and the grid clamps at 127."""
    codes = np.array([[0xAA, 0xBB, 0x66, 0xFF]], np.uint8)  # levels 2,2,3,3,-2,-2,7,7
    s_rel = np.array([[1.25, 1.25 / 1.0]], np.float32)  # group 4: cols 0-3 and 4-7
    _, _, v = O.w4a8_expand(codes, s_rel, O.F32, None, k=8, group=4, return_values=True)
    assert list(v[0]) == [2.0, 2.0, 4.0, 4.0, -2.0, -2.0, 9.0, 9.0]
    big = np.array([[40.0, 40.0]], np.float32)
    _, _, v = O.w4a8_expand(codes, big, O.F32, None, k=8, group=4, return_values=True)
    assert list(v[0]) == [80.0, 80.0, 120.0, 120.0, -80.0, -80.0, 127.0, 127.0]


def test_requantiser_is_the_plain_row_quantiser():
    rng = np.random.default_rng(6)
    codes = rng.integers(0, 256, (12, 128), dtype=np.uint8)
    s_rel = rng.uniform(0.5, 14, (12, 4)).astype(np.float32)
    sch = rng.uniform(1e-3, 1e-2, 12).astype(np.float32)
    q, s, v = O.w4a8_expand(codes, s_rel, O.F32, sch, k=256, group=64, return_values=True)
    q2, s2 = O.quantize_rows(v, rotate=False)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) absent")


@needs_ref
@pytest.mark.parametrize("with_cb", [False, True])
@pytest.mark.parametrize("with_corr", [False, True])
def test_nibble4_decode_matches_reference_build(with_cb, with_corr):
    rng = np.random.default_rng(7 + with_cb + 2 * with_corr)
    rows, k, group = 20, 512, 64
    codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
    s_rel = rng.uniform(0.25, 14, (rows, k // group)).astype(np.float32)
    s_rel[0, 0] = 0.5  # with code 3 / 5 levels this lands on exact .5 grid ties
    sch = rng.uniform(1e-3, 1e-2, rows).astype(np.float32)
    cb = (rng.standard_normal(16) * 4).astype(np.float32) if with_cb else None
    corr = (rng.standard_normal((k // group, rows)) * 1e-3).astype(np.float32) if with_corr else None
    _, _, v = O.w4a8_expand(codes, s_rel, O.F32, sch, k=k, group=group, codebook=cb,
                            correction=corr, return_values=True)
    vr = O.ref_grouped_decode(codes, s_rel, sch, k=k, group=group, codebook=cb, correction=corr)
    assert np.array_equal(v.view(np.uint32), vr.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("with_corr", [False, True])
def test_packed6_decode_matches_reference_build(with_corr):
    rng = np.random.default_rng(11)
    rows, k, group = 12, 768, 64
    codes = rng.integers(0, 256, (rows, k // 2 + k // 4), dtype=np.uint8)
    s_rel = rng.uniform(0.25, 3.5, (rows, k // group)).astype(np.float32)
    sch = rng.uniform(1e-3, 1e-2, rows).astype(np.float32)
    corr = (rng.standard_normal((k // group, rows)) * 1e-3).astype(np.float32) if with_corr else None
    _, _, v = O.w4a8_expand(codes, s_rel, O.F32, sch, k=k, group=group, layout=1, correction=corr,
                            return_values=True)
    vr = O.ref_grouped_decode(codes, s_rel, sch, k=k, group=group, correction=corr, six=True)
    assert np.array_equal(v.view(np.uint32), vr.view(np.uint32))


@needs_ref
def test_expanded_weight_equals_reference_requantiser():
    """decode (reference) -> quantize_weight without rotation (reference) equals
    the oracle's expand end to end."""
    rng = np.random.default_rng(12)
    rows, k, group = 16, 512, 128
    codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
    s_rel = rng.uniform(0.25, 14, (rows, k // group)).astype(np.float32)
    sch = rng.uniform(1e-3, 1e-2, rows).astype(np.float32)
    q, s = O.w4a8_expand(codes, s_rel, O.F32, sch, k=k, group=group)
    vr = O.ref_grouped_decode(codes, s_rel, sch, k=k, group=group)
    qr, sr = O.ref_quantize(vr, rotate=False)
    assert np.array_equal(q, qr) and np.array_equal(s.view(np.uint32), sr.view(np.uint32))


def test_gelu_oracle_against_torch():
    x = np.linspace(-8, 8, 20001, dtype=np.float32)
    got = O.gelu_tanh(x)
    want = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
