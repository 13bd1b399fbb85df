"""Oracle pins for the convrot_w4a4 family (CPU).

* The signed-int4 packer (quantize_convrot_w4a4, core/host/quant.cpp:247-272)
  against the reference's own function, compiled from its sources into
  oracle/_ref/phiref, and against closed forms: codes round half away from
  zero onto +-7, the row's largest rotated value maps to +-7, an all-zero row
  has scale 1, and the nibbles are low-first.
* The int4 GEMM (core/kernels/h3_kernels.cpp:546-635) against numpy's int64
  product of independently unpacked nibbles, and the fp32 epilogue's order
  ((acc * sa) * sb, no fma) against the other order on data chosen so the two
  differ.
"""
import numpy as np
import pytest

import oracle


def unpack_signed(packed, K):
    lo = (packed & 0x0F).astype(np.int16)
    hi = (packed >> 4).astype(np.int16)
    v = np.empty((packed.shape[0], K), dtype=np.int16)
    v[:, 0::2] = lo
    v[:, 1::2] = hi
    return np.where(v >= 8, v - 16, v).astype(np.int64)


def weights(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    w[:, rng.integers(0, cols, 3)] *= 20
    return w


@pytest.mark.skipif(not oracle.ref_available(), reason="reference build unavailable")
@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (33, 3072)])
def test_w4a4_packer_matches_reference_build(rows, cols):
    w = weights(rows, cols, rows + cols)
    w[0, :] = 0.0  # all-zero row: scale 1, codes 0
    p, s = oracle.quantize_convrot_w4a4(w)
    rp, rs = oracle.ref_w4a4pack(w)
    assert np.array_equal(p, rp)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_w4a4_packer_closed_forms():
    w = weights(9, 1024, 3)
    w[1] = 0.0
    p, s = oracle.quantize_convrot_w4a4(w)
    v = unpack_signed(p, 1024)
    rot = oracle.convrot(w)
    assert s[1] == 1.0 and np.all(v[1] == 0)
    for r in (0, 2, 5):
        amax = np.abs(rot[r]).max()
        assert s[r] == np.float32(amax / np.float32(7.0))
        assert np.abs(v[r]).max() == 7
        assert v[r, np.argmax(np.abs(rot[r]))] == np.sign(rot[r, np.argmax(np.abs(rot[r]))]) * 7
        # every code is the half-away rounding of v / s, clamped
        d = (rot[r] / s[r]).astype(np.float32).astype(np.float64)
        want = np.clip(np.sign(d) * np.floor(np.abs(d) + 0.5), -7, 7)
        assert np.array_equal(v[r], want)


def test_w4a4_packer_ties_go_away_from_zero():
    # A single nonzero group whose rotation is known: e_0 rotates to the
    # all-(+-1/16) column, so feed values that land exactly on k + 1/2 after
    # the division instead, via the inverse rotation (H is its own inverse).
    target = np.zeros((1, 256), dtype=np.float32)
    target[0, :8] = [7.0, 2.5, -2.5, 0.5, -0.5, 1.5, -3.5, 6.5]
    w = oracle.convrot(target)  # H target; rotating it again gives target back (exact here)
    assert np.array_equal(oracle.convrot(w), target)
    p, s = oracle.quantize_convrot_w4a4(w)
    assert s[0] == 1.0
    v = unpack_signed(p, 256)[0, :8]
    assert list(v) == [7, 3, -3, 1, -1, 2, -4, 7]


@pytest.mark.parametrize("M,N,K", [(1, 1, 512), (5, 7, 512), (64, 48, 1024)])
def test_int4_gemm_against_numpy(M, N, K):
    rng = np.random.default_rng(M * N + K)
    a = rng.integers(-7, 8, (M, K)).astype(np.int8)
    b = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    sa = rng.uniform(0.01, 0.2, M).astype(np.float32)
    sb = rng.uniform(0.01, 0.2, N).astype(np.float32)
    c = oracle.int4_gemm(a, b, sa, sb)
    acc = a.astype(np.int64) @ unpack_signed(b, K).T
    want = (acc.astype(np.float32) * sa[:, None]).astype(np.float32) * sb[None, :]
    assert np.array_equal(c.view(np.uint32), want.astype(np.float32).view(np.uint32))
    # nibble order: all codes 0x8f -> even columns -1, odd columns -8
    b2 = np.full((N, K // 2), 0x8F, dtype=np.uint8)
    c2 = oracle.int4_gemm(np.ones((M, K), np.int8), b2, np.ones(M, np.float32), np.ones(N, np.float32))
    assert np.all(c2 == -(K // 2) * 9)


def test_int4_gemm_epilogue_order():
    """((acc * sa) * sb): on these scales the other association differs."""
    rng = np.random.default_rng(5)
    M, N, K = 16, 16, 512
    a = rng.integers(-7, 8, (M, K)).astype(np.int8)
    b = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    sa = rng.uniform(0.001, 0.3, M).astype(np.float32)
    sb = rng.uniform(0.001, 0.3, N).astype(np.float32)
    c = oracle.int4_gemm(a, b, sa, sb)
    acc = (a.astype(np.int64) @ unpack_signed(b, K).T).astype(np.float32)
    other = acc * (sa[:, None] * sb[None, :]).astype(np.float32)
    assert not np.array_equal(c, other.astype(np.float32))
