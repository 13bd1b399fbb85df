"""Oracle pins for the LoRA tail (CPU): out += (x A^T) B^T.

The reference computes both products as fp32 fma chains in a fixed order
(core/kernels/gemm_f16.cpp:56-200 and :237-308 under NVRTC's --fmad=true).
The oracle is checked against an independent exact-rational emulation of
those chains (each step one rounding of a*b + acc), against float64 within
the chain's error bound, and on data where the order of the chain decides
the result."""
from fractions import Fraction

import numpy as np
import pytest

import oracle


def rnd_f32(v: Fraction) -> np.float32:
    f = np.float32(float(v))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - v), int(np.float32(c).view(np.uint32)) & 1))
    return np.float32(best)


def fma_f32(a, b, c):
    """fmaf(a, b, c): the exact a*b + c rounded once (ties to even); an exact
    zero is -0 only when the product and c are both -0 (IEEE 754, nearest)."""
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    if exact != 0:
        return rnd_f32(exact)
    prod_zero_neg = (a == 0 or b == 0) and (np.signbit(np.float32(a)) != np.signbit(np.float32(b)))
    return np.float32(-0.0) if prod_zero_neg and np.signbit(np.float32(c)) else np.float32(0.0)


def fma_chain(pairs, start):
    acc = np.float32(start)
    for a, b in pairs:
        acc = fma_f32(a, b, acc)
    return acc


def test_lora_down_is_the_k_ordered_fma_chain():
    rng = np.random.default_rng(1)
    M, K, R = 3, 40, 4
    x = (rng.standard_normal((M, K)) * np.exp2(rng.integers(-6, 6, (M, K)))).astype(np.float32)
    a = (rng.standard_normal((R, K)) * np.exp2(rng.integers(-6, 6, (R, K)))).astype(np.float32)
    h = oracle.lora_down(x, a)
    for m in range(M):
        for r in range(R):
            want = fma_chain(zip(x[m], a[r]), 0.0)
            want = fma_f32(0.0, 0.0, want)  # K % 32 != 0: the padding's one visible step
            assert h[m, r].view(np.uint32) == want.view(np.uint32), (m, r)


def test_lora_rank_add_is_the_r_ordered_fma_chain_from_c():
    rng = np.random.default_rng(2)
    M, N, R = 3, 5, 17
    h = (rng.standard_normal((M, R)) * np.exp2(rng.integers(-6, 6, (M, R)))).astype(np.float32)
    b = (rng.standard_normal((N, R)) * np.exp2(rng.integers(-6, 6, (N, R)))).astype(np.float32)
    c = (rng.standard_normal((M, N)) * 4).astype(np.float32)
    out = oracle.lora_rank_add(h, b, c)
    for m in range(M):
        for n in range(N):
            want = fma_chain(zip(h[m], b[n]), c[m, n])
            assert out[m, n].view(np.uint32) == want.view(np.uint32), (m, n)


def test_chain_order_decides_the_result():
    # 2^24 + 1 - 2^24: ascending order loses the 1 (acc = 2^24 after the second
    # step), any order that pairs the big terms first keeps it.
    x = np.array([[1.0, 1.0, 1.0]], dtype=np.float32)
    a = np.array([[2.0 ** 24, 1.0, -(2.0 ** 24)]], dtype=np.float32)
    assert oracle.lora_down(x, a)[0, 0] == 0.0
    c = np.array([[2.0 ** 24]], dtype=np.float32)
    assert oracle.lora_rank_add(np.array([[1.0, -(2.0 ** 24)]], np.float32), np.array([[1.0, 1.0]], np.float32), c)[0, 0] == 0.0


def test_lora_tail_against_float64():
    rng = np.random.default_rng(3)
    M, K, R, N = 20, 256, 8, 30
    x = rng.standard_normal((M, K)).astype(np.float32)
    a = (rng.standard_normal((R, K)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((N, R)) * 0.05).astype(np.float32)
    out0 = rng.standard_normal((M, N)).astype(np.float32)
    out = oracle.lora_rank_add(oracle.lora_down(x, a), b, out0)
    ref = out0.astype(np.float64) + (x.astype(np.float64) @ a.T.astype(np.float64)) @ b.T.astype(np.float64)
    # a chain of n fp32 roundings: |err| <= n * 2^-24 * sum |terms| (loose)
    bound = (K + R) * 2.0 ** -24 * (np.abs(out0) + np.abs(x) @ np.abs(a).T @ np.abs(b).T)
    assert np.all(np.abs(out - ref) <= bound)


@pytest.mark.parametrize("K", [32, 40])
def test_lora_down_zero_sign_padding(K):
    # Every product -0 (x = -0, a > 0): the chain ends at -0 ... +0 from the
    # start value; with K % 32 != 0 the padding fma leaves +0 either way.
    x = np.full((1, K), -0.0, dtype=np.float32)
    a = np.ones((1, K), dtype=np.float32)
    h = oracle.lora_down(x, a)
    assert h[0, 0] == 0.0 and not np.signbit(h[0, 0])
