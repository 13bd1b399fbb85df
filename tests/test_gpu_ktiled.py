"""GPU parity of the K-tiled operand path (phi_hip_pack_k_tiled,
phi_hip_quant_rotate_kt / _mod_kt / _act_kt, phi_hip_i8_gemm_kt,
phi_hip_i8_gemm_residual_kt, phi_hip_q8_linear_kt, and phi_hip_q8_linear_kq: K-tiled
activations against a row-major weight).

The K-tiled layout is a re-arrangement of the same bytes, so the bar is
identity with the row-major path, which the other GPU tests hold bit-exact
against the oracle:
* pack_k_tiled is the permutation the header documents (checked against a
  numpy gather on small matrices, partial strips included) and loses nothing
  (unpacking restores the matrix);
* quant_rotate_kt writes the same codes and scales as quant_rotate, in that
  permutation, with and without the modulation or an activation in front;
* the K-tiled GEMM and linear give the row-major path's outputs bit for bit
  (int32, fp32 and bf16), at small, ragged and the configs' full sizes, on
  each tile plan (mixed, 256 x 256 only, 128 x 128 only), and so does the
  gated residual update.
"""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


def kt_index(rows, K):
    """For each (r, k) of a rows x K matrix, its byte position in the K-tiled
    layout (the header's formula, evaluated with numpy)."""
    r = np.arange(rows)[:, None]
    k = np.arange(K)[None, :]
    s, rr = r // 256, r % 256
    h = np.minimum(256, rows - 256 * s)
    slot = ((k // 16) % 4) ^ ((rr // 4) % 4)
    return 256 * K * s + h * 64 * (k // 64) + 64 * rr + 16 * slot + k % 16


@pytest.mark.parametrize("rows,K", [(1, 256), (16, 512), (100, 256), (256, 768), (300, 512), (513, 1024)])
def test_pack_is_the_documented_permutation(dev, rows, K):
    W = synth.int8_weight(rows, K, seed=rows + K)
    packed = Q.pack_k_tiled(W.to(dev)).cpu().numpy()
    idx = kt_index(rows, K)
    assert np.array_equal(np.sort(idx.ravel()), np.arange(rows * K))  # a permutation of rows * K bytes
    assert np.array_equal(packed[idx], W.numpy())


def test_pack_with_row_pitch(dev):
    """A source with row pitch > K packs only its first K columns."""
    rows, K, ld = 300, 512, 640
    big = synth.int8_weight(rows, ld, seed=5).to(dev)
    packed = Q.pack_k_tiled(big[:, :K]).cpu().numpy()
    assert np.array_equal(packed[kt_index(rows, K)], big[:, :K].cpu().numpy())


@pytest.mark.parametrize("rows,K", [(1, 256), (77, 3072), (300, 1024), (4352, 3072), (4352, 12288)])
def test_quant_rotate_kt_is_quant_rotate_packed(dev, rows, K):
    x = synth.activations(rows, K, seed=rows, device=dev)
    q, s = Q.quant_rotate(x)
    qk, sk = Q.quant_rotate_kt(x)
    assert torch.equal(s, sk)
    assert torch.equal(qk, Q.pack_k_tiled(q))


GEMM_SHAPES = [(1, 256, 256), (100, 264, 512), (300, 1000, 768), (513, 520, 1024), (4352, 12288, 3072),
               (4352, 3072, 12288), (32760, 512, 512)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("out", ["bf16", "f32", "i32"])
def test_gemm_kt_matches_row_major(dev, M, N, K, out):
    A = synth.int8_weight(M, K, seed=M, device=dev)
    B = synth.int8_weight(N, K, seed=N + 1, device=dev)
    sA = torch.rand(M, device=dev) * 0.01 + 1e-3
    sB = torch.rand(N, device=dev) * 0.01 + 1e-3
    bias = synth.bias(N, seed=3, device=dev)
    odt = {"bf16": torch.bfloat16, "f32": torch.float32, "i32": torch.int32}[out]
    want = Q.i8_gemm(A, B, sA, sB, bias, out_dtype=odt)
    got = Q.i8_gemm_kt(Q.pack_k_tiled(A), Q.pack_k_tiled(B), M, N, K, sA, sB, bias, out_dtype=odt)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16 if out == "bf16" else torch.int32),
                       want.view(torch.int16 if out == "bf16" else torch.int32))


@pytest.mark.parametrize("plan", ["persist256", "persist128"])
def test_gemm_kt_each_tile_plan(dev, monkeypatch, plan):
    """Forced single-size plans: 256 x 256 tiles over a partial last strip,
    and 128 x 128 tiles in both halves of every strip."""
    monkeypatch.setenv("PHI_GEMM_KERNEL", plan)
    M, N, K = 700, 1040, 1536
    A = synth.int8_weight(M, K, seed=11, device=dev)
    B = synth.int8_weight(N, K, seed=12, device=dev)
    want = Q.i8_gemm(A, B, None, None, out_dtype=torch.int32)
    got = Q.i8_gemm_kt(Q.pack_k_tiled(A), Q.pack_k_tiled(B), M, N, K, None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("M,K,N", [(1, 256, 512), (77, 3072, 1000), (4352, 3072, 12288), (4352, 12288, 3072)])
def test_q8_linear_kt_matches_q8_linear(dev, M, K, N):
    x = synth.activations(M, K, seed=M + 7, device=dev)
    W = synth.int8_weight(N, K, seed=1, device=dev)
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=2, device=dev)
    q8 = torch.empty((M, K), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    want = Q.q8_linear(x, W, sW, b, q8=q8, s8=s8)
    qk = torch.empty((M * K,), dtype=torch.int8, device=dev)
    sk = torch.empty((M,), dtype=torch.float32, device=dev)
    got = Q.q8_linear_kt(x, Q.pack_k_tiled(W), N, sW, b, q8=qk, s8=sk)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(sk, s8)
    assert torch.equal(qk, Q.pack_k_tiled(q8))


def _kq_against_q8_linear(dev, M, K, N, *, ldw=None, out=torch.bfloat16, bias=True, seed=0):
    """q8_linear_kq against q8_linear on the same inputs: C and s8 bit for
    bit; q8 holds the row-major codes, K-tiled (the mixed plan) or as they are
    (where the call falls back to q8_linear).  Returns which layout q8 took."""
    x = synth.activations(M, K, seed=M + seed, device=dev)
    Ww = synth.int8_weight(N, ldw or K, seed=3 + seed, device=dev)
    W = Ww[:, :K]
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=2, device=dev) if bias else None
    q8 = torch.empty((M, K), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    want = Q.q8_linear(x, W.contiguous(), sW, b, q8=q8, s8=s8, out_dtype=out)
    qk = torch.empty((M, K), dtype=torch.int8, device=dev)
    sk = torch.empty((M,), dtype=torch.float32, device=dev)
    got = Q.q8_linear_kq(x, W, sW, b, q8=qk, s8=sk, out_dtype=out)
    torch.cuda.synchronize()
    bits = torch.int16 if out == torch.bfloat16 else torch.int32
    assert torch.equal(got.view(bits), want.view(bits))
    assert torch.equal(sk, s8)
    if torch.equal(qk, q8):
        return "row-major"
    assert torch.equal(qk.view(-1), Q.pack_k_tiled(q8).view(-1))
    return "k-tiled"


@pytest.mark.parametrize("M,K,N", [(4352, 3072, 12288), (4352, 12288, 3072), (4352, 3072, 9216)])
def test_q8_linear_kq_at_dit_shapes(dev, M, K, N):
    """The drop-in's row-major weight at the DiT shapes: the mixed plan (A
    K-tiled, B gathered row by row on the 272 x 192 kernel) takes them."""
    assert _kq_against_q8_linear(dev, M, K, N) == "k-tiled"


@pytest.mark.parametrize("M,K,N,ldw", [(300, 512, 200, 512), (1000, 1024, 4000, 1040), (2000, 512, 30000, 512),
                                       (555, 3072, 9216, 3088), (100, 1024, 8, 1024)])
@pytest.mark.parametrize("out", [torch.bfloat16, torch.float32])
def test_q8_linear_kq_forced_mixed(dev, monkeypatch, M, K, N, ldw, out):
    """The mixed plan forced (PHI_GEMM_T272=1) over ragged shapes, weights
    with a row pitch above K, several tiles a workgroup."""
    monkeypatch.setenv("PHI_GEMM_T272", "1")
    assert _kq_against_q8_linear(dev, M, K, N, ldw=ldw, out=out, seed=ldw) == "k-tiled"


@pytest.mark.parametrize("M,K,N", [(256, 3072, 3072), (77, 768, 300), (64, 256, 512)])
def test_q8_linear_kq_falls_back(dev, M, K, N):
    """Shapes the mixed plan does not take (too few tiles to pay, K not a
    multiple of 512) run q8_linear itself."""
    assert _kq_against_q8_linear(dev, M, K, N, bias=False) == "row-major"


@pytest.mark.parametrize("M,K", [(1, 256), (77, 3072), (300, 1024), (4352, 3072)])
def test_fused_prologues_kt(dev, M, K):
    """The modulation and the activations in front of the K-tiled quantiser
    give the row-major codes, packed, and the same scales."""
    g = torch.Generator(device=dev).manual_seed(M + K)
    x = synth.activations(M, K, seed=M, device=dev)
    sc = torch.randn(K, generator=g, device=dev) * 0.1
    sh = torch.randn(K, generator=g, device=dev) * 0.1
    q, s = Q.quant_rotate(x, mod_scale=sc, mod_shift=sh)
    qk, sk = Q.quant_rotate_kt(x, mod_scale=sc, mod_shift=sh)
    assert torch.equal(sk, s) and torch.equal(qk, Q.pack_k_tiled(q))
    q, s = Q.quant_rotate(x, act="gelu_tanh")
    qk, sk = Q.quant_rotate_kt(x, act="gelu_tanh")
    assert torch.equal(sk, s) and torch.equal(qk, Q.pack_k_tiled(q))
    gx = synth.activations(M, 2 * K, seed=M + 1, device=dev)
    q, s = Q.quant_rotate(gx, act="silu_gate")
    qk, sk = Q.quant_rotate_kt(gx, act="silu_gate")
    assert torch.equal(sk, s) and torch.equal(qk, Q.pack_k_tiled(q))


@pytest.mark.parametrize("M,N,K", [(300, 1000, 768), (4352, 3072, 12288), (700, 1040, 1536)])
def test_gemm_residual_kt_matches_row_major(dev, M, N, K):
    A = synth.int8_weight(M, K, seed=M, device=dev)
    B = synth.int8_weight(N, K, seed=N, device=dev)
    sA = torch.rand(M, device=dev) * 0.01 + 1e-3
    sB = synth.weight_scale(0.002, device=dev)
    bias = synth.bias(N, seed=3, device=dev)
    gate = torch.randn(N, device=dev) * 0.1
    H0 = torch.randn(M, N, device=dev)
    H_row, H_kt = H0.clone(), H0.clone()
    Q.i8_gemm_residual(A, B, sA, sB, bias, gate, H_row)
    Q.i8_gemm_residual_kt(Q.pack_k_tiled(A), Q.pack_k_tiled(B), M, N, K, sA, sB, bias, gate, H_kt)
    torch.cuda.synchronize()
    assert torch.equal(H_kt.view(torch.int32), H_row.view(torch.int32))
