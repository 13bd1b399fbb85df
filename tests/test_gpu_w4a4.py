"""GPU parity: the convrot_w4a4 int4 GEMM (phi_hip_i4_gemm).

Bar: bit-exact with the oracle's restatement of the reference's int4_gemm
(core/kernels/h3_kernels.cpp:546-635): int32 accumulators of signed nibbles,
then C = ((float)acc * sa) * sb in fp32 (bf16 output: that value rounded RNE).
Every kernel path is exercised: the persistent kernel with the constant
signed-nibble table (both tile sizes), the expand-once path through the
caller's workspace, and the register-staged kernel (forced, or for code rows
that are not 16-byte aligned)."""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


def operands(M, N, K, seed, ldb_pad=0):
    g = torch.Generator().manual_seed(seed)
    A = torch.randint(-7, 8, (M, K), generator=g, dtype=torch.int8)
    Bw = torch.randint(0, 256, (N, K // 2 + ldb_pad), generator=g, dtype=torch.uint8)
    sA = torch.rand(M, generator=g) * 0.2 + 0.01
    sB = torch.rand(N, generator=g) * 0.2 + 0.01
    return A, Bw, sA, sB


def unpack_signed(packed, K):
    p = packed[:, :K // 2].astype(np.int16)
    v = np.empty((packed.shape[0], K), dtype=np.int16)
    v[:, 0::2] = p & 0x0F
    v[:, 1::2] = p >> 4
    return np.where(v >= 8, v - 16, v).astype(np.int64)


SHAPES = [(1, 64, 512), (37, 136, 1024), (256, 3072, 512), (777, 1032, 1536), (1024, 512, 5120)]
KERNELS = ["auto", "persist256", "persist128", "tile128"]


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("with_ws", [False, True])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_i4_gemm_matches_oracle(dev, orc, monkeypatch, kernel, with_ws, M, N, K):
    if kernel != "auto":
        monkeypatch.setenv("PHI_GEMM_KERNEL", kernel)
    A, Bw, sA, sB = operands(M, N, K, M + N + K)
    ws = Q.i4_workspace(M, N, K, dev) if with_ws else None
    if with_ws and ws is None and M >= 512:
        pytest.fail("a workspace is expected from 512 rows")
    C = Q.i4_gemm(A.to(dev), Bw.to(dev), sA.to(dev), sB.to(dev), workspace=ws)
    torch.cuda.synchronize()
    want = orc.int4_gemm(A.numpy(), Bw.numpy(), sA.numpy(), sB.numpy())
    got = C.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{(got != want).sum()} mismatches"


@pytest.mark.parametrize("M,N,K", [(64, 256, 512), (300, 1000, 1024)])
def test_i4_gemm_int32_and_bf16_outputs(dev, orc, M, N, K):
    A, Bw, sA, sB = operands(M, N, K, 9)
    acc = Q.i4_gemm(A.to(dev), Bw.to(dev), None, None, out_dtype=torch.int32)
    Cb = Q.i4_gemm(A.to(dev), Bw.to(dev), sA.to(dev), sB.to(dev), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    want_acc = A.numpy().astype(np.int64) @ unpack_signed(Bw.numpy(), K).T
    assert np.array_equal(acc.cpu().numpy(), want_acc.astype(np.int32))
    want = torch.from_numpy(orc.int4_gemm(A.numpy(), Bw.numpy(), sA.numpy(), sB.numpy())).to(torch.bfloat16)
    assert torch.equal(Cb.cpu().view(torch.int16), want.view(torch.int16))


def test_i4_gemm_unaligned_code_rows_take_the_staged_kernel(dev, orc):
    M, N, K = 200, 264, 1024
    A, Bw, sA, sB = operands(M, N, K, 4, ldb_pad=8)  # row pitch K/2 + 8: 8-byte, not 16-byte, aligned
    C = Q.i4_gemm(A.to(dev), Bw.to(dev), sA.to(dev), sB.to(dev))
    torch.cuda.synchronize()
    want = orc.int4_gemm(A.numpy(), np.ascontiguousarray(Bw.numpy()[:, :K // 2]), sA.numpy(), sB.numpy())
    assert np.array_equal(C.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_w4a4_linear_end_to_end(dev, orc):
    """The text encoder's linear (core/models/text_encoder_32b.cpp:898-936):
    quant_convrot with qmax 7, then int4_gemm, on weights packed by the
    reference's quantize_convrot_w4a4 (oracle restatement)."""
    M, K, N = 333, 1536, 640
    x = synth.activations(M, K, seed=21).float()
    g = torch.Generator().manual_seed(22)
    w = torch.randn(N, K, generator=g)
    packed, sw = orc.quantize_convrot_w4a4(w.numpy())
    q, s = Q.quant_rotate(x.to(dev), qmax=7.0)
    C = Q.i4_gemm(q, torch.from_numpy(packed).to(dev), s, torch.from_numpy(sw).to(dev))
    torch.cuda.synchronize()
    qo, so = orc.quantize_rows(x.numpy(), qmax=7.0)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert int(np.abs(qo).max()) == 7
    want = orc.int4_gemm(qo, packed, so, sw)
    assert np.array_equal(C.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # and it approximates the float linear of the rotated operands (H is orthonormal)
    ref = x.numpy().astype(np.float64) @ w.numpy().astype(np.float64).T
    err = np.linalg.norm(C.cpu().numpy() - ref) / np.linalg.norm(ref)
    assert err < 0.25


@pytest.mark.parametrize("M", [512, 4352])
def test_i4_gemm_large_expand_once_equals_in_register(dev, M):
    N, K = 1024, 3072
    A, Bw, sA, sB = operands(M, N, K, M)
    A, Bw, sA, sB = A.to(dev), Bw.to(dev), sA.to(dev), sB.to(dev)
    c1 = Q.i4_gemm(A, Bw, sA, sB)
    c2 = Q.i4_gemm(A, Bw, sA, sB, workspace=Q.i4_workspace(M, N, K, dev))
    acc = Q.i4_gemm(A, Bw, None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    assert torch.equal(c1.view(torch.int32), c2.view(torch.int32))
    # checksum identity on the full size: sum_n acc[m, n] = A[m] . (sum_n w[n])
    w = torch.from_numpy(unpack_signed(Bw.cpu().numpy(), K)).double()
    assert torch.equal(acc.double().sum(1).cpu(), A.double().cpu() @ w.sum(0))
