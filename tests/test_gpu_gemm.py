"""GPU parity: int8 MFMA GEMM + epilogue (phi_hip_i8_gemm) vs the oracle.

Bar: int32 accumulators bit-exact; fp32 / bf16 outputs bit-exact against the
oracle's epilogue fma((float)acc*sa, sb, bias) (reference
core/kernels/int8_gemm.cpp:588-620), and within 1 bf16 ulp of the separately
rounded form (the tolerance stated for floating point, rel <= 8e-3).
At full benchmark sizes the int32 product is checked by row/column checksums
(sum_n C = A . sum_n B, sum_m C = (sum_m A) . B), exact in float64."""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu

BF16_REL_TOL = 8e-3  # 1 bf16 ulp (2^-7), as stated for the bf16 outputs


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def rand_i8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)


# "<kernel>:2stage" runs the persistent plan on the two-stage kernel
# (PHI_GEMM_PIPE=0) instead of the four-stage pipeline.
KERNELS = ["auto", "persist", "persist256", "persist128", "persist:2stage", "persist256:2stage",
           "persist128:2stage", "tile256", "tile256w4", "tile128"]


def select_kernel(monkeypatch, name):
    """The PHI_GEMM_KERNEL / PHI_GEMM_PIPE A/B switches."""
    kern, _, variant = name.partition(":")
    if kern == "auto":
        monkeypatch.delenv("PHI_GEMM_KERNEL", raising=False)
    else:
        monkeypatch.setenv("PHI_GEMM_KERNEL", kern)
    if variant == "2stage":
        monkeypatch.setenv("PHI_GEMM_PIPE", "0")
    else:
        monkeypatch.delenv("PHI_GEMM_PIPE", raising=False)


@pytest.fixture(params=KERNELS)
def kernel(request, monkeypatch):
    """Every GEMM kernel sees every shape."""
    select_kernel(monkeypatch, request.param)
    return request.param


@pytest.mark.parametrize("M,N,K", [(1, 1, 64), (1, 37, 128), (5, 300, 192), (256, 256, 3072),
                                   (257, 129, 640), (300, 1000, 256), (512, 384, 1024),
                                   (33, 4100, 64), (1000, 70, 576), (513, 777, 320),
                                   # shapes the persistent kernel takes (K % 256 == 0, N % 4 == 0):
                                   # partial tiles in M and N, one to several tiles per workgroup,
                                   # the shortest K it accepts
                                   (1, 4, 512), (300, 1000, 512), (257, 264, 768), (777, 520, 1280),
                                   (2049, 2052, 512), (4100, 4104, 1024), (129, 136, 256),
                                   (640, 384, 256)])
def test_int32_accumulators_exact(dev, orc, kernel, M, N, K):
    A, B = rand_i8((M, K), M + K), rand_i8((N, K), N + 7)
    C = Q.i8_gemm(A.to(dev), B.to(dev), None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    want = orc.gemm_i8_i32_fast(A.numpy(), B.numpy())
    assert np.array_equal(C.cpu().numpy(), want)


def test_extreme_accumulators(dev, orc):
    """All +-127 at K = 12288: |acc| = 1.98e8 > 2^24, so (float)acc rounds."""
    M, N, K = 64, 128, 12288
    A = torch.full((M, K), 127, dtype=torch.int8)
    A[1::2] = -127
    B = torch.full((N, K), 127, dtype=torch.int8)
    B[:, ::3] = -127
    sa = torch.rand(M) * 0.01 + 0.001
    sb = torch.rand(N) * 0.01 + 0.001
    C32 = Q.i8_gemm(A.to(dev), B.to(dev), None, None, out_dtype=torch.int32).cpu().numpy()
    acc = orc.gemm_i8_i32_fast(A.numpy(), B.numpy())
    assert np.array_equal(C32, acc)
    Cf = Q.i8_gemm(A.to(dev), B.to(dev), sa.to(dev), sb.to(dev), out_dtype=torch.float32)
    want = orc.epilogue(acc, sa.numpy(), sb.numpy(), out="f32")
    assert np.array_equal(Cf.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bias_kind", [None, "f32", "bf16"])
@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("sb_scalar", [True, False])
@pytest.mark.parametrize("M,N,K", [(130, 262, 384), (130, 264, 512), (600, 776, 1024)])
def test_epilogue_bit_exact(dev, orc, kernel, bias_kind, out, sb_scalar, M, N, K):
    A, B = rand_i8((M, K), 3), rand_i8((N, K), 4)
    g = torch.Generator().manual_seed(9)
    sa = torch.rand(M, generator=g) * 0.05 + 0.002
    sb = torch.full((1,), 0.002) if sb_scalar else torch.rand(N, generator=g) * 0.05 + 0.002
    bias = None
    if bias_kind == "f32":
        bias = torch.randn(N, generator=g) * 0.02
    elif bias_kind == "bf16":
        bias = (torch.randn(N, generator=g) * 0.02).to(torch.bfloat16)
    C = Q.i8_gemm(A.to(dev), B.to(dev), sa.to(dev), sb.to(dev),
                  None if bias is None else bias.to(dev),
                  out_dtype=torch.bfloat16 if out == "bf16" else torch.float32)
    acc = orc.gemm_i8_i32_fast(A.numpy(), B.numpy())
    b_np = None if bias is None else (u16(bias) if bias.dtype == torch.bfloat16 else bias.numpy())
    want = orc.epilogue(acc, sa.numpy(), sb.numpy(), b_np, out=out)
    got = u16(C) if out == "bf16" else C.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, want if out == "bf16" else want.view(np.uint32))
    if out == "bf16" and bias is not None:
        # vs the separately rounded epilogue: within one bf16 ulp
        alt = orc.bf16_to_f32(orc.epilogue(acc, sa.numpy(), sb.numpy(), b_np, out="bf16", fused=False))
        g32 = orc.bf16_to_f32(got)
        np.testing.assert_allclose(g32, alt, rtol=BF16_REL_TOL, atol=1e-30)


@pytest.mark.parametrize("layout", ["row", "kt"])
@pytest.mark.parametrize("M,N,K", [(4352, 4352, 512), (3000, 8000, 768)])
def test_epilogue_many_tiles_per_workgroup(dev, orc, layout, M, N, K):
    """The default plan at small K with more tiles than CUs: every workgroup
    runs several tiles, so the next tile's first MFMAs inside the epilogue, the
    once-a-tile bias conversion and the tile order's divisions all run between
    tiles.  bf16 bias and bf16 output, bit for bit against the oracle."""
    A, B = rand_i8((M, K), M + 11), rand_i8((N, K), N + 13)
    g = torch.Generator().manual_seed(M + N)
    sa = torch.rand(M, generator=g) * 0.05 + 0.002
    sb = torch.rand(N, generator=g) * 0.05 + 0.002
    bias = (torch.randn(N, generator=g) * 0.02).to(torch.bfloat16)
    Ad, Bd = A.to(dev), B.to(dev)
    if layout == "row":
        C = Q.i8_gemm(Ad, Bd, sa.to(dev), sb.to(dev), bias.to(dev), out_dtype=torch.bfloat16)
    else:
        C = Q.i8_gemm_kt(Q.pack_k_tiled(Ad), Q.pack_k_tiled(Bd), M, N, K, sa.to(dev), sb.to(dev), bias.to(dev),
                         out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    acc = orc.gemm_i8_i32_fast(A.numpy(), B.numpy())
    want = orc.epilogue(acc, sa.numpy(), sb.numpy(), u16(bias), out="bf16")
    got = u16(C)
    assert np.array_equal(got, want), f"{(got != want).sum()} of {got.size} outputs differ"


def test_reference_gemm_int8_equality(dev, orc):
    """No bias, fp32 out: the product equals the reference host gemm_int8's
    (float)acc * sx[m] * sw[n] (core/host/quant.cpp:223-236) bit for bit."""
    if not orc.ref_available():
        pytest.skip("reference build (oracle/_ref) not present on this machine")
    M, N, K = 64, 96, 512
    A, B = rand_i8((M, K), 21), rand_i8((N, K), 22)
    sa = torch.rand(M) * 0.01 + 0.001
    sb = torch.rand(N) * 0.01 + 0.001
    C = Q.i8_gemm(A.to(dev), B.to(dev), sa.to(dev), sb.to(dev), out_dtype=torch.float32)
    want = orc.ref_gemm(A.numpy(), sa.numpy(), B.numpy(), sb.numpy())
    assert np.array_equal(C.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("out", [torch.int32, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K,pad", [(300, 290, 448, 3), (300, 296, 512, 8)])
def test_strided_and_unaligned_operands(dev, orc, kernel, out, M, N, K, pad):
    """lda > K, ldb > K, and an output row pitch that is not a multiple of 4
    (the epilogue's scalar-store path) or padded by 8 (the persistent
    kernel's whole-row stores), with a bias view at an odd offset."""
    Aw, Bw = rand_i8((M, K + 64), 31), rand_i8((N, K + 128), 32)
    A, B = Aw[:, 16:16 + K], Bw[:, 32:32 + K]
    g = torch.Generator().manual_seed(33)
    sa = torch.rand(M, generator=g) * 0.05 + 0.002
    sbw = torch.rand(N + 1, generator=g) * 0.05 + 0.002
    biasw = torch.randn(N + 1, generator=g) * 0.02
    Ad, Bd = Aw.to(dev)[:, 16:16 + K], Bw.to(dev)[:, 32:32 + K]
    Cw = torch.zeros((M, N + pad), dtype=out, device=dev)
    C = Cw[:, :N]
    scaled = out != torch.int32
    Q.i8_gemm(Ad, Bd, sa.to(dev) if scaled else None, sbw.to(dev)[1:] if scaled else None,
              biasw.to(dev)[1:] if scaled else None, C=C)
    acc = orc.gemm_i8_i32_fast(A.contiguous().numpy(), B.contiguous().numpy())
    if not scaled:
        assert np.array_equal(C.cpu().numpy(), acc)
    else:
        o = "bf16" if out == torch.bfloat16 else "f32"
        want = orc.epilogue(acc, sa.numpy(), sbw[1:].numpy(), biasw[1:].numpy(), out=o)
        got = u16(C.contiguous()) if o == "bf16" else C.cpu().contiguous().numpy().view(np.uint32)
        assert np.array_equal(got, want if o == "bf16" else want.view(np.uint32))
    assert torch.count_nonzero(Cw[:, N:]) == 0, "wrote past the row"


def checksums_ok(A, B, C32):
    """Exact ABFT identities in float64 on the device."""
    Af, Bf, Cf = A.double(), B.double(), C32.double()
    row_ok = torch.equal(Cf.sum(1), Af @ Bf.sum(0))
    col_ok = torch.equal(Cf.sum(0), Bf @ Af.sum(0))
    return row_ok and col_ok


@pytest.mark.slow
@pytest.mark.parametrize("M,N,K", [(4352, 12288, 3072), (4352, 3072, 12288), (4352, 9216, 3072),
                                   (32760, 5120, 5120), (32760, 13824, 5120)])
def test_full_size_checksums(dev, kernel, M, N, K):
    A = synth.int8_weight(M, K, seed=M, device=dev)
    B = synth.int8_weight(N, K, seed=N, device=dev)
    C32 = Q.i8_gemm(A, B, None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    assert checksums_ok(A, B, C32)
    # A sampled block against an independent exact product.
    rs = torch.arange(0, M, 97, device=dev)[:64]
    cs = torch.arange(0, N, 89, device=dev)[:64]
    blk = (A[rs].double() @ B[cs].double().t()).to(torch.int64)
    assert torch.equal(C32[rs][:, cs].to(torch.int64), blk)
    # bf16 epilogue at full size: same accumulators through the scaled store.
    sa = torch.rand(M, device=dev) * 0.01 + 1e-3
    sb = torch.full((1,), 0.002, device=dev)
    Cb = Q.i8_gemm(A, B, sa, sb, out_dtype=torch.bfloat16)
    want = (C32.float() * sa[:, None] * sb).to(torch.bfloat16)
    assert torch.equal(Cb.view(torch.int16), want.view(torch.int16))


def test_contract_errors(dev):
    B = torch.zeros((4, 64), dtype=torch.int8, device=dev)
    A = torch.zeros((0, 64), dtype=torch.int8, device=dev)
    with pytest.raises(Q.QLinearError, match="empty problem"):
        Q.i8_gemm(A, B, None, None, out_dtype=torch.int32)
    # A row scale at an address that is not a multiple of 4.
    A = torch.zeros((4, 64), dtype=torch.int8, device=dev)
    s = torch.ones(8, device=dev)
    C = torch.empty((4, 4), device=dev)
    st = Q.load().phi_hip_i8_gemm(None, Q._ptr(A), 64, Q._ptr(B), 64, s.data_ptr() + 2, s.data_ptr(), 1, None,
                                  Q.F32, Q._ptr(C), Q.F32, 4, 4, 4, 64, None, 0)
    assert st == 3 and "sA is misaligned" in Q.last_error()


# ---------------------------------------------------------------- any K, any offset
# The reference serves any K > 0 at any byte offset through its dp4a kernel
# (core/runtime/compute.cpp:566-575, core/kernels/int8_gemm.cpp:136-290); here
# the register-staged MFMA kernel takes them with byte-safe loads and a
# zero-filled K tail.
def offset_view(t, off, device):
    """t's bytes copied into a device buffer at byte offset `off` (any
    alignment), viewed with t's shape and a row pitch of t.shape[1]."""
    M, K = t.shape
    buf = torch.zeros(M * K + off + 64, dtype=torch.int8, device=device)
    buf[off:off + M * K] = t.reshape(-1).to(device)
    return buf[off:off + M * K].view(M, K)


@pytest.mark.parametrize("K", [1, 32, 96, 100, 127, 3000])
@pytest.mark.parametrize("aoff,boff", [(1, 3), (0, 5), (7, 0), (16, 16)])
@pytest.mark.parametrize("out", ["i32", "f32", "bf16"])
def test_any_k_and_offsets(dev, orc, K, aoff, boff, out):
    M, N = 77, 130
    A, B = rand_i8((M, K), K + aoff), rand_i8((N, K), K + boff + 1)
    Ad, Bd = offset_view(A, aoff, dev), offset_view(B, boff, dev)
    assert (Ad.data_ptr() % 16 == 0) == (aoff % 16 == 0)
    acc = orc.gemm_i8_i32_fast(A.numpy(), B.numpy())
    if out == "i32":
        C = Q.i8_gemm(Ad, Bd, None, None, out_dtype=torch.int32)
        assert np.array_equal(C.cpu().numpy(), acc)
        return
    g = torch.Generator().manual_seed(K)
    sa = torch.rand(M, generator=g) * 0.01 + 0.001
    sb = torch.rand(N, generator=g) * 0.01 + 0.001
    bias = torch.randn(N, generator=g) * 0.02
    C = Q.i8_gemm(Ad, Bd, sa.to(dev), sb.to(dev), bias.to(dev),
                  out_dtype=torch.float32 if out == "f32" else torch.bfloat16)
    want = orc.epilogue(acc, sa.numpy(), sb.numpy(), bias.numpy(), out=out)
    got = C.cpu().numpy().view(np.uint32) if out == "f32" else u16(C)
    assert np.array_equal(got, want.view(np.uint32) if out == "f32" else want)


@pytest.mark.parametrize("M,N,K", [(256, 256, 3072), (300, 1000, 512), (1, 4, 64), (513, 777, 320)])
def test_any_k_kernel_on_aligned_shapes(dev, orc, monkeypatch, M, N, K):
    """PHI_GEMM_KERNEL=any forces the any-K kernel where the MFMA pipelines
    would run (the reference's PHI_INT8_DP4A A/B switch): same exact product."""
    monkeypatch.setenv("PHI_GEMM_KERNEL", "any")
    A, B = rand_i8((M, K), M + 1), rand_i8((N, K), N + 2)
    C = Q.i8_gemm(A.to(dev), B.to(dev), None, None, out_dtype=torch.int32)
    assert np.array_equal(C.cpu().numpy(), orc.gemm_i8_i32_fast(A.numpy(), B.numpy()))


# ---------------------------------------------------------------- two tile sizes
# Shapes whose 256 x 256 tiles leave a partial last round on 256 CUs: the
# persistent path then covers the bottom rows with 128 x 128 tiles in a second
# launch.  The default plan, each tile size alone, and the register-staged
# kernel must all give the same exact product.
MIXED_SHAPES = [(4352, 12288, 512), (4352, 9216, 768), (4352, 4352, 256), (4100, 4104, 512),
                (2304, 8192, 1024), (300, 1000, 512)]


def exact_product(A, B):
    return (A.double() @ B.double().t()).to(torch.int64)


@pytest.mark.parametrize("M,N,K", MIXED_SHAPES)
def test_tile_size_plans_exact(dev, monkeypatch, M, N, K):
    A = rand_i8((M, K), M + 3).to(dev)
    B = rand_i8((N, K), N + 5).to(dev)
    want = exact_product(A, B)
    for kern in ("persist", "persist256", "persist128", "persist:2stage", "persist256:2stage",
                 "persist128:2stage"):
        select_kernel(monkeypatch, kern)
        C = Q.i8_gemm(A, B, None, None, out_dtype=torch.int32)
        torch.cuda.synchronize()
        assert torch.equal(C.to(torch.int64), want), kern


@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_tile_size_plan_epilogue(dev, orc, monkeypatch, out):
    """The second launch's row offset reaches the row scales and the output."""
    monkeypatch.delenv("PHI_GEMM_KERNEL", raising=False)
    M, N, K = 4352, 4352, 512
    A, B = rand_i8((M, K), 41), rand_i8((N, K), 42)
    g = torch.Generator().manual_seed(43)
    sa = torch.rand(M, generator=g) * 0.05 + 0.002
    sb = torch.rand(N, generator=g) * 0.05 + 0.002
    bias = (torch.randn(N, generator=g) * 0.02).to(torch.bfloat16)
    C = Q.i8_gemm(A.to(dev), B.to(dev), sa.to(dev), sb.to(dev), bias.to(dev),
                  out_dtype=torch.bfloat16 if out == "bf16" else torch.float32)
    acc = exact_product(A.to(dev), B.to(dev)).cpu().numpy().astype(np.int32)
    want = orc.epilogue(acc, sa.numpy(), sb.numpy(), u16(bias), out=out)
    got = u16(C) if out == "bf16" else C.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, want if out == "bf16" else want.view(np.uint32))
