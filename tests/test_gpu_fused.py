"""GPU parity: the linear's fused neighbours.

phi_hip_quant_rotate_mod (adaLN ModAdd in front of the rotation) and
phi_hip_i8_gemm_residual (gated residual AddMul behind the epilogue) against
the oracle's unfused sequence (oracle.mod_add -> quantize_rows; epilogue ->
oracle.add_mul), bit for bit: int8 codes, fp32 scales and the fp32 residual
stream.  The sequence is the reference's (core/models/av_dit.cpp:1264-1267 and
:1382-1390)."""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def mods(K, seed, which="both"):
    g = torch.Generator().manual_seed(seed)
    sc = (torch.randn(K, generator=g) * 0.3) if which in ("both", "scale") else None
    sh = (torch.randn(K, generator=g) * 0.5) if which in ("both", "shift") else None
    return sc, sh


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("which", ["both", "scale", "shift"])
@pytest.mark.parametrize("M,K", [(1, 256), (37, 3072), (300, 1024), (4, 16640), (129, 5120)])
def test_quant_rotate_mod_matches_modadd_then_quantise(dev, orc, dtype, which, M, K):
    x = synth.activations(M, K, seed=M + K)
    x = x if dtype == torch.bfloat16 else x.float() * 1.5
    sc, sh = mods(K, K + 1, which)
    q, s = Q.quant_rotate(x.to(dev), mod_scale=None if sc is None else sc.to(dev),
                          mod_shift=None if sh is None else sh.to(dev))
    torch.cuda.synchronize()
    xf = x.float().numpy()
    xm = orc.mod_add(xf, None if sc is None else sc.numpy(), None if sh is None else sh.numpy())
    qo, so = orc.quantize_rows(xm)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


def test_quant_rotate_mod_zero_modulation_is_plain(dev):
    x = synth.activations(64, 3072, seed=5, device=dev)
    z = torch.zeros(3072, device=dev)
    q0, s0 = Q.quant_rotate(x)
    q1, s1 = Q.quant_rotate(x, mod_scale=z, mod_shift=z)
    assert torch.equal(q0, q1) and torch.equal(s0.view(torch.int32), s1.view(torch.int32))


@pytest.mark.parametrize("kernel", ["auto", "persist256", "persist128"])
@pytest.mark.parametrize("bias_kind", [None, "f32", "bf16"])
@pytest.mark.parametrize("M,N,K", [(64, 256, 512), (300, 1000, 1024), (4352, 3072, 512),
                                   (777, 520, 768)])
def test_gemm_residual_matches_epilogue_then_addmul(dev, orc, monkeypatch, kernel, bias_kind, M, N, K):
    if kernel == "auto":
        monkeypatch.delenv("PHI_GEMM_KERNEL", raising=False)
    else:
        monkeypatch.setenv("PHI_GEMM_KERNEL", kernel)
    g = torch.Generator().manual_seed(M * 7 + N)
    A = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    B = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 0.02 + 1e-3
    sb = torch.rand(N, generator=g) * 0.02 + 1e-3
    gate = torch.randn(N, generator=g)
    H0 = torch.randn(M, N, generator=g) * 3
    bias = None
    if bias_kind == "f32":
        bias = torch.randn(N, generator=g) * 0.02
    elif bias_kind == "bf16":
        bias = (torch.randn(N, generator=g) * 0.02).to(torch.bfloat16)
    H = H0.to(dev)
    Q.i8_gemm_residual(A.to(dev), B.to(dev), sa.to(dev), sb.to(dev),
                       None if bias is None else bias.to(dev), gate.to(dev), H)
    torch.cuda.synchronize()
    acc = orc.gemm_i8_i32_fast(A.numpy(), B.numpy())
    b_np = None if bias is None else (u16(bias) if bias.dtype == torch.bfloat16 else bias.numpy())
    lin = orc.epilogue(acc, sa.numpy(), sb.numpy(), b_np, out="f32")
    want = orc.add_mul(H0.numpy(), lin, gate.numpy())
    assert np.array_equal(H.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_gemm_residual_strided_stream(dev, orc):
    """A residual stream with a padded row pitch: the pad stays untouched."""
    M, N, K = 300, 264, 512
    g = torch.Generator().manual_seed(3)
    A = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    B = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa, sb = torch.rand(M, generator=g) * 0.02, torch.full((1,), 0.002)
    gate = torch.randn(N, generator=g)
    Hw = torch.randn(M, N + 12, generator=g)
    Hd = Hw.to(dev)
    Q.i8_gemm_residual(A.to(dev), B.to(dev), sa.to(dev), sb.to(dev), None, gate.to(dev), Hd[:, :N])
    acc = orc.gemm_i8_i32_fast(A.numpy(), B.numpy())
    lin = orc.epilogue(acc, sa.numpy(), sb.numpy(), None, out="f32")
    want = orc.add_mul(Hw[:, :N].contiguous().numpy(), lin, gate.numpy())
    got = Hd.cpu()
    assert np.array_equal(got[:, :N].contiguous().numpy().view(np.uint32), want.view(np.uint32))
    assert torch.equal(got[:, N:], Hw[:, N:])


def test_dit_attention_sublayer_chain(dev, orc):
    """The H3 block's modulate -> W8A8 projection -> gated residual, through
    the two fused entry points, against the unfused oracle sequence."""
    M, K, N = 256, 3072, 3072
    h0 = synth.activations(M, K, seed=9).float().numpy() * 2  # residual stream (fp32)
    x = synth.activations(M, K, seed=10)                       # normed input (bf16)
    W = synth.int8_weight(N, K, seed=11)
    sW = synth.weight_scale(0.002)
    sc, sh = mods(K, 12)
    gate = torch.randn(N, generator=torch.Generator().manual_seed(13))
    q8, s8 = Q.quant_rotate(x.to(dev), mod_scale=sc.to(dev), mod_shift=sh.to(dev))
    H = torch.from_numpy(h0).to(dev)
    Q.i8_gemm_residual(q8, W.to(dev), s8, sW.to(dev), None, gate.to(dev), H)
    torch.cuda.synchronize()
    qo, so = orc.quantize_rows(orc.mod_add(x.float().numpy(), sc.numpy(), sh.numpy()))
    acc = orc.gemm_i8_i32_fast(qo, W.numpy())
    lin = orc.epilogue(acc, so, sW.numpy(), None, out="f32")
    want = orc.add_mul(h0, lin, gate.numpy())
    assert np.array_equal(H.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_contract_errors(dev):
    A = torch.zeros((4, 128), dtype=torch.int8, device=dev)
    B = torch.zeros((8, 128), dtype=torch.int8, device=dev)
    s = torch.ones(8, device=dev)
    H = torch.zeros((4, 8), device=dev)
    with pytest.raises(Q.QLinearError, match="K % 256"):
        Q.i8_gemm_residual(A, B, s[:4], s, None, s, H)
    x = torch.zeros((2, 300), device=dev)
    with pytest.raises(Q.QLinearError, match="multiple of 256"):
        Q.quant_rotate(x, mod_scale=torch.zeros(300, device=dev))
