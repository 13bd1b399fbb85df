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


@pytest.mark.parametrize("kernel", ["auto", "persist256", "persist128", "auto:2stage", "auto:t272"])
@pytest.mark.parametrize("bias_kind", [None, "f32", "bf16"])
@pytest.mark.parametrize("M,N,K", [(64, 256, 512), (300, 1000, 1024), (4352, 3072, 512),
                                   (777, 520, 768), (300, 1000, 256)])
def test_gemm_residual_matches_epilogue_then_addmul(dev, orc, monkeypatch, kernel, bias_kind, M, N, K):
    kern, _, variant = kernel.partition(":")
    if kern == "auto":
        monkeypatch.delenv("PHI_GEMM_KERNEL", raising=False)
    else:
        monkeypatch.setenv("PHI_GEMM_KERNEL", kern)
    if variant == "2stage":
        monkeypatch.setenv("PHI_GEMM_PIPE", "0")
    else:
        monkeypatch.delenv("PHI_GEMM_PIPE", raising=False)
    # t272: the 272 x 192 kernel's gated fp32 epilogue wherever it applies
    # (K % 512 == 0); the other shapes keep the square plan.
    if variant == "t272":
        monkeypatch.setenv("PHI_GEMM_T272", "1")
    else:
        monkeypatch.delenv("PHI_GEMM_T272", raising=False)
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


@pytest.mark.parametrize("t272", ["0", "1"])
def test_gemm_residual_strided_stream(dev, orc, monkeypatch, t272):
    """A residual stream with a padded row pitch: the pad stays untouched
    (on the square plan and on the 272 x 192 kernel)."""
    monkeypatch.setenv("PHI_GEMM_T272", t272)
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


# ---------------------------------------------------------------- activations
# GELU-tanh (core/kernels/ops.cpp:83-89) and the SiLU gate
# (core/kernels/conv3d_causal.cpp:997-1013) in front of the rotation.  The
# fused prologue must equal our own unfused pair (fp32 intermediate) bit for
# bit; against the oracle the activation differs in its last bits (GELU's
# sigmoid-form evaluation, expf of the device library vs the host's libm), so
# codes may move by one step where a value sits on a rounding boundary, and
# scales by a few ulps.
ACT_SHAPES = [(1, 256), (37, 3072), (300, 1024), (129, 12288), (4, 16640), (3, 20480)]


def act_input(M, K, dtype, seed):
    x = synth.activations(M, K, seed=seed)
    return x if dtype == torch.bfloat16 else x.float() * 1.5


def close_to_oracle(q, s, qo, so):
    q = q.cpu().numpy().astype(np.int32)
    s = s.cpu().numpy()
    d = np.abs(q - qo.astype(np.int32))
    assert d.max() <= 1
    assert (d > 0).mean() <= 1e-3
    np.testing.assert_allclose(s, so, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,K", ACT_SHAPES)
def test_quant_rotate_gelu_equals_gelu_then_quantise(dev, orc, dtype, M, K):
    x = act_input(M, K, dtype, M * 7 + K).to(dev)
    q, s = Q.quant_rotate(x, act="gelu_tanh")
    h = Q.gelu_tanh(x, out=torch.empty(x.shape, dtype=torch.float32, device=dev))
    qu, su = Q.quant_rotate(h)
    torch.cuda.synchronize()
    assert torch.equal(q, qu)
    assert torch.equal(s.view(torch.int32), su.view(torch.int32))
    qo, so = orc.quantize_rows(orc.gelu_tanh(x.float().cpu().numpy()))
    close_to_oracle(q, s, qo, so)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,K", ACT_SHAPES)
@pytest.mark.parametrize("pad", [0, 256])
def test_quant_rotate_silu_equals_silu_then_quantise(dev, orc, dtype, M, K, pad):
    wide = act_input(M, 2 * K + pad, dtype, M * 5 + K).to(dev)
    gx = wide[:, :2 * K]  # row stride 2K + pad
    q, s = Q.quant_rotate(gx, act="silu_gate")
    h = Q.silu_gate(gx, out_dtype=torch.float32)
    qu, su = Q.quant_rotate(h)
    torch.cuda.synchronize()
    assert torch.equal(q, qu)
    assert torch.equal(s.view(torch.int32), su.view(torch.int32))
    qo, so = orc.quantize_rows(orc.silu_gate(gx.float().cpu().numpy()))
    close_to_oracle(q, s, qo, so)


def test_quant_rotate_act_half_even_and_qmax(dev, orc):
    x = act_input(64, 3072, torch.bfloat16, 11).to(dev)
    for rm, qmax in [(Q.ROUND_HALF_EVEN, 127.0), (Q.ROUND_HALF_AWAY, 7.0)]:
        q, s = Q.quant_rotate(x, act="gelu_tanh", round_mode=rm, qmax=qmax)
        h = Q.gelu_tanh(x, out=torch.empty(x.shape, dtype=torch.float32, device=dev))
        qu, su = Q.quant_rotate(h, round_mode=rm, qmax=qmax)
        torch.cuda.synchronize()
        assert torch.equal(q, qu) and torch.equal(s.view(torch.int32), su.view(torch.int32))
        assert int(q.abs().max()) == int(qmax)


def bf16_within_one_ulp(got_bf16, want_f32):
    """got (bf16 tensor) is want rounded to bf16, or one bf16 step from it."""
    want = torch.from_numpy(want_f32).to(torch.bfloat16)
    a = u16(got_bf16).astype(np.int32)
    b = want.view(torch.int16).numpy().view(np.uint16).astype(np.int32)
    # sign-magnitude bf16 bits -> a monotone integer line
    a = np.where(a & 0x8000, -(a & 0x7fff), a)
    b = np.where(b & 0x8000, -(b & 0x7fff), b)
    assert np.abs(a - b).max() <= 1


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("ydt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,cols", [(1, 8), (5, 13), (300, 1024), (64, 3072)])
def test_silu_gate_standalone(dev, orc, xdt, ydt, rows, cols):
    gx = act_input(rows, 2 * cols, xdt, rows + cols).to(dev)
    out = Q.silu_gate(gx, out_dtype=ydt)
    torch.cuda.synchronize()
    want = orc.silu_gate(gx.float().cpu().numpy())
    if ydt == torch.float32:
        np.testing.assert_allclose(out.cpu().numpy(), want, rtol=2e-6, atol=1e-30)
    else:
        bf16_within_one_ulp(out, want)


def test_silu_gate_scalar_path_matches_vector_path(dev):
    base = act_input(33, 2 * 1024 + 8, torch.bfloat16, 3).to(dev)
    vec = Q.silu_gate(base[:, :2048], out_dtype=torch.float32)       # 16-B aligned rows
    mis = Q.silu_gate(base[:, 1:2049], out_dtype=torch.float32)      # rows start 2 B in: scalar path
    ref = Q.silu_gate(base[:, 1:2049].contiguous(), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(mis.view(torch.int32), ref.view(torch.int32))
    assert vec.shape == mis.shape


@pytest.mark.parametrize("n", [8, 100003, 4352 * 12288 // 64 + 5])
def test_gelu_vector_tail_and_misaligned_paths_agree(dev, orc, n):
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(n + 1, generator=g) * 3).to(torch.bfloat16).to(dev)
    full = Q.gelu_tanh(x)                                    # vector chunks + tail
    mis = Q.gelu_tanh(x[1:])                                 # 2-byte offset: scalar path
    torch.cuda.synchronize()
    assert torch.equal(full[1:].view(torch.int16), mis.view(torch.int16))
    xf = x.float().cpu().numpy()
    err = np.abs(full.float().cpu().numpy() - orc.gelu_tanh(xf))
    assert np.all(err <= 2.0 ** -8 * np.abs(orc.gelu_tanh(xf)) + 4e-7 * np.abs(xf))
    inplace = x.clone()
    Q.gelu_tanh(inplace, out=inplace)
    torch.cuda.synchronize()
    assert torch.equal(inplace.view(torch.int16), full.view(torch.int16))
