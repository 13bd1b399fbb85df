"""GPU parity: the runtime LoRA correction out += (x A^T) B^T
(phi_hip_lora_down / _rank_add / _tail; apply_lora_tail
core/models/model_common.cpp:1667-1700).

Bar: bit-exact with the oracle, whose fp32 fma chains follow the reference's
order (k ascending from 0 for h, r ascending from out's value for the
update); the oracle itself is pinned by an exact-rational emulation of those
chains (tests/test_oracle_lora.py)."""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


def factors(M, K, R, N, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    A = torch.randn(R, K, generator=g) * 0.05
    B = torch.randn(N, R, generator=g) * 0.05
    out = torch.randn(M, N, generator=g)
    return x, A, B, out


def bits(t):
    return t.cpu().contiguous().view(torch.int32).numpy()


@pytest.mark.parametrize("tr", ["1", "2", "4"])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,K,R", [(1, 256, 1), (37, 72, 17), (300, 3072, 64), (129, 1000, 256), (65, 33, 33),
                                   (70, 640, 37)])
def test_lora_down_bit_exact(dev, orc, monkeypatch, tr, xdt, M, K, R):
    """tr: ranks per wave of the main form (the PHI_LORA_TR A/B switch); the
    shapes with K % 64 == 0 take the main form, the others the general one."""
    monkeypatch.setenv("PHI_LORA_TR", tr)
    x, A, _, _ = factors(M, K, R, 1, M + K + R)
    x = x.to(xdt)
    h = Q.lora_down(x.to(dev), A.to(dev))
    torch.cuda.synchronize()
    want = orc.lora_down(x.float().numpy(), A.numpy())
    assert np.array_equal(bits(h), want.view(np.int32))


@pytest.mark.parametrize("cdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,R", [(1, 1, 1), (37, 1000, 17), (300, 513, 64), (129, 256, 256), (200, 130, 33)])
def test_lora_rank_add_bit_exact(dev, orc, cdt, M, N, R):
    g = torch.Generator().manual_seed(M * N + R)
    h = torch.randn(M, R, generator=g)
    B = torch.randn(N, R, generator=g) * 0.1
    C = torch.randn(M, N, generator=g).to(cdt)
    Cd = C.to(dev)
    Q.lora_rank_add(h.to(dev), B.to(dev), Cd)
    torch.cuda.synchronize()
    want = orc.lora_rank_add(h.numpy(), B.numpy(), C.float().numpy())
    if cdt == torch.float32:
        assert np.array_equal(bits(Cd), want.view(np.int32))
    else:
        assert torch.equal(Cd.cpu().view(torch.int16), torch.from_numpy(want).to(torch.bfloat16).view(torch.int16))


def test_lora_rank_add_strided_c(dev, orc):
    M, N, R, ldc = 70, 300, 16, 320
    g = torch.Generator().manual_seed(5)
    h, B = torch.randn(M, R, generator=g), torch.randn(N, R, generator=g)
    wide = torch.randn(M, ldc, generator=g)
    Cd = wide.to(dev)
    Q.lora_rank_add(h.to(dev), B.to(dev), Cd[:, :N])
    torch.cuda.synchronize()
    want = orc.lora_rank_add(h.numpy(), B.numpy(), wide[:, :N].numpy())
    got = Cd.cpu()
    assert np.array_equal(got[:, :N].contiguous().view(torch.int32).numpy(), want.view(np.int32))
    assert torch.equal(got[:, N:], wide[:, N:])  # the padding columns are untouched


def test_lora_tail_after_the_linear(dev, orc):
    """The reference's order: linear_gemm writes fp32 out, apply_lora_tail adds
    the correction (core/models/image_dit.cpp:955-960)."""
    M, K, N, R = 333, 1024, 640, 24
    x = synth.activations(M, K, seed=31).float()
    W = synth.int8_weight(N, K, seed=32)
    sW = torch.rand(N, generator=torch.Generator().manual_seed(33)) * 0.002 + 0.001
    _, A, B, _ = factors(M, K, R, N, 34)
    xd = x.to(dev)
    y = Q.q8_linear(xd, W.to(dev), sW.to(dev), out_dtype=torch.float32)
    h = torch.empty((M, R), dtype=torch.float32, device=dev)
    Q.lora_tail(xd, A.to(dev), B.to(dev), y, h=h)
    torch.cuda.synchronize()
    y0 = orc.q8_linear(x.numpy(), W.numpy(), sW.numpy(), out="f32")[0]
    want = orc.lora_rank_add(orc.lora_down(x.numpy(), A.numpy()), B.numpy(), y0)
    assert np.array_equal(bits(y), want.view(np.int32))


def test_lora_tail_contract(dev):
    x = torch.randn(8, 256, device=dev)
    A, B = torch.randn(4, 256, device=dev), torch.randn(16, 4, device=dev)
    out = torch.zeros(8, 16, device=dev)
    with pytest.raises(Q.QLinearError) as e:
        Q.lora_tail(x, A, B, out, h=torch.empty(8 * 4 - 1, device=dev))
    assert "hidden-form scratch" in str(e.value)
    # an inactive tail (rank 0) leaves out alone
    L = Q.load()
    assert L.phi_hip_lora_tail(None, x.data_ptr(), Q.F32, 256, 8, 256, None, None, 0, 16, out.data_ptr(), Q.F32,
                               16, None, 0) == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0


def test_lora_tail_full_size_rows_sampled(dev, orc):
    """Config 1's up-projection with a rank-64 correction; rows sampled for the oracle."""
    M, K, N, R = 4352, 3072, 12288, 64
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(M, K, generator=g, device=dev)
    A = torch.randn(R, K, generator=g, device=dev) * 0.02
    B = torch.randn(N, R, generator=g, device=dev) * 0.02
    out = torch.randn(M, N, generator=g, device=dev)
    out0 = out.clone()
    Q.lora_tail(x, A, B, out)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 255, 256, 2049, 4095, 4096, 4351])
    xs = x[rows.to(dev)].cpu().numpy()
    want = orc.lora_rank_add(orc.lora_down(xs, A.cpu().numpy()), B.cpu().numpy(), out0[rows.to(dev)].cpu().numpy())
    assert np.array_equal(out[rows.to(dev)].cpu().contiguous().view(torch.int32).numpy(), want.view(np.int32))


def test_lora_down_both_forms_agree(dev, orc):
    """16-byte aligned rows take the row-streaming kernel; a row base 4 bytes in
    takes the LDS-tiled one.  Both run the same chains."""
    M, K, R = 130, 512, 40
    x, A, _, _ = factors(M, K + 1, R, 1, 77)
    A = A[:, :K].contiguous()
    xd = x.to(dev)
    h_vec = Q.lora_down(xd[:, :K].contiguous(), A.to(dev))
    h_gen = Q.lora_down(xd[:, 1:], A.to(dev))  # base 4 bytes in, row pitch K + 1
    torch.cuda.synchronize()
    assert np.array_equal(bits(h_vec), orc.lora_down(x[:, :K].numpy(), A.numpy()).view(np.int32))
    assert np.array_equal(bits(h_gen), orc.lora_down(x[:, 1:].contiguous().numpy(), A.numpy()).view(np.int32))
