"""GPU parity: the fused W8A8 linear (phi_hip_q8_linear) and the C++ host layer.

Config 0 is checked end to end against the oracle:
int8 activations, fp32 scales, int32 accumulators and bf16 outputs bit-exact.
The config-1 MLP pair runs at full size with the GELU between the linears."""
import os
import subprocess

import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def c0_operands(device="cpu"):
    x = synth.activations(256, 3072, seed=0, device=device)
    W = synth.int8_weight(3072, 3072, seed=1, device=device)
    sW = synth.weight_scale(0.002, device=device)
    b = synth.bias(3072, seed=2, device=device)
    return x, W, sW, b


def test_config0_end_to_end(dev, orc):
    x, W, sW, b = c0_operands()
    q8 = torch.empty((256, 3072), dtype=torch.int8, device=dev)
    s8 = torch.empty((256,), dtype=torch.float32, device=dev)
    y = Q.q8_linear(x.to(dev), W.to(dev), sW.to(dev), b.to(dev), q8=q8, s8=s8)
    acc = Q.i8_gemm(q8, W.to(dev), None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    yo, qo, so, acco = orc.q8_linear(u16(x), W.numpy(), sW.numpy(), u16(b))
    assert np.array_equal(q8.cpu().numpy(), qo)
    assert np.array_equal(s8.cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(acc.cpu().numpy(), acco)
    assert np.array_equal(u16(y), yo)


@pytest.mark.parametrize("M,K,N", [(1, 256, 64), (7, 1024, 100), (300, 2048, 640)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_linear_shapes(dev, orc, M, K, N, xdt):
    x = synth.activations(M, K, seed=M + K, dtype=xdt)
    W = synth.int8_weight(N, K, seed=N)
    sW = torch.rand(N) * 0.01 + 0.001
    y = Q.q8_linear(x.to(dev), W.to(dev), sW.to(dev), out_dtype=torch.float32)
    xin = u16(x) if xdt == torch.bfloat16 else x.numpy()
    yo, _, _, _ = orc.q8_linear(xin, W.numpy(), sW.numpy(), out="f32")
    assert np.array_equal(y.cpu().numpy().view(np.uint32), yo.view(np.uint32))


@pytest.mark.slow
def test_config1_mlp_pair(dev, orc):
    """4352 tokens: up 3072->12288, GELU-tanh in bf16, down 12288->3072.
    The down projection's activation quantisation is checked bit-exact against
    the oracle on a row sample; the products by checksums."""
    M, D, H = 4352, 3072, 12288
    x = synth.activations(M, D, seed=0, device=dev)
    Wu = synth.int8_weight(H, D, seed=1, device=dev)
    Wd = synth.int8_weight(D, H, seed=4, device=dev)
    s = synth.weight_scale(0.002, device=dev)
    h = Q.q8_linear(x, Wu, s)
    g = Q.gelu_tanh(h)
    q8 = torch.empty((M, H), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = Q.q8_linear(g, Wd, s, q8=q8, s8=s8)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    rows = np.arange(0, M, 271)
    qo, so = orc.quantize_rows(u16(g[rows]))
    assert np.array_equal(q8[rows].cpu().numpy(), qo)
    assert np.array_equal(s8[rows].cpu().numpy().view(np.uint32), so.view(np.uint32))
    acc = Q.i8_gemm(q8, Wd, None, None, out_dtype=torch.int32)
    assert torch.equal(acc.double().sum(1), q8.double() @ Wd.double().sum(0))
    want = (acc.float() * s8[:, None] * s).to(torch.bfloat16)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))


def test_cpp_host_layer(dev):
    """The C++ mirror of the reference call surface (linear_gemm,
    dispatch_quant_convrot, dispatch_int8_gemm, dispatch_w4a8_expand, MediaError)
    driven by its own test program against the oracle."""
    exe = os.path.join(ROOT, "tests", "cpp", "host_layer_test")
    if not os.path.exists(exe):
        pytest.fail(f"{exe} was not built (run __graft_entry__.build())")
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
