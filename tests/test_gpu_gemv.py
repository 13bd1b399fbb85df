"""GPU parity: batched small-M linear (phi_hip_i8_gemv_batched) and GELU-tanh.

GEMV bar: int32 accumulators and the epilogue bit-exact with the oracle (same
contract as the GEMM).  GELU bar: the reference computes tanhf in fp32
(core/kernels/ops.cpp:83-89); device and host tanhf may differ by a few fp32
ulps, so the fp32 result is compared with rtol 2e-6 and the bf16 result within
one bf16 ulp (rel 8e-3)."""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("M", [1, 2, 5, 8])
@pytest.mark.parametrize("out", ["bf16", "f32", "i32"])
def test_gemv_batch_matches_oracle(dev, orc, M, out):
    K, N, n_items = 3072, 1000, 5
    x = synth.activations(M, K, seed=M)
    qo, so = orc.quantize_rows(u16(x))
    q8, s8 = torch.from_numpy(qo).to(dev), torch.from_numpy(so).to(dev)
    Ws = [synth.int8_weight(N, K, seed=10 + i) for i in range(n_items)]
    scales = [torch.rand(N) * 0.01 + 0.001 if i % 2 else torch.tensor([0.002]) for i in range(n_items)]
    biases = [synth.bias(N, seed=20 + i) for i in range(n_items)] if out != "i32" else None
    odt = {"bf16": torch.bfloat16, "f32": torch.float32, "i32": torch.int32}[out]
    outs = Q.gemv_batched(q8, s8, [w.to(dev) for w in Ws], [s.to(dev) for s in scales],
                          biases=None if biases is None else [b.to(dev) for b in biases],
                          out_dtype=odt)
    torch.cuda.synchronize()
    for i in range(n_items):
        acc = orc.gemm_i8_i32_fast(qo, Ws[i].numpy())
        if out == "i32":
            assert np.array_equal(outs[i].cpu().numpy(), acc)
            continue
        want = orc.epilogue(acc, so, scales[i].numpy(), u16(biases[i]), out=out)
        got = u16(outs[i]) if out == "bf16" else outs[i].cpu().numpy()
        assert np.array_equal(got.view(np.uint16 if out == "bf16" else np.uint32),
                              want.view(np.uint16 if out == "bf16" else np.uint32))


def test_gemv_ragged_k_and_many_items(dev, orc):
    """K not a multiple of 1024 (tail chunks), N not a multiple of 16, and more
    items than one launch carries (64)."""
    M, K, N, n_items = 2, 784, 37, 70
    x = synth.activations(M, 1024, seed=3)[:, :K].contiguous()
    qo, so = orc.quantize_rows(u16(x), rotate=False)
    q8, s8 = torch.from_numpy(qo).to(dev), torch.from_numpy(so).to(dev)
    Ws = [synth.int8_weight(N, K, seed=100 + i) for i in range(n_items)]
    sc = [torch.tensor([0.003]) for _ in range(n_items)]
    outs = Q.gemv_batched(q8, s8, [w.to(dev) for w in Ws], [s.to(dev) for s in sc],
                          out_dtype=torch.float32)
    torch.cuda.synchronize()
    for i in (0, 17, 47, 48, 63, 64, 69):
        acc = orc.gemm_i8_i32_fast(qo, Ws[i].numpy())
        want = orc.epilogue(acc, so, sc[i].numpy(), out="f32")
        assert np.array_equal(outs[i].cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.slow
def test_config4_sweep_shape(dev, orc):
    """The adaLN modulation batch: M=1, K=3072, N=18432, 60 distinct weights.
    Every output is checked against the same product from the GEMM path."""
    M, K, N, n_items = 1, 3072, 18432, 60
    x = synth.activations(M, K, seed=0, device=dev)
    q8, s8 = Q.quant_rotate(x)
    Ws = [synth.int8_weight(N, K, seed=200 + i, device=dev) for i in range(n_items)]
    sc = [torch.full((1,), 0.002, device=dev) for _ in range(n_items)]
    outs = Q.gemv_batched(q8, s8, Ws, sc, out_dtype=torch.int32)
    torch.cuda.synchronize()
    for i in range(0, n_items, 7):
        acc = (Ws[i].double() @ q8[0].double()).to(torch.int32)
        assert torch.equal(outs[i][0], acc)


@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float32)])
def test_gelu_tanh(dev, orc, xdt, ydt):
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(100000, generator=g) * 3).to(xdt)
    y = Q.gelu_tanh(x.to(dev), torch.empty(100000, dtype=ydt, device=dev))
    torch.cuda.synchronize()
    xf = x.float().numpy()
    want = orc.gelu_tanh(xf)
    got = y.float().cpu().numpy()
    # The kernel evaluates 0.5 (1 + tanh t) as 1 / (1 + e^(-2t)): within
    # 3e-7 |x| of the reference formula (the cancellation in 1 + tanh(t) for
    # t << 0 included); bf16 adds its rounding, at most 2^-8 relative.
    err = np.abs(got - want)
    if ydt == torch.float32:
        assert np.all(err <= 4e-7 * np.abs(xf))
    else:
        assert np.all(err <= 2.0 ** -8 * np.abs(want) + 4e-7 * np.abs(xf))
    tref = torch.nn.functional.gelu(x.float(), approximate="tanh").numpy()
    np.testing.assert_allclose(orc.gelu_tanh(x.float().numpy()), tref, rtol=1e-5, atol=1e-6)
