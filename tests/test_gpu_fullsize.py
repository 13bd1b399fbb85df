"""GPU parity at the benchmark configs' full sizes, through the C ABI.

* config 1 up: the benched call (the K-tiled linear with bias) on the bench's
  own inputs, sampled rows from every 256-row strip against oracle.q8_linear.
* config 3: the fused W8A8 linear (bf16 x -> rotate + quantise -> int8 GEMM ->
  bf16) at M=32760, K=5120 for both of its shapes (N=5120 attention out-proj and
  N=13824 MLP up).  Sampled rows are compared bit for bit against the oracle
  (int8 codes, fp32 scales, int32 accumulators, bf16 outputs); every row and
  column of the int32 product is covered by the exact ABFT checksums.
* config 4: the adaLN GEMV at M=2, K=3072, N=18432 against the oracle on every
  output of several of the 60 weights.

Reference: core/host/quant.cpp:109-169 (rotate + quantise), :223-236 (GEMM),
core/kernels/int8_gemm.cpp:588-620 (epilogue), core/runtime/compute.cpp:551-684
(the two dispatchers)."""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def checksums_ok(A, B, C32):
    """sum_n C = A . (sum_n B) and sum_m C = (sum_m A) . B, exact in float64."""
    Af, Bf, Cf = A.double(), B.double(), C32.double()
    return torch.equal(Cf.sum(1), Af @ Bf.sum(0)) and torch.equal(Cf.sum(0), Bf @ Af.sum(0))


@pytest.mark.parametrize("N", [5120, 13824])
def test_config3_fused_linear(dev, orc, N):
    M, K = 32760, 5120
    print(f"config 3 fused linear M={M} K={K} N={N}", flush=True)
    x = synth.activations(M, K, seed=0, device=dev)
    W = synth.int8_weight(N, K, seed=1, device=dev)
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=2, device=dev)
    q8 = torch.empty((M, K), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = Q.q8_linear(x, W, sW, b, q8=q8, s8=s8)
    acc = Q.i8_gemm(q8, W, None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    assert checksums_ok(q8, W, acc)
    # Rows spread over every 256-row tile band, the last row included.
    rows = np.unique(np.concatenate([np.arange(0, M, 509), [M - 1, M - 256, 4095, 4096]]))
    ri = torch.from_numpy(rows).to(dev)
    qo, so = orc.quantize_rows(u16(x[ri]))
    assert np.array_equal(q8[ri].cpu().numpy(), qo)
    assert np.array_equal(s8[ri].cpu().numpy().view(np.uint32), so.view(np.uint32))
    acco = orc.gemm_i8_i32_fast(qo, W.cpu().numpy())
    assert np.array_equal(acc[ri].cpu().numpy(), acco)
    yo = orc.epilogue(acco, so, sW.cpu().numpy(), u16(b))
    assert np.array_equal(u16(y[ri]), yo)


def _k_tiled_rows(qk, rows, M, K):
    """Rows of a K-tiled int8 matrix (M rows, K columns) as a dense array: the
    byte position of (r, k) as the layout defines it."""
    r, k = rows[:, None], np.arange(K)[None, :]
    s, rr = r // 256, r % 256
    h = np.minimum(256, M - 256 * s)
    pos = 256 * K * s + h * 64 * (k // 64) + 64 * rr + 16 * (((k // 16) % 4) ^ ((rr // 4) % 4)) + k % 16
    return qk.cpu().numpy()[pos]


@pytest.mark.parametrize("N", [5120, 13824])
def test_config3_fused_linear_k_tiled(dev, orc, N):
    """Config 3's linears on K-tiled operands, the path the plan sends to
    272 x 192 tiles (13 and 35 rounds): rows from every 256-row strip against
    oracle.q8_linear (codes, scales, accumulators, bf16 outputs)."""
    M, K = 32760, 5120
    print(f"config 3 K-tiled fused linear M={M} K={K} N={N}", flush=True)
    assert Q.gemm_plan_get(M, N, K, k_tiled=True)["tile"] == Q.PLAN_TILE_272
    x = synth.activations(M, K, seed=0, device=dev)
    W = synth.int8_weight(N, K, seed=1, device=dev)
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=2, device=dev)
    Wk = Q.pack_k_tiled(W)
    qk = torch.empty((M * K,), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = Q.q8_linear_kt(x, Wk, N, sW, b, q8=qk, s8=s8)
    acc = Q.i8_gemm_kt(qk, Wk, M, N, K, None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    # a row of every fourth 256-row strip at a varying offset, both sides of
    # the first tile-row boundary, and the last (partial) tile row's first and
    # last rows
    rows = np.array([256 * s + (37 * s) % 256 for s in range(0, (M + 255) // 256, 4)] +
                    [271, 272, 120 * 272, M - 1])
    rows = np.unique(rows[rows < M])
    q_rows = _k_tiled_rows(qk, rows, M, K)
    ri = torch.from_numpy(rows).to(dev)
    yo, qo, so, acco = orc.q8_linear(u16(x[ri]), W.cpu().numpy(), sW.cpu().numpy(), u16(b))
    assert np.array_equal(q_rows, qo), f"{(q_rows != qo).sum()} code mismatches"
    assert np.array_equal(s8[ri].cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(acc[ri].cpu().numpy(), acco)
    assert np.array_equal(u16(y[ri]), yo)


def test_config1_up_benched_linear(dev, orc):
    """The call the headline bench times, on its own inputs: phi_hip_q8_linear_kt
    with the bf16 bias at M=4352, K=3072, N=12288 (weight packed K-tiled once).
    Rows sampled from all 17 256-row strips (each strip's first and last rows,
    and a stride through the rest) are compared bit for bit with oracle.q8_linear:
    the int8 codes and fp32 scales the prologue wrote (unpacked from the K-tiled
    layout), the int32 accumulators of the same kernel plan (i8_gemm_kt, int32
    out, on those codes), and the bf16 outputs."""
    M, K, N = 4352, 3072, 12288
    print(f"config 1 up benched linear M={M} K={K} N={N}", flush=True)
    x = synth.activations(M, K, seed=0, device=dev)
    W = synth.int8_weight(N, K, seed=1, device=dev)
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=2, device=dev)
    Wk = Q.pack_k_tiled(W)
    qk = torch.empty((M * K,), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = Q.q8_linear_kt(x, Wk, N, sW, b, q8=qk, s8=s8)
    acc = Q.i8_gemm_kt(qk, Wk, M, N, K, None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    strips = np.arange(0, M, 256)
    rows = np.unique(np.concatenate([strips, strips + 255, np.arange(0, M, 61), [M - 1]]))
    assert len(np.unique(rows // 256)) == 17
    q_rows = _k_tiled_rows(qk, rows, M, K)
    ri = torch.from_numpy(rows).to(dev)
    yo, qo, so, acco = orc.q8_linear(u16(x[ri]), W.cpu().numpy(), sW.cpu().numpy(), u16(b))
    assert np.array_equal(q_rows, qo), f"{(q_rows != qo).sum()} code mismatches"
    assert np.array_equal(s8[ri].cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(acc[ri].cpu().numpy(), acco)
    got = u16(y[ri])
    assert np.array_equal(got, yo), f"{(got != yo).sum()} bf16 mismatches"


@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_config4_gemv_m2(dev, orc, out):
    """M=2 timestep rows against 18432 x 3072 weights: every output of every
    seventh weight of the 60 against the oracle."""
    M, K, N, n_items = 2, 3072, 18432, 60
    x = synth.activations(M, K, seed=4)
    qo, so = orc.quantize_rows(u16(x))
    q8, s8 = torch.from_numpy(qo).to(dev), torch.from_numpy(so).to(dev)
    Ws = [synth.int8_weight(N, K, seed=300 + i, device=dev) for i in range(n_items)]
    sc = [torch.full((1,), 0.002, device=dev) if i % 2 else torch.rand(N, device=dev) * 0.01 + 1e-3
          for i in range(n_items)]
    bs = [synth.bias(N, seed=400 + i, device=dev) for i in range(n_items)]
    odt = torch.bfloat16 if out == "bf16" else torch.float32
    outs = Q.gemv_batched(q8, s8, Ws, sc, biases=bs, out_dtype=odt)
    torch.cuda.synchronize()
    for i in range(0, n_items, 7):
        acc = orc.gemm_i8_i32_fast(qo, Ws[i].cpu().numpy())
        want = orc.epilogue(acc, so, sc[i].cpu().numpy(), u16(bs[i]), out=out)
        got = u16(outs[i]) if out == "bf16" else outs[i].cpu().numpy().view(np.uint32)
        assert np.array_equal(got, want if out == "bf16" else want.view(np.uint32)), i
