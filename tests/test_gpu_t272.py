"""GPU parity of the 272 x 192 persistent GEMM (i8_gemm_t272.hip).

The kernel serves problems whose rounds it costs less than the square plan
(configs 1, 2 and 3), on K-tiled or row-major operands.  Its outputs must
equal the square plan's bit for bit (PHI_GEMM_T272=0; that plan is held
bit-exact against the oracle by the other GPU tests), and at config 1 down
the oracle itself checks sampled rows of every tile row:
* forced on (PHI_GEMM_T272=1) over ragged shapes: M and N not multiples of
  the tile, partial 256-row strips of the K-tiled layout, fewer tiles than
  CUs, several tiles a workgroup (a workgroup's odd tiles walk K downward),
  K from 512 up;
* the same on row-major operands, with packed and with pitched rows;
* every output kind (bf16, fp32, int32), per-column or scalar column scales,
  no / fp32 / bf16 bias;
* the shapes the plan picks it for by itself, against the square plan in the
  same process.
"""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu

ODT = {"bf16": torch.bfloat16, "f32": torch.float32, "i32": torch.int32}


def _bits(t):
    return t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


def _operands(dev, M, N, K, seed):
    A = synth.int8_weight(M, K, seed=seed, device=dev)
    B = synth.int8_weight(N, K, seed=seed + 1, device=dev)
    sA = torch.rand(M, device=dev) * 0.01 + 1e-3
    sB = torch.rand(N, device=dev) * 0.01 + 1e-3
    return A, B, sA, sB


SHAPES = [
    (272, 192, 512),      # one tile
    (300, 200, 512),      # ragged in both, four tiles
    (100, 8, 1024),       # a partial tile, N = one 16-byte piece
    (4352, 3072, 512),    # config 1 down's tile grid at small K
    (1000, 4000, 1024),   # partial strips
    (2000, 30000, 512),   # ragged, about five tiles a workgroup (odd ones walk K downward)
    (4352, 12288, 512),   # config 1 up's grid, four tiles a workgroup
    (555, 9216, 3072),
]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("out", ["bf16", "f32", "i32"])
def test_forced_matches_row_major(dev, monkeypatch, M, N, K, out):
    A, B, sA, sB = _operands(dev, M, N, K, seed=M + N)
    bias = synth.bias(N, seed=3, device=dev)
    monkeypatch.setenv("PHI_GEMM_T272", "0")
    want = Q.i8_gemm(A, B, sA, sB, bias, out_dtype=ODT[out])
    monkeypatch.setenv("PHI_GEMM_T272", "1")
    got = Q.i8_gemm_kt(Q.pack_k_tiled(A), Q.pack_k_tiled(B), M, N, K, sA, sB, bias, out_dtype=ODT[out])
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("out", ["bf16", "f32", "i32"])
def test_forced_row_major_operands(dev, monkeypatch, M, N, K, out):
    """Row-major A and B: each DMA lane fetches its row's chunk directly; rows
    past the operand read zeros."""
    A, B, sA, sB = _operands(dev, M, N, K, seed=M + 2 * N)
    bias = synth.bias(N, seed=8, device=dev)
    monkeypatch.setenv("PHI_GEMM_T272", "0")
    want = Q.i8_gemm(A, B, sA, sB, bias, out_dtype=ODT[out])
    monkeypatch.setenv("PHI_GEMM_T272", "1")
    got = Q.i8_gemm(A, B, sA, sB, bias, out_dtype=ODT[out])
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("M,N,K,pa,pb", [(300, 200, 512, 32, 16), (1000, 4000, 1024, 512, 1536),
                                         (4352, 3072, 512, 16, 64)])
def test_forced_row_major_pitched(dev, monkeypatch, M, N, K, pa, pb):
    """Row-major operands whose rows are K + pa and K + pb bytes apart (views
    into wider buffers, the padding filled with other codes)."""
    Aw = synth.int8_weight(M, K + pa, seed=41, device=dev)
    Bw = synth.int8_weight(N, K + pb, seed=42, device=dev)
    A, B = Aw[:, :K], Bw[:, :K]
    sA = torch.rand(M, device=dev) * 0.01 + 1e-3
    sB = torch.rand(N, device=dev) * 0.01 + 1e-3
    bias = synth.bias(N, seed=9, device=dev)
    monkeypatch.setenv("PHI_GEMM_T272", "0")
    want = Q.i8_gemm(A.contiguous(), B.contiguous(), sA, sB, bias, out_dtype=torch.bfloat16)
    monkeypatch.setenv("PHI_GEMM_T272", "1")
    got = Q.i8_gemm(A, B, sA, sB, bias, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("bias_kind", ["none", "f32", "bf16"])
@pytest.mark.parametrize("scalar_sb", [False, True])
def test_epilogue_operands(dev, monkeypatch, bias_kind, scalar_sb):
    M, N, K = 600, 1000, 1024
    A, B, sA, sB = _operands(dev, M, N, K, seed=21)
    if scalar_sb:
        sB = synth.weight_scale(0.002, device=dev)
    bias = {"none": None, "f32": torch.randn(N, device=dev) * 0.02,
            "bf16": synth.bias(N, seed=4, device=dev)}[bias_kind]
    monkeypatch.setenv("PHI_GEMM_T272", "0")
    want = Q.i8_gemm(A, B, sA, sB, bias, out_dtype=torch.bfloat16)
    monkeypatch.setenv("PHI_GEMM_T272", "1")
    got = Q.i8_gemm_kt(Q.pack_k_tiled(A), Q.pack_k_tiled(B), M, N, K, sA, sB, bias, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("M,N,K", [(4352, 12288, 3072), (4352, 3072, 12288), (4352, 9216, 3072),
                                   (32760, 5120, 5120), (32760, 13824, 5120)])
def test_chosen_plan_matches_square_plan(dev, monkeypatch, M, N, K):
    """At the DiT shapes the plan takes 272 x 192 tiles by itself (config 3's
    with a partial last round); the result equals the square plan's."""
    assert Q.gemm_plan_get(M, N, K, k_tiled=True)["tile"] == Q.PLAN_TILE_272
    A, B, sA, sB = _operands(dev, M, N, K, seed=7)
    sB = synth.weight_scale(0.002, device=dev)
    bias = synth.bias(N, seed=5, device=dev)
    Ak, Bk = Q.pack_k_tiled(A), Q.pack_k_tiled(B)
    monkeypatch.setenv("PHI_GEMM_T272", "0")
    want = Q.i8_gemm_kt(Ak, Bk, M, N, K, sA, sB, bias, out_dtype=torch.bfloat16)
    monkeypatch.delenv("PHI_GEMM_T272")
    got = Q.i8_gemm_kt(Ak, Bk, M, N, K, sA, sB, bias, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))


def test_config1_down_rows_against_oracle(dev, orc):
    """The linear at config 1 down's shape (K = 12288 -> N = 3072, bf16 bias,
    bf16 out) on the plan's own choice, with the first and last row of each of
    the 16 tile rows of 272 and a stride through the rest compared bit for bit
    with the oracle: the int8 codes (unpacked from the K-tiled layout), the
    fp32 scales, the int32 accumulators of the same plan and the outputs."""
    M, K, N = 4352, 12288, 3072
    print(f"t272 config 1 down M={M} K={K} N={N}", flush=True)
    x = synth.activations(M, K, seed=31, device=dev)
    W = synth.int8_weight(N, K, seed=32, device=dev)
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=33, device=dev)
    Wk = Q.pack_k_tiled(W)
    qk = torch.empty((M * K,), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = Q.q8_linear_kt(x, Wk, N, sW, b, q8=qk, s8=s8)
    acc = Q.i8_gemm_kt(qk, Wk, M, N, K, None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    tiles = np.arange(0, M, 272)
    rows = np.unique(np.concatenate([tiles, tiles + 271, np.arange(5, M, 97)]))
    assert len(np.unique(rows // 272)) == 16
    r, k = rows[:, None], np.arange(K)[None, :]
    s, rr = r // 256, r % 256
    h = np.minimum(256, M - 256 * s)
    pos = 256 * K * s + h * 64 * (k // 64) + 64 * rr + 16 * (((k // 16) % 4) ^ ((rr // 4) % 4)) + k % 16
    q_rows = qk.cpu().numpy()[pos]

    def u16(t):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)

    ri = torch.from_numpy(rows).to(dev)
    yo, qo, so, acco = orc.q8_linear(u16(x[ri]), W.cpu().numpy(), sW.cpu().numpy(), u16(b))
    assert np.array_equal(q_rows, qo), f"{(q_rows != qo).sum()} code mismatches"
    assert np.array_equal(s8[ri].cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(acc[ri].cpu().numpy(), acco)
    got = u16(y[ri])
    assert np.array_equal(got, yo), f"{(got != yo).sum()} bf16 mismatches"


# ---------------------------------------------------------------- W4A8
W4_SHAPES = [
    (64, 256, 1024, 128),     # one partial tile row, N past one tile
    (300, 520, 3072, 128),    # ragged in both
    (130, 128, 2048, 256),    # N below one tile
    (1, 200, 1024, 64),       # one row, group = one K-step
    (777, 1032, 2048, 1024),  # group = half of K
    (4352, 9216, 1024, 128),  # config 2's tile grid, three tiles a workgroup
]


@pytest.mark.parametrize("M,N,K,group", W4_SHAPES)
@pytest.mark.parametrize("with_ws", [False, True])
def test_w4_in_lds_equals_expand_then_w8a8(dev, monkeypatch, M, N, K, group, with_ws):
    """asym_w4a8 on the 272 x 192 pipeline (codes and tables DMA'd, expanded
    in LDS; PHI_W4_T272=1 takes it also when a workspace is given) against
    expand-then-W8A8, bit for bit."""
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=M + N + K)
    cd, rd, sd, kd = codes.to(dev), s_rel.to(dev), sch.to(dev), corr.to(dev)
    x = synth.activations(M, K, seed=M, device=dev)
    q, s = Q.w4a8_expand(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    lut, s2 = Q.w4a8_prepare(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    ws = Q.w4a8_workspace(M, N, K, group, dev) if with_ws else None
    monkeypatch.setenv("PHI_W4_T272", "1")
    y = Q.w4a8_linear(x, cd, lut, s2, group=group, workspace=ws)
    monkeypatch.delenv("PHI_W4_T272")
    monkeypatch.setenv("PHI_GEMM_T272", "0")
    y_ref = Q.q8_linear(x, q, s)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


@pytest.mark.parametrize("N,K,group,pad", [(200, 1024, 128, 0), (384, 2048, 64, 16), (5, 1024, 1024, 32)])
def test_w4_pack_banded_is_the_documented_layout(dev, N, K, group, pad):
    """phi_hip_w4a8_pack_banded against the layout written out with numpy:
    code blocks (band, K-step) of 192 rows x 32 bytes, then table blocks
    (band, group) of 192 rows x 16 bytes, rows past N zero."""
    g = torch.Generator().manual_seed(N + K)
    codes = torch.randint(0, 256, (N, K // 2 + pad), generator=g, dtype=torch.uint8)
    lut = torch.randint(-127, 128, (N, K // group, 16), generator=g, dtype=torch.int8)
    got = Q.w4a8_pack_banded(codes.to(dev), lut.to(dev), k=K, group=group).cpu().numpy()
    bands, KT, G = (N + 191) // 192, K // 64, K // group
    c = np.zeros((bands * 192, K // 2), np.uint8)
    c[:N] = codes.numpy()[:, :K // 2]
    t = np.zeros((bands * 192, G, 16), np.int8)
    t[:N] = lut.numpy()
    want_c = c.reshape(bands, 192, KT, 32).transpose(0, 2, 1, 3).reshape(-1)
    want_t = t.reshape(bands, 192, G, 16).transpose(0, 2, 1, 3).reshape(-1).view(np.uint8)
    assert got.size == Q.load().phi_hip_w4a8_banded_bytes(N, K, group)
    assert np.array_equal(got, np.concatenate([want_c, want_t]))


@pytest.mark.parametrize("M,N,K,group", W4_SHAPES + [(4352, 9216, 3072, 128)])
def test_w4_banded_equals_expand_then_w8a8(dev, monkeypatch, M, N, K, group):
    """The band-packed weight on the in-LDS kernel against expand-then-W8A8,
    bit for bit (config 2's shape included)."""
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=M + 2 * N + K)
    cd, rd, sd, kd = codes.to(dev), s_rel.to(dev), sch.to(dev), corr.to(dev)
    x = synth.activations(M, K, seed=M + 1, device=dev)
    b = synth.bias(N, seed=4, device=dev)
    q, s = Q.w4a8_expand(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    lut, s2 = Q.w4a8_prepare(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    banded = Q.w4a8_pack_banded(cd, lut, k=K, group=group)
    y = Q.w4a8_linear_banded(x, banded, s2, N=N, group=group, bias=b)
    monkeypatch.setenv("PHI_GEMM_T272", "0")
    y_ref = Q.q8_linear(x, q, s, b)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


@pytest.mark.parametrize("out", ["bf16", "f32", "i32"])
@pytest.mark.parametrize("bias_kind", ["none", "f32", "bf16"])
def test_w4_in_lds_outputs_and_padded_code_rows(dev, monkeypatch, out, bias_kind):
    """Every output kind and bias, with code rows padded past K / 2 bytes."""
    M, N, K, group = 600, 776, 2048, 128
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=17)
    padded = torch.zeros((N, K // 2 + 48), dtype=torch.uint8)
    padded[:, :K // 2] = codes
    cd = padded.to(dev)[:, :K // 2]
    rd, sd, kd = s_rel.to(dev), sch.to(dev), corr.to(dev)
    x = synth.activations(M, K, seed=5, device=dev)
    q, s = Q.w4a8_expand(codes.to(dev), rd, Q.F16, sd, k=K, group=group, correction=kd)
    lut, s2 = Q.w4a8_prepare(codes.to(dev), rd, Q.F16, sd, k=K, group=group, correction=kd)
    bias = {"none": None, "f32": torch.randn(N, device=dev) * 0.02,
            "bf16": synth.bias(N, seed=6, device=dev)}[bias_kind]
    monkeypatch.setenv("PHI_W4_T272", "1")
    y = Q.w4a8_linear(x, cd, lut, s2, group=group, bias=bias, out_dtype=ODT[out])
    monkeypatch.delenv("PHI_W4_T272")
    monkeypatch.setenv("PHI_GEMM_T272", "0")
    xq, xs = Q.quant_rotate(x)
    y_ref = Q.i8_gemm(xq, q, xs, s, bias, out_dtype=ODT[out])
    torch.cuda.synchronize()
    assert torch.equal(_bits(y), _bits(y_ref))
