"""GPU parity: grouped 4/6-bit weights (phi_hip_w4a8_expand / _prepare / _linear).

Bar: int8 codes and fp32 row scales bit-exact with the oracle's restatement of
the reference decode + requantise (core/host/quant.cpp:315-389, :134-169;
device core/kernels/w4a8_expand.cpp:151-258); the in-register W4A8 linear is
bit-exact with expand-then-W8A8 (same int32 accumulators, same bf16 bits)."""
import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def np_of(t):
    if t is None:
        return None
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    if t.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return t.cpu().view(torch.uint8).numpy()
    return t.cpu().numpy()


def rel_table(rows, groups, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    v = torch.rand((rows, groups), generator=g) * 14 + 0.25
    if dtype == Q.F32:
        return v
    if dtype == Q.F16:
        return v.to(torch.float16)
    if dtype == Q.BF16:
        return v.to(torch.bfloat16)
    if dtype == Q.F8_E4M3:
        return v.to(torch.float8_e4m3fn)
    if dtype == Q.U8_E4M3:
        return v.to(torch.float8_e4m3fn).view(torch.uint8)
    return v.to(torch.float8_e5m2)


def check_expand(dev, orc, codes, s_rel, dt, sch, *, k, group, codebook=None, correction=None,
                 layout=0):
    q, s = Q.w4a8_expand(codes.to(dev), None if s_rel is None else s_rel.to(dev), dt,
                         None if sch is None else sch.to(dev), k=k, group=group,
                         codebook=None if codebook is None else codebook.to(dev),
                         correction=None if correction is None else correction.to(dev),
                         layout=layout)
    torch.cuda.synchronize()
    qo, so = orc.w4a8_expand(codes.numpy(), np_of(s_rel), dt, np_of(sch), k=k, group=group,
                             codebook=np_of(codebook), correction=np_of(correction), layout=layout)
    assert np.array_equal(q.cpu().numpy(), qo), f"{(q.cpu().numpy() != qo).sum()} code mismatches"
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    return q, s


@pytest.mark.parametrize("dt", [Q.F32, Q.F16, Q.BF16, Q.F8_E4M3, Q.F8_E5M2, Q.U8_E4M3])
@pytest.mark.parametrize("with_cb", [False, True])
def test_nibble4_every_scale_dtype(dev, orc, dt, with_cb):
    rows, k, group = 40, 512, 32
    g = torch.Generator().manual_seed(dt * 7 + with_cb)
    codes = torch.randint(0, 256, (rows, k // 2), generator=g, dtype=torch.uint8)
    sch = torch.rand(rows, generator=g) * 0.01 + 0.001
    cb = (torch.randn(16, generator=g) * 4) if with_cb else None
    check_expand(dev, orc, codes, rel_table(rows, k // group, dt, dt), dt, sch, k=k, group=group,
                 codebook=cb)


def test_packed6(dev, orc):
    rows, k, group = 24, 768, 64
    g = torch.Generator().manual_seed(66)
    codes = torch.randint(0, 256, (rows, k // 2 + k // 4), generator=g, dtype=torch.uint8)
    sch = torch.rand(rows, generator=g) * 0.01 + 0.001
    check_expand(dev, orc, codes, rel_table(rows, k // group, Q.F32, 1), Q.F32, sch, k=k,
                 group=group, layout=1)


def test_scalar_and_missing_channel_scale(dev, orc):
    rows, k, group = 16, 256, 16
    g = torch.Generator().manual_seed(5)
    codes = torch.randint(0, 256, (rows, k // 2), generator=g, dtype=torch.uint8)
    rel = rel_table(rows, k // group, Q.F16, 2)
    check_expand(dev, orc, codes, rel, Q.F16, torch.tensor([0.004]), k=k, group=group)
    check_expand(dev, orc, codes, rel, Q.F16, None, k=k, group=group)


def test_config2_parameterisation_with_correction(dev, orc):
    """Config 2's weights (codes, fp16 per-group scale, zero point) in the
    reference's parameterisation, including the additive correction plane."""
    N, K, group = 512, 3072, 128
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=3)
    check_expand(dev, orc, codes, s_rel, Q.F16, sch, k=K, group=group, correction=corr)


def test_prepare_table_reproduces_expand(dev, orc):
    N, K, group = 256, 1024, 128
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=8)
    cd, rd, sd, kd = codes.to(dev), s_rel.to(dev), sch.to(dev), corr.to(dev)
    q, s = Q.w4a8_expand(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    lut, s2 = Q.w4a8_prepare(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    torch.cuda.synchronize()
    assert torch.equal(s.view(torch.int32), s2.view(torch.int32))
    c = codes.to(torch.int64)
    nib = torch.stack([c & 15, c >> 4], dim=2).reshape(N, K)  # low nibble = even column
    gidx = torch.arange(K) // group
    looked = lut.cpu()[torch.arange(N)[:, None], gidx[None, :], nib]
    assert torch.equal(looked, q.cpu())


@pytest.mark.parametrize("with_ws", [False, True])
@pytest.mark.parametrize("kernel", ["auto", "persist256", "persist128", "tile128"])
@pytest.mark.parametrize("M,N,K,group", [(64, 256, 1024, 128), (300, 520, 3072, 128),
                                         (1, 64, 512, 64), (130, 128, 2048, 256),
                                         (777, 1032, 768, 128), (4352, 2304, 512, 256), (640, 264, 1280, 128)])
def test_in_register_linear_equals_expand_then_w8a8(dev, monkeypatch, kernel, with_ws, M, N, K, group):
    """Every W4A8 GEMM (persistent in both tile sizes and their mix, the
    register-staged kernel, and with a workspace the expand-once path for
    many rows) against expand-then-W8A8."""
    if kernel == "auto":
        monkeypatch.delenv("PHI_GEMM_KERNEL", raising=False)
    else:
        monkeypatch.setenv("PHI_GEMM_KERNEL", kernel)
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=M + N)
    cd, rd, sd, kd = codes.to(dev), s_rel.to(dev), sch.to(dev), corr.to(dev)
    x = synth.activations(M, K, seed=M, device=dev)
    q, s = Q.w4a8_expand(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    lut, s2 = Q.w4a8_prepare(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    ws = Q.w4a8_workspace(M, N, K, group, dev) if with_ws else None
    y = Q.w4a8_linear(x, cd, lut, s2, group=group, workspace=ws)
    monkeypatch.delenv("PHI_GEMM_KERNEL", raising=False)
    y_ref = Q.q8_linear(x, q, s)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


@pytest.mark.parametrize("M,N,K,group", [(600, 520, 3072, 128), (777, 1032, 768, 128), (4352, 2304, 512, 256),
                                         (640, 264, 1280, 128)])
def test_expand_once_row_major_switch(dev, monkeypatch, M, N, K, group):
    """The expand-once path (512 rows and more) with its operands row-major (PHI_GEMM_KT=0),
    and K-tiled with the expansion in its own launch (PHI_W4_FUSE=0) instead of beside the
    prologue, gives the bits of its K-tiled default and of expand-then-W8A8."""
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=M + N + 1)
    cd, rd, sd, kd = codes.to(dev), s_rel.to(dev), sch.to(dev), corr.to(dev)
    x = synth.activations(M, K, seed=M + 1, device=dev)
    q, s = Q.w4a8_expand(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    lut, s2 = Q.w4a8_prepare(cd, rd, Q.F16, sd, k=K, group=group, correction=kd)
    ws = Q.w4a8_workspace(M, N, K, group, dev)
    assert ws is not None
    y_kt = Q.w4a8_linear(x, cd, lut, s2, group=group, workspace=ws)
    monkeypatch.setenv("PHI_GEMM_KT", "0")
    y_row = Q.w4a8_linear(x, cd, lut, s2, group=group, workspace=ws)
    monkeypatch.delenv("PHI_GEMM_KT")
    ws.fill_(0)
    monkeypatch.setenv("PHI_W4_FUSE", "0")
    y_sep = Q.w4a8_linear(x, cd, lut, s2, group=group, workspace=ws)
    monkeypatch.delenv("PHI_W4_FUSE")
    y_ref = Q.q8_linear(x, q, s)
    torch.cuda.synchronize()
    assert torch.equal(y_kt.view(torch.int16), y_ref.view(torch.int16))
    assert torch.equal(y_row.view(torch.int16), y_ref.view(torch.int16))
    assert torch.equal(y_sep.view(torch.int16), y_ref.view(torch.int16))


@pytest.mark.slow
def test_config2_full_size(dev, orc):
    """M=4352, K=3072, N=9216, group 128: in-register path vs expand + W8A8,
    and the expand vs the oracle on a row sample."""
    M, N, K, group = 4352, 9216, 3072, 128
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=3, device=dev)
    x = synth.activations(M, K, seed=0, device=dev)
    q, s = Q.w4a8_expand(codes, s_rel, Q.F16, sch, k=K, group=group, correction=corr)
    lut, s2 = Q.w4a8_prepare(codes, s_rel, Q.F16, sch, k=K, group=group, correction=corr)
    y_ref = Q.q8_linear(x, q, s)
    y = Q.w4a8_linear(x, codes, lut, s2, group=group)
    y_ws = Q.w4a8_linear(x, codes, lut, s2, group=group, workspace=Q.w4a8_workspace(M, N, K, group, dev))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    assert torch.equal(y_ws.view(torch.int16), y_ref.view(torch.int16))
    rows = torch.arange(0, N, 577)
    qo, so = orc.w4a8_expand(np_of(codes[rows]), np_of(s_rel[rows]), Q.F16, np_of(sch[rows]),
                             k=K, group=group, correction=np_of(corr[:, rows]))
    assert np.array_equal(q[rows].cpu().numpy(), qo)
    assert np.array_equal(s[rows].cpu().numpy().view(np.uint32), so.view(np.uint32))


def test_contract_errors(dev):
    codes = torch.zeros((4, 100), dtype=torch.uint8, device=dev)
    rel = torch.ones((4, 4), dtype=torch.float32, device=dev)
    with pytest.raises(Q.QLinearError, match="not a multiple of group"):
        Q.w4a8_expand(codes, rel, Q.F32, None, k=200, group=64)
    with pytest.raises(Q.QLinearError, match="packed bytes"):
        Q.w4a8_expand(torch.zeros((4, 50), dtype=torch.uint8, device=dev), rel, Q.F32, None,
                      k=128, group=32)
    with pytest.raises(Q.QLinearError, match="codebook"):
        Q.w4a8_expand(codes, rel, Q.F32, None, k=128, group=32, layout=1,
                      codebook=torch.zeros(16, device=dev))
