"""GPU: linears loaded from safetensors checkpoints through the C++ host
layer (load_quant_linear, upload_quant_linear_w4a4), run end to end
(tests/cpp/st_tool), against the oracle fed the same stored tensors.

Bar: bit-exact fp32 outputs.  int8_tensorwise: the oracle's W8A8 linear on the
stored codes and scales.  asym_w4a8_int8 / w6a8_int8: the oracle's decode +
row requantise (core/host/quant.cpp:315-389) of the stored codes, relative
scales, channel scale, codebook and correction, then the W8A8 linear.
convrot_w4a4: quantise with qmax 7, then the int4 GEMM."""
import os

import numpy as np
import pytest
import torch

import ckpt_util as C
import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _tool():
    if not os.path.exists(C.ST_TOOL):
        pytest.fail(f"{C.ST_TOOL} was not built (run __graft_entry__.build())")


def run_linear(dev, path, base, x, op="linear"):
    xf = os.path.join(os.path.dirname(path), "x.f32")
    of = os.path.join(os.path.dirname(path), "y.f32")
    x.numpy().astype(np.float32).tofile(xf)
    C.run(op, path, base, xf, x.shape[0], of)
    return np.fromfile(of, np.float32)


def np_of(t):
    if t is None:
        return None
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return t.view(torch.uint8).numpy()
    return t.numpy()


REL = {torch.float32: Q.F32, torch.float16: Q.F16, torch.bfloat16: Q.BF16,
       torch.float8_e4m3fn: Q.F8_E4M3, torch.float8_e5m2: Q.F8_E5M2, torch.uint8: Q.U8_E4M3}


def test_int8_tensorwise_checkpoint(dev, orc, tmp_path):
    N, K, M = 200, 1024, 37
    g = torch.Generator().manual_seed(5)
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = torch.rand(N, generator=g) * 0.004 + 0.001
    path = C.write(str(tmp_path / "a.safetensors"), {
        "l.weight": W, "l.weight_scale": s,
        "l.comfy_quant": C.comfy_blob({"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 256})})
    x = synth.activations(M, K, seed=6).float()
    y = run_linear(dev, path, "l", x).reshape(M, N)
    want = orc.q8_linear(x.numpy(), W.numpy(), s.numpy(), out="f32")[0]
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ["asym_w4a8_int8", "w6a8_int8"])
@pytest.mark.parametrize("rel", [torch.float16, torch.bfloat16, torch.float32, torch.float8_e4m3fn, torch.uint8])
@pytest.mark.parametrize("variant", ["plain", "codebook", "scalar_channel", "correction"])
def test_grouped_checkpoint(dev, orc, tmp_path, fmt, rel, variant):
    six = fmt == "w6a8_int8"
    if six and variant == "codebook":
        pytest.skip("six-bit weights carry no codebook")
    N, K, M, group = 136, 1024, 45, 64
    g = torch.Generator().manual_seed(K + int(six) + len(variant))
    stored = K // 2 + K // 4 if six else K // 2
    codes = torch.randint(-128, 128, (N, stored), generator=g, dtype=torch.int8)
    srel = torch.rand(N, K // group, generator=g) * 6 + 0.5
    srel = srel.to(torch.float8_e4m3fn).view(torch.uint8) if rel == torch.uint8 else srel.to(rel)
    sch = torch.rand(1 if variant == "scalar_channel" else N, generator=g) * 0.01 + 0.001
    t = {"b.weight": codes, "b.weight_s_rel": srel, "b.weight_s_channel": sch,
         "b.comfy_quant": C.comfy_blob({"format": fmt, "group_size": group, "convrot_groupsize": 256})}
    cb = torch.randn(16, generator=g) * 4 if variant == "codebook" else None
    corr = torch.randn(K // group, N, generator=g) * 0.002 if variant == "correction" else None
    if cb is not None:
        t["b.weight_codebook"] = cb
    if corr is not None:
        t["b.weight_correction"] = corr
    path = C.write(str(tmp_path / "g.safetensors"), t)
    x = synth.activations(M, K, seed=7).float()
    y = run_linear(dev, path, "b", x).reshape(M, N)
    q, s = orc.w4a8_expand(codes.view(torch.uint8).numpy(), np_of(srel), REL[rel], sch.numpy(), k=K, group=group,
                           codebook=None if cb is None else cb.numpy(),
                           correction=None if corr is None else corr.numpy(), layout=1 if six else 0)
    want = orc.q8_linear(x.numpy(), q, s, out="f32")[0]
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_convrot_w4a4_checkpoint(dev, orc, tmp_path):
    N, K, M = 96, 1024, 50
    g = torch.Generator().manual_seed(9)
    w = torch.randn(N, K, generator=g)
    packed, sw = orc.quantize_convrot_w4a4(w.numpy())
    path = C.write(str(tmp_path / "w4a4.safetensors"), {
        "te.weight": torch.from_numpy(packed.view(np.int8)), "te.weight_scale": torch.from_numpy(sw),
        "te.comfy_quant": C.comfy_blob({"format": "convrot_w4a4"})})
    x = synth.activations(M, K, seed=10).float()
    y = run_linear(dev, path, "te", x, op="int4").reshape(M, N)
    qo, so = orc.quantize_rows(x.numpy(), qmax=7.0)
    want = orc.int4_gemm(qo, packed, so, sw)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_unsupported_families_are_named(dev, tmp_path):
    xf = str(tmp_path / "x.f32")
    np.zeros((4, 256), np.float32).tofile(xf)
    dense = C.write(str(tmp_path / "d.safetensors"), {"d.weight": torch.randn(8, 256)})
    out = C.run("linear", dense, "d", xf, 4, str(tmp_path / "y.f32"), check=False)
    assert out.returncode == 3 and "F32 without a comfy_quant spec" in out.stdout
    w4a4 = C.write(str(tmp_path / "e.safetensors"), {
        "e.weight": torch.zeros(8, 128, dtype=torch.int8), "e.weight_scale": torch.ones(8),
        "e.comfy_quant": C.comfy_blob({"format": "convrot_w4a4"})})
    out = C.run("linear", w4a4, "e", xf, 4, str(tmp_path / "y.f32"), check=False)
    assert out.returncode == 3 and "upload_quant_linear_w4a4" in out.stdout
    bad = C.write(str(tmp_path / "f.safetensors"), {
        "f.weight": torch.zeros(8, 128, dtype=torch.int8), "f.weight_s_rel": torch.ones(8, 3),
        "f.comfy_quant": C.comfy_blob({"format": "asym_w4a8_int8", "group_size": 64})})
    out = C.run("linear", bad, "f", xf, 4, str(tmp_path / "y.f32"), check=False)
    assert out.returncode == 3 and "weight_s_rel is not [N, K/group]" in out.stdout
