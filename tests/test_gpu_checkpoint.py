"""GPU: linears loaded from safetensors checkpoints through the C++ host
layer (load_quant_linear, upload_quant_linear_w4a4), run end to end
(tests/cpp/st_tool), against the oracle fed the same stored tensors.

Bar: bit-exact fp32 outputs.  int8_tensorwise: the oracle's W8A8 linear on the
stored codes and scales.  asym_w4a8_int8 / w6a8_int8: the oracle's decode +
row requantise (core/host/quant.cpp:315-389) of the stored codes, relative
scales, channel scale, codebook and correction, then the W8A8 linear.
convrot_w4a4: quantise with qmax 7, then the int4 GEMM."""
import json
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
    """op "linear_kt" loads with GpuCtx::k_tiled_weights: the weight must come
    out K-tiled and linear_gemm must give the row-major path's bits."""
    xf = os.path.join(os.path.dirname(path), "x.f32")
    of = os.path.join(os.path.dirname(path), "y.f32")
    x.numpy().astype(np.float32).tofile(xf)
    out = C.run(op, path, base, xf, x.shape[0], of)
    if op == "linear_kt":
        assert '"k_tiled": true' in out.stdout, out.stdout
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


@pytest.mark.parametrize("op", ["linear", "linear_kt"])
def test_int8_tensorwise_checkpoint(dev, orc, tmp_path, op):
    N, K, M = 200, 1024, 37
    g = torch.Generator().manual_seed(5)
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = torch.rand(N, generator=g) * 0.004 + 0.001
    path = C.write(str(tmp_path / "a.safetensors"), {
        "l.weight": W, "l.weight_scale": s,
        "l.comfy_quant": C.comfy_blob({"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 256})})
    x = synth.activations(M, K, seed=6).float()
    y = run_linear(dev, path, "l", x, op=op).reshape(M, N)
    want = orc.q8_linear(x.numpy(), W.numpy(), s.numpy(), out="f32")[0]
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ["asym_w4a8_int8", "w6a8_int8"])
@pytest.mark.parametrize("rel", [torch.float16, torch.bfloat16, torch.float32, torch.float8_e4m3fn, torch.uint8])
@pytest.mark.parametrize("variant", ["plain", "codebook", "scalar_channel", "correction"])
@pytest.mark.parametrize("op", ["linear", "linear_kt"])
def test_grouped_checkpoint(dev, orc, tmp_path, fmt, rel, variant, op):
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
    y = run_linear(dev, path, "b", x, op=op).reshape(M, N)
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
    assert out.returncode == 3 and "is f32: a dense float weight runs the dense GEMM" in out.stdout
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


# ---------------------------------------------------------------- the loaders' other paths
import struct  # noqa: E402


def loaded(tmp_path, how, path, *bases, loras=()):
    """st_tool weights: the int8 weight and row scales a loader produced."""
    out = str(tmp_path / f"{how}.bin")
    args = ["weights", how, path, out, *bases]
    for lp, strength in loras:
        args += ["lora", lp, strength]
    C.run(*args)
    raw = open(out, "rb").read()
    n, k = struct.unpack("<qq", raw[:16])
    q = np.frombuffer(raw[16:16 + n * k], np.int8).reshape(n, k)
    s = np.frombuffer(raw[16 + n * k:16 + n * k + 4 * n], np.float32)
    return q, s


def int8_weight_tensors(prefix, N, K, seed, convrot=True, spec=True):
    g = torch.Generator().manual_seed(seed)
    t = {f"{prefix}.weight": torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8),
         f"{prefix}.weight_scale": torch.rand(N, generator=g) * 0.004 + 0.001}
    if spec:
        t[f"{prefix}.comfy_quant"] = C.comfy_blob({"format": "int8_tensorwise", "convrot": convrot,
                                                   "convrot_groupsize": 256})
    return t


def dequant_i8(t, prefix):
    """SafeTensors::dequant_rows of an int8 weight: (float)q * s per row."""
    return t[f"{prefix}.weight"].numpy().astype(np.float32) * t[f"{prefix}.weight_scale"].numpy()[:, None]


def grouped_weight_tensors(prefix, N, K, group, seed):
    g = torch.Generator().manual_seed(seed)
    return {f"{prefix}.weight": torch.randint(-128, 128, (N, K // 2), generator=g, dtype=torch.int8),
            f"{prefix}.weight_s_rel": (torch.rand(N, K // group, generator=g) * 6 + 0.5).to(torch.float16),
            f"{prefix}.weight_s_channel": torch.rand(N, generator=g) * 0.01 + 0.001,
            f"{prefix}.comfy_quant": C.comfy_blob({"format": "asym_w4a8_int8", "group_size": group,
                                                   "convrot_groupsize": 256})}


def oracle_grouped(orc, t, prefix, K, group):
    return orc.w4a8_expand(t[f"{prefix}.weight"].view(torch.uint8).numpy(),
                           t[f"{prefix}.weight_s_rel"].view(torch.int16).numpy().view(np.uint16), Q.F16,
                           t[f"{prefix}.weight_s_channel"].numpy(), k=K, group=group)


@pytest.mark.parametrize("how", ["load3", "load3_kt"])
def test_load3_int8_concatenates(dev, tmp_path, how):
    """Three int8_tensorwise weights: rows q then k then v, scales likewise,
    verbatim (core/models/model_common.cpp:1457-1480); load3_kt stores the
    stacked matrix K-tiled, which unpacks to the same bytes."""
    K = 512
    t = {**int8_weight_tensors("a.to_q", 96, K, 1), **int8_weight_tensors("a.to_k", 32, K, 2),
         **int8_weight_tensors("a.to_v", 64, K, 3)}
    path = C.write(str(tmp_path / "qkv.safetensors"), t)
    q, s = loaded(tmp_path, how, path, "a.to_q", "a.to_k", "a.to_v")
    want_q = np.concatenate([t[f"a.to_{x}.weight"].numpy() for x in "qkv"])
    want_s = np.concatenate([t[f"a.to_{x}.weight_scale"].numpy() for x in "qkv"])
    assert np.array_equal(q, want_q) and np.array_equal(s.view(np.uint32), want_s.view(np.uint32))


@pytest.mark.parametrize("how", ["load3", "load3_kt"])
def test_load3_grouped_and_mixed(dev, orc, tmp_path, how):
    """Grouped q|k|v: each part's rows are its decode + row requantise; a plain
    int8 part among them is decoded and requantised without a rotation (the
    requant spec of a stored-rotated base_q), as the reference's requant path."""
    K, group = 1024, 128
    t = {**grouped_weight_tensors("b.q", 64, K, group, 4), **grouped_weight_tensors("b.k", 32, K, group, 5),
         **grouped_weight_tensors("b.v", 48, K, group, 6)}
    path = C.write(str(tmp_path / "g.safetensors"), t)
    q, s = loaded(tmp_path, how, path, "b.q", "b.k", "b.v")
    parts = [oracle_grouped(orc, t, x, K, group) for x in ("b.q", "b.k", "b.v")]
    assert np.array_equal(q, np.concatenate([p[0] for p in parts]))
    assert np.array_equal(s.view(np.uint32), np.concatenate([p[1] for p in parts]).view(np.uint32))
    t2 = {**grouped_weight_tensors("c.q", 64, K, group, 7), **int8_weight_tensors("c.k", 40, K, 8),
          **grouped_weight_tensors("c.v", 48, K, group, 9)}
    path = C.write(str(tmp_path / "m.safetensors"), t2)
    q, s = loaded(tmp_path, how, path, "c.q", "c.k", "c.v")
    qk, sk = orc.quantize_rows(dequant_i8(t2, "c.k"), rotate=False)
    assert np.array_equal(q[64:104], qk) and np.array_equal(s[64:104].view(np.uint32), sk.view(np.uint32))
    qq, sq = oracle_grouped(orc, t2, "c.q", K, group)
    assert np.array_equal(q[:64], qq) and np.array_equal(s[:64].view(np.uint32), sq.view(np.uint32))


@pytest.mark.parametrize("src", ["int8_convrot", "int8_plain", "int8_nospec", "bf16", "f16", "f32",
                                 "f32_rotated", "grouped"])
def test_upload_quant_linear_i8(dev, orc, tmp_path, src):
    """The streaming upload's three paths (core/models/model_common.cpp:1095-1283):
    a grouped weight expanded, an int8 weight whose file declares convrot
    verbatim, anything else decoded and requantised (rotated unless the file
    says it is stored rotated)."""
    N, K = 72, 768
    g = torch.Generator().manual_seed(11)
    if src.startswith("int8"):
        t = int8_weight_tensors("u", N, K, 12, convrot=src == "int8_convrot", spec=src != "int8_nospec")
        vals, rotated = dequant_i8(t, "u"), src == "int8_convrot"
    elif src == "grouped":
        t = grouped_weight_tensors("u", N, K, 128, 13)
    else:
        dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32, "f32_rotated": torch.float32}[src]
        w = (torch.randn(N, K, generator=g) * 0.05).to(dt)
        t = {"u.weight": w}
        if src == "f32_rotated":
            t["u.comfy_quant"] = C.comfy_blob({"format": "int8_tensorwise", "convrot": True})
        vals, rotated = w.float().numpy(), src == "f32_rotated"
    path = C.write(str(tmp_path / "u.safetensors"), t)
    q, s = loaded(tmp_path, "upload_i8", path, "u")
    if src == "grouped":
        wq, ws = oracle_grouped(orc, t, "u", K, 128)
    elif src == "int8_convrot":
        wq, ws = t["u.weight"].numpy(), t["u.weight_scale"].numpy()
    else:
        wq, ws = orc.quantize_rows(vals, rotate=not rotated)
    assert np.array_equal(q, wq) and np.array_equal(s.view(np.uint32), ws.view(np.uint32))


def test_bare_int4_weight(dev, orc, tmp_path):
    """A bare I4 tensor (no comfy_quant): two signed nibbles a byte times the
    row scale, then the requantiser with a rotation (core/host/st.cpp:636-656)."""
    N, K = 40, 512
    g = torch.Generator().manual_seed(14)
    packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    sc = torch.rand(N, generator=g) * 0.01 + 0.001
    path = C.write_raw(str(tmp_path / "i4.safetensors"), [
        ("n.weight", "I4", (N, K // 2), packed.numpy().tobytes()),
        ("n.weight_scale", "F32", (N,), sc.numpy().tobytes())])
    q, s = loaded(tmp_path, "load", path, "n")
    p = packed.numpy().astype(np.int32)
    nib = np.stack([p & 15, p >> 4], axis=2).reshape(N, K)
    vals = np.where(nib >= 8, nib - 16, nib).astype(np.float32) * sc.numpy()[:, None]
    wq, ws = orc.quantize_rows(vals, rotate=True)
    assert np.array_equal(q, wq) and np.array_equal(s.view(np.uint32), ws.view(np.uint32))


def lora_tensors(prefix, n, k, r, seed, zero_row=None):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(r, k, generator=g) * 0.05
    B = torch.randn(n, r, generator=g) * 0.05
    if zero_row is not None:
        B[zero_row, :] = 0.0
    return {f"{prefix}.lora_A.weight": A, f"{prefix}.lora_B.weight": B}, A.numpy(), B.numpy()


def fold(w, A, B, scale):
    """w[o][i] += (scale * B[o][r]) * A[r][i], r ascending, B == 0 skipped,
    every product and sum rounded to fp32 (core/models/lora.cpp:182-201)."""
    w = w.copy()
    scale = np.float32(scale)
    for r in range(A.shape[0]):
        s = (scale * B[:, r]).astype(np.float32)
        upd = (w + (s[:, None] * A[r][None, :]).astype(np.float32)).astype(np.float32)
        w = np.where((B[:, r] != 0)[:, None], upd, w)
    return w


def lora_scale(strength, alpha, rank):
    return np.float32(np.float32(np.float32(strength) * np.float32(alpha)) / np.float32(rank))


@pytest.mark.parametrize("how", ["load", "load_kt"])
@pytest.mark.parametrize("convrot", [True, False])
def test_lora_fold_load_quant_linear(dev, orc, tmp_path, convrot, how):
    """load_quant_linear with a LoRA that touches the module: decode, rotate
    back to the original basis, add the deltas file by file, rotate and
    quantise (core/models/model_common.cpp:1011-1030); load_kt stores the
    result K-tiled, which unpacks to the same bytes."""
    N, K, r = 64, 512, 8
    t = int8_weight_tensors("blk.attn", N, K, 15, convrot=convrot)
    path = C.write(str(tmp_path / "w.safetensors"), t)
    f1, A1, B1 = lora_tensors("blk.attn", N, K, r, 16, zero_row=3)
    f2, A2, B2 = lora_tensors("diffusion_model.blk.attn", N, K, 4, 17)
    l1 = C.lora_file(str(tmp_path / "l1.safetensors"), f1)
    l2 = C.lora_file(str(tmp_path / "l2.safetensors"), f2, metadata={"lora_alpha": "2"})
    q, s = loaded(tmp_path, how, path, "blk.attn", loras=((l1, 0.7), (l2, 1.5)))
    w = dequant_i8(t, "blk.attn")
    if convrot:
        w = orc.convrot(w)
    w = fold(w, A1, B1, lora_scale(0.7, r, r))
    w = fold(w, A2, B2, lora_scale(1.5, 2.0, 4))
    wq, ws = orc.quantize_rows(w, rotate=True)
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(q, wq), f"{(q != wq).sum()} code mismatches"
    # A LoRA for another module leaves the weight verbatim.
    f3, _, _ = lora_tensors("blk.mlp", N, K, r, 18)
    l3 = C.lora_file(str(tmp_path / "l3.safetensors"), f3)
    q, s = loaded(tmp_path, how, path, "blk.attn", loras=((l3, 1.0),))
    if convrot:
        assert np.array_equal(q, t["blk.attn.weight"].numpy())


def test_lora_fold_upload_and_load3(dev, orc, tmp_path):
    """upload_quant_linear_i8 folds slab by slab (rotate back a stored-rotated
    weight, add, rotate and quantise); load_quant3_linear folds each part in its
    original basis and quantises the stack with base_q's requant spec, which
    for a stored-rotated checkpoint does not rotate again
    (core/models/model_common.cpp:1160-1216, :1486-1503)."""
    N, K, r = 48, 512, 4
    t = {**int8_weight_tensors("x.q", N, K, 19), **int8_weight_tensors("x.k", N, K, 20),
         **int8_weight_tensors("x.v", N, K, 21)}
    path = C.write(str(tmp_path / "w.safetensors"), t)
    fq, Aq, Bq = lora_tensors("x.q", N, K, r, 22)
    fv, Av, Bv = lora_tensors("x.v", N, K, r, 23)
    lp = C.lora_file(str(tmp_path / "l.safetensors"), {**fq, **fv})
    q, s = loaded(tmp_path, "upload_i8", path, "x.q", loras=((lp, 1.0),))
    w = fold(orc.convrot(dequant_i8(t, "x.q")), Aq, Bq, lora_scale(1.0, r, r))
    wq, ws = orc.quantize_rows(w, rotate=True)
    assert np.array_equal(q, wq) and np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    q, s = loaded(tmp_path, "load3", path, "x.q", "x.k", "x.v", loras=((lp, 1.0),))
    parts = [fold(orc.convrot(dequant_i8(t, "x.q")), Aq, Bq, lora_scale(1.0, r, r)),
             orc.convrot(dequant_i8(t, "x.k")),
             fold(orc.convrot(dequant_i8(t, "x.v")), Av, Bv, lora_scale(1.0, r, r))]
    wq, ws = orc.quantize_rows(np.concatenate(parts), rotate=False)
    assert np.array_equal(q, wq) and np.array_equal(s.view(np.uint32), ws.view(np.uint32))


def test_load_lora_tail_layout(dev, tmp_path):
    """load_lora_tail over a fused q|k|v: A stacked along the rank axis, B
    placed at each module's output rows with its scale folded in
    (core/models/model_common.cpp:1587-1652)."""
    n1, k = 32, 256
    fq, Aq, Bq = lora_tensors("blocks.0.attn.to_q", n1, k, 4, 24)
    fv, Av, Bv = lora_tensors("blocks.0.attn.to_v", n1, k, 2, 25)
    lp = C.lora_file(str(tmp_path / "l.safetensors"), {**fq, **fv})
    out = str(tmp_path / "tail.bin")
    res = json.loads(C.run("tail", out, 3 * n1, k, f"blocks.0.attn.to_q:0:{n1}", f"blocks.0.attn.to_k:{n1}:{n1}",
                           f"blocks.0.attn.to_v:{2 * n1}:{n1}", "lora", lp, 0.5).stdout)
    assert res["rank"] == 6 and res["touches"]
    raw = open(out, "rb").read()
    rank = struct.unpack("<q", raw[:8])[0]
    at = np.frombuffer(raw[8:8 + rank * k * 4], np.float32).reshape(rank, k)
    bt = np.frombuffer(raw[8 + rank * k * 4:], np.float32).reshape(3 * n1, rank)
    assert np.array_equal(at, np.concatenate([Aq, Av]))
    want = np.zeros((3 * n1, rank), np.float32)
    want[:n1, :4] = lora_scale(0.5, 4, 4) * Bq
    want[2 * n1:, 4:] = lora_scale(0.5, 2, 2) * Bv
    assert np.array_equal(bt, want)


# ---------------------------------------------------------------- fp8 and nvfp4 / mxfp4 weights
def _to_blocked(scales: np.ndarray) -> np.ndarray:
    """The cuBLAS tiled block-scale layout (as tests/test_oracle_fp4.py builds it)."""
    rows, cols = scales.shape
    R, Cc = -(-rows // 128) * 128, -(-cols // 4) * 4
    pad = np.zeros((R, Cc), scales.dtype)
    pad[:rows, :cols] = scales
    t = pad.reshape(R // 128, 128, Cc // 4, 4).transpose(0, 2, 1, 3).reshape(-1, 4, 32, 4).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(t.reshape(R, Cc))


def _e4m3_codes(g, shape, lo=0x20, hi=0x58):
    """Positive finite E4M3 codes (scale values about 0.03 to 20)."""
    return torch.randint(lo, hi, shape, generator=g, dtype=torch.int32).to(torch.uint8)


@pytest.mark.parametrize("fmt,block", [("nvfp4", 16), ("mxfp4", 32)])
def test_dequant_fp4_rows_c_abi(dev, orc, fmt, block):
    """phi_hip_dequant_fp4_rows against the oracle bit for bit, a slice from a
    row past the first 128-row tile included (the table is indexed by the
    weight's own row), and a table too small for the rows asked is refused."""
    N, K = 300, 1024
    g = torch.Generator().manual_seed(21 + block)
    codes = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    table8 = _to_blocked(_e4m3_codes(g, (N, K // block)).numpy())
    table = torch.from_numpy(table8).view(torch.float8_e4m3fn).float()
    glob = torch.rand(N, generator=g) + 0.5
    got = Q.dequant_fp4_rows(codes.to(dev), K, table.to(dev), block=block, global_scale=glob.to(dev))
    want = orc.dequant_fp4_rows(codes.numpy(), K, table8, orc.U8_E4M3, block, glob.numpy())
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    r0 = 130
    part = Q.dequant_fp4_rows(codes[r0:].to(dev), K, table.to(dev), block=block, global_scale=glob[:1].to(dev),
                              row0=r0)
    want_p = orc.dequant_fp4_rows(codes[r0:].numpy(), K, table8, orc.U8_E4M3, block, glob.numpy()[:1], row0=r0)
    assert np.array_equal(part.cpu().numpy().view(np.uint32), want_p.view(np.uint32))
    with pytest.raises(RuntimeError, match="block-scale table does not cover"):
        Q.dequant_fp4_rows(codes.to(dev), K, table[:128].contiguous().to(dev), block=block)


@pytest.mark.parametrize("dtype", ["e4m3", "e5m2"])
def test_dequant_fp8_rows_c_abi(dev, orc, dtype):
    g = torch.Generator().manual_seed(31)
    codes = torch.randint(0, 256, (64, 512), generator=g, dtype=torch.int32).to(torch.uint8)
    sc = torch.rand(64, generator=g) * 0.01 + 0.001
    kind = Q.F8_E4M3 if dtype == "e4m3" else Q.F8_E5M2
    for scale in (sc, sc[:1], None):
        got = Q.dequant_rows(codes.to(dev), kind, 512, None if scale is None else scale.to(dev)).cpu().numpy()
        want = orc.dequant_fp8_rows(codes.numpy(), orc.F8_E4M3 if dtype == "e4m3" else orc.F8_E5M2,
                                    None if scale is None else scale.numpy())
        assert np.array_equal(np.isnan(got), np.isnan(want))
        ok = ~np.isnan(want)
        assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


@pytest.mark.parametrize("variant", ["e4m3_rows", "e4m3_scalar", "e5m2_none", "e4m3_spec"])
def test_upload_fp8_weight(dev, orc, tmp_path, variant):
    """An fp8 checkpoint through the streaming int8 upload: each code decoded
    times the optional row scale (core/host/st.cpp:610-621), then rotated and
    quantised per row (core/models/model_common.cpp:1095-1283)."""
    N, K = 200, 512
    g = torch.Generator().manual_seed(41)
    e5 = variant.startswith("e5m2")
    tdt = torch.float8_e5m2 if e5 else torch.float8_e4m3fn
    lo, hi = (0x20, 0x50) if e5 else (0x20, 0x58)
    codes = torch.randint(lo, hi, (N, K), generator=g, dtype=torch.int32).to(torch.uint8)
    codes |= (torch.randint(0, 2, (N, K), generator=g, dtype=torch.int32) << 7).to(torch.uint8)  # signs
    t = {"f.weight": codes.view(tdt)}
    scale = None
    if variant == "e4m3_rows":
        scale = torch.rand(N, generator=g) * 0.01 + 0.001
    elif variant in ("e4m3_scalar", "e4m3_spec"):
        scale = torch.tensor([0.004])
    if scale is not None:
        t["f.weight_scale"] = scale
    if variant == "e4m3_spec":
        t["f.comfy_quant"] = C.comfy_blob({"format": "float8_e4m3fn"})
    path = C.write(str(tmp_path / "f8.safetensors"), t)
    q, s = loaded(tmp_path, "upload_i8", path, "f")
    vals = orc.dequant_fp8_rows(codes.numpy(), orc.F8_E5M2 if e5 else orc.F8_E4M3,
                                None if scale is None else scale.numpy())
    wq, ws = orc.quantize_rows(vals, rotate=True)
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(q, wq), f"{(q != wq).sum()} code mismatches"


@pytest.mark.parametrize("variant", ["nvfp4", "nvfp4_swapped", "nvfp4_f8_table", "mxfp4", "nvfp4_no_global"])
def test_upload_fp4_weight(dev, orc, tmp_path, variant):
    """An nvfp4 / mxfp4 checkpoint through the streaming int8 upload: E2M1
    codes times the tiled block table and the global scale (core/host/st.cpp:
    465-503, with the scale-name mapping of :850-880), then rotated and
    quantised per row.  200 rows: the table's last row tile is partial."""
    N, K = 200, 1024
    block = 32 if variant == "mxfp4" else 16
    g = torch.Generator().manual_seed(51 + len(variant))
    codes = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    table8 = _to_blocked(_e4m3_codes(g, (N, K // block)).numpy())
    table_t = torch.from_numpy(table8)
    if variant == "nvfp4_f8_table":
        table_t = table_t.view(torch.float8_e4m3fn)
    glob = torch.tensor(0.37)  # a 0-dim scalar, as ComfyUI writes it
    fmt = "mxfp4" if variant == "mxfp4" else "nvfp4"
    t = {"p.weight": codes, "p.comfy_quant": C.comfy_blob({"format": fmt, "group_size": block})}
    if variant == "nvfp4_swapped":
        t["p.weight_scale_2"], t["p.weight_scale"] = table_t, glob
    else:
        t["p.weight_scale"] = table_t
        if variant != "nvfp4_no_global":
            t["p.weight_scale_2"] = glob
    path = C.write(str(tmp_path / "fp4.safetensors"), t)
    p = C.probe(path, "p")
    assert p["k"] == K and p["packed"] and p["known"]
    q, s = loaded(tmp_path, "upload_i8", path, "p")
    gl = None if variant == "nvfp4_no_global" else np.full(1, 0.37, np.float32)
    vals = orc.dequant_fp4_rows(codes.numpy(), K, table8, orc.U8_E4M3, block, gl)
    wq, ws = orc.quantize_rows(vals, rotate=True)
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(q, wq), f"{(q != wq).sum()} code mismatches"
