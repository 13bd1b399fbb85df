"""CPU checks of the checkpoint readers (phi-agent_amd/host/safetensors.cpp):
the comfy_quant blob (core/host/quant.cpp:18-38), the weight-layout rules
(core/host/st.cpp:839-935), scale-table decoding, and malformed files.  The
files are written with the safetensors library (independent of this code)."""
import json
import os
import struct
import subprocess

import numpy as np
import pytest
import torch

import ckpt_util as C


@pytest.fixture(scope="module", autouse=True)
def _tool():
    if not os.path.exists(C.ST_TOOL):
        pytest.fail(f"{C.ST_TOOL} was not built (run __graft_entry__.build())")


def spec(text):
    return json.loads(C.run("spec", text).stdout)


def test_quant_spec_blob():
    s = spec('{"format": "asym_w4a8_int8", "group_size": 16, "convrot_groupsize": 256}    ')
    assert s == {"valid": True, "format": "asym_w4a8_int8", "convrot": False, "convrot_groupsize": 256,
                 "group_size": 16}
    # defaults: int8_tensorwise, convrot off, group 256 / 0
    assert spec("{}") == {"valid": True, "format": "int8_tensorwise", "convrot": False, "convrot_groupsize": 256,
                          "group_size": 0}
    s = spec('{"format": "int8_tensorwise", "convrot": true, "convrot_groupsize": -4, "group_size": -1}')
    assert s["convrot"] and s["convrot_groupsize"] == 256 and s["group_size"] == 0
    # text past the last '}' is padding; no '}' or bad JSON is an invalid spec
    assert spec('{"format": "w6a8_int8"} trailing')["format"] == "w6a8_int8"
    assert spec("no json here")["valid"] is False
    assert spec('{"format": }')["valid"] is False


def int8_file(tmp_path, N=24, K=512, scale_dtype=torch.float32, with_spec=True):
    g = torch.Generator().manual_seed(1)
    t = {"blk.0.mlp.weight": torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8),
         "blk.0.mlp.weight_scale": (torch.rand(N, generator=g) * 0.01 + 0.001).to(scale_dtype),
         "blk.0.other.bias": torch.zeros(N)}
    if with_spec:
        t["blk.0.mlp.comfy_quant"] = C.comfy_blob({"format": "int8_tensorwise", "convrot": True,
                                                    "convrot_groupsize": 256})
    return C.write(str(tmp_path / "int8.safetensors"), t), t


def test_probe_int8_tensorwise(tmp_path):
    path, t = int8_file(tmp_path)
    p = C.probe(path, "blk.0.mlp")
    assert p["tensors"] == 4 and p["dtype"] == "I8" and (p["n"], p["k"]) == (24, 512)
    assert p["plain_int8"] and not p["packed"] and p["known"] and p["bits"] == 8 and p["group"] == 0
    assert p["row_scale"] == "blk.0.mlp.weight_scale"
    assert p["spec"]["format"] == "int8_tensorwise" and p["spec"]["convrot"]
    assert np.float32(p["row_scale0"]) == t["blk.0.mlp.weight_scale"][0].item()
    # no comfy_quant sidecar: still plain int8 (codes plus a weight_scale)
    path2, _ = int8_file(tmp_path, with_spec=False)
    assert C.probe(path2, "blk.0.mlp")["plain_int8"]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_scale_tables_decode(tmp_path, dt):
    path, t = int8_file(tmp_path, scale_dtype=dt)
    p = C.probe(path, "blk.0.mlp")
    assert np.float32(p["row_scale0"]) == np.float32(t["blk.0.mlp.weight_scale"][0].float().item())


def grouped_tensors(N, K, group, fmt, *, codebook=False, channel="s_channel", rel=torch.float16, spec_group=True):
    g = torch.Generator().manual_seed(K + group)
    six = fmt.startswith("w6a8")
    stored = K // 2 + K // 4 if six else K // 2
    t = {"m.weight": torch.randint(-128, 128, (N, stored), generator=g, dtype=torch.int8),
         "m.weight_s_rel": (torch.rand(N, K // group, generator=g) * 4 + 0.5).to(rel)}
    sp = {"format": fmt, "convrot_groupsize": 256}
    if spec_group:
        sp["group_size"] = group
    t["m.comfy_quant"] = C.comfy_blob(sp)
    if channel:
        t[f"m.weight_{channel}"] = torch.rand(N, generator=g) * 0.01 + 0.001
    if codebook:
        t["m.weight_codebook"] = torch.randn(16, generator=g) * 3
    return t


def test_probe_asym_w4a8(tmp_path):
    path = C.write(str(tmp_path / "w4.safetensors"), grouped_tensors(40, 1024, 128, "asym_w4a8_int8", codebook=True))
    p = C.probe(path, "m")
    assert (p["n"], p["k"]) == (40, 1024) and p["bits"] == 4 and p["packed"] and p["group"] == 128
    assert p["codebook"] and not p["plain_int8"] and p["rel_scale"] == "m.weight_s_rel"
    assert p["row_scale"] == "m.weight_s_channel"
    assert p["spec"]["convrot"]  # the grouped families are stored rotated
    # group_size absent: the family's default (16 for asym_w4a8_int8)
    path = C.write(str(tmp_path / "w4d.safetensors"),
                   grouped_tensors(8, 512, 16, "asym_w4a8_int8", spec_group=False))
    assert C.probe(path, "m")["group"] == 16


def test_probe_w6a8_and_scale_fallback(tmp_path):
    # w6a8 with the channel scale under weight_scale (no weight_s_channel)
    path = C.write(str(tmp_path / "w6.safetensors"),
                   grouped_tensors(16, 1024, 32, "w6a8_int8", channel="scale", spec_group=False))
    p = C.probe(path, "m")
    assert (p["n"], p["k"]) == (16, 1024) and p["bits"] == 6 and p["group"] == 32
    assert p["row_scale"] == "m.weight_scale"


def test_probe_convrot_w4a4(tmp_path):
    g = torch.Generator().manual_seed(3)
    t = {"te.weight": torch.randint(-128, 128, (32, 512), generator=g, dtype=torch.int8),
         "te.weight_scale": torch.rand(32, generator=g),
         "te.comfy_quant": C.comfy_blob({"format": "convrot_w4a4"})}
    p = C.probe(C.write(str(tmp_path / "w4a4.safetensors"), t), "te")
    assert (p["n"], p["k"]) == (32, 1024) and not p["packed"] and p["spec"]["convrot"] and not p["plain_int8"]


@pytest.mark.parametrize("swapped", [False, True])
def test_probe_nvfp4_scale_mapping(tmp_path, swapped):
    """nvfp4's two scales are told apart by shape, whichever name each is
    stored under (core/host/st.cpp:850-880): the >= 2-D multi-entry one is the
    block table, the single value the global scale; fp4 has no row scale.  K is
    twice the stored width; the family is packed 4-bit with group 16."""
    table = torch.randint(0x20, 0x58, (128, 8), dtype=torch.int32).to(torch.uint8)
    glob = torch.tensor(0.5)
    t = {"n.weight": torch.zeros(64, 32, dtype=torch.uint8),
         "n.comfy_quant": C.comfy_blob({"format": "nvfp4"})}
    if swapped:
        t["n.weight_scale"], t["n.weight_scale_2"] = glob, table
    else:
        t["n.weight_scale"], t["n.weight_scale_2"] = table, glob
    p = C.probe(C.write(str(tmp_path / "n.safetensors"), t), "n")
    assert p["k"] == 64 and p["bits"] == 4 and p["group"] == 16 and p["packed"] and p["known"]
    assert p["rel_scale"] == ("n.weight_scale_2" if swapped else "n.weight_scale")
    assert p["global_scale"] == ("n.weight_scale" if swapped else "n.weight_scale_2")
    assert p["row_scale"] == "" and not p["plain_int8"]


def test_probe_fp8_family(tmp_path):
    t = {"e.weight": torch.zeros(8, 256).to(torch.float8_e4m3fn), "e.weight_scale": torch.tensor([0.5]),
         "e.comfy_quant": C.comfy_blob({"format": "float8_e4m3fn"})}
    p = C.probe(C.write(str(tmp_path / "e.safetensors"), t), "e")
    assert p["dtype"] == "F8_E4M3" and p["k"] == 256 and p["known"] and not p["packed"]
    assert p["row_scale"] == "e.weight_scale" and p["row_scale0"] == 0.5


def test_malformed_files(tmp_path):
    path, _ = int8_file(tmp_path)
    raw = open(path, "rb").read()
    hlen = struct.unpack("<Q", raw[:8])[0]
    cases = {
        "short": b"\x01\x02",
        "hlen_past_end": struct.pack("<Q", len(raw)) + raw[8:],
        "bad_json": struct.pack("<Q", 5) + b"{oops" + raw[8 + hlen:],
        "truncated_data": raw[:-16],
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.safetensors"
        p.write_bytes(data)
        out = C.run("probe", str(p), "blk.0.mlp", check=False)
        assert out.returncode == 3 and out.stdout.startswith("error: safetensors"), (name, out.stdout)
    out = C.run("probe", path, "nope", check=False)
    assert out.returncode == 3 and "tensor not found: nope.weight" in out.stdout


def test_dtype_spellings_and_skipped_entries(tmp_path):
    """The header spellings the reference's reader accepts
    (dtype_from_name, core/util/media_common.cpp:31-44): torch names
    (float8_e4m3fn, bfloat16, int8) and the packed I4; entries whose dtype it
    cannot name, or without data_offsets, are skipped (core/host/st.cpp:242,
    :257), not errors."""
    N, K = 8, 512
    g = torch.Generator().manual_seed(4)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sc = (torch.rand(N, generator=g) * 4 + 0.5).to(torch.float8_e4m3fn)
    path = C.write_raw(str(tmp_path / "sp.safetensors"), [
        ("a.weight", "int8", (N, K), w.numpy().tobytes()),
        ("a.weight_scale", "float8_e4m3fn", (N,), sc.view(torch.uint8).numpy().tobytes()),
        ("junk.x", "complex64", (2,), b"\0" * 16),
        ("nodata.x", "F32", (2,), None),
        ("b.weight", "I4", (N, K // 2), bytes(range(256)) * (N * K // 2 // 256)),
        ("b.weight_scale", "bfloat16", (N,), torch.ones(N, dtype=torch.bfloat16).view(torch.int16).numpy().tobytes()),
    ])
    p = C.probe(path, "a")
    assert p["tensors"] == 4, p  # complex64 and the offset-less entry are skipped
    assert p["dtype"] == "I8" and p["plain_int8"] and (p["n"], p["k"]) == (N, K)
    assert np.float32(p["row_scale0"]) == np.float32(sc[0].float().item())
    q = C.probe(path, "b")
    assert q["dtype"] == "I4" and (q["n"], q["k"]) == (N, K), q  # two values per packed byte
    out = C.run("probe", path, "junk", check=False)
    assert out.returncode == 3 and "tensor not found" in out.stdout


def test_header_overflow_is_refused(tmp_path):
    """A shape whose element count wraps 64 bits must not pass the size check."""
    path = C.write_raw(str(tmp_path / "ov.safetensors"), [
        ("o.weight", "I8", (2 ** 32, 2 ** 32), b""),
        ("o.weight_scale", "F32", (1,), b"\0\0\x80\x3f"),
    ])
    out = C.run("probe", path, "o", check=False)
    assert out.returncode == 3 and "overflows" in out.stdout, out.stdout
    path = C.write_raw(str(tmp_path / "ov2.safetensors"), [
        ("o.weight", "F32", (2 ** 62,), b""),
    ])
    out = C.run("probe", path, "o", check=False)
    assert out.returncode == 3 and "error: safetensors" in out.stdout, out.stdout


def lora_probe(target, n, k, *files):
    args = ["lora_probe", target, n, k]
    for path, strength in files:
        args += ["lora", path, strength]
    return json.loads(C.run(*args).stdout)


def test_lora_key_conventions(tmp_path):
    """The three key conventions normalise to the module name
    (core/models/lora.cpp:14-84), alpha from a per-module tensor, then the file
    metadata, then the rank; strength multiplies the delta's scale."""
    n, k, r = 16, 64, 4
    g = torch.Generator().manual_seed(2)
    A = torch.randn(r, k, generator=g)
    B = torch.randn(n, r, generator=g)
    peft = C.lora_file(str(tmp_path / "peft.safetensors"), {
        "diffusion_model.blocks.0.attn.to_q.lora_A.weight": A,
        "diffusion_model.blocks.0.attn.to_q.lora_B.weight": B})
    # kohya's lora_unet_ form: every '_' of the module path stands for '.'
    kohya = C.lora_file(str(tmp_path / "kohya.safetensors"), {
        "lora_unet_blocks_0_attn_qkv.lora_down.weight": A * 2,
        "lora_unet_blocks_0_attn_qkv.lora_up.weight": B,
        "lora_unet_blocks_0_attn_qkv.alpha": torch.tensor(2.0)})
    meta = C.lora_file(str(tmp_path / "meta.safetensors"), {
        "transformer.blocks.0.attn.to_q.lora_A.weight": A,
        "transformer.blocks.0.attn.to_q.lora_B.weight": B}, metadata={"ss_network_alpha": "8"})
    p = lora_probe("blocks.0.attn.to_q", n, k, (peft, 1.0))
    assert p["touches"] and len(p["deltas"]) == 1
    d = p["deltas"][0]
    assert d["rank"] == r and np.float32(d["scale"]) == np.float32(1.0)  # alpha = rank
    assert np.float32(d["a0"]) == A[0, 0].item() and np.float32(d["b0"]) == B[0, 0].item()
    p = lora_probe("blocks.0.attn.qkv", n, k, (kohya, 0.5))
    assert np.float32(p["deltas"][0]["scale"]) == np.float32(0.5 * 2.0 / r)
    assert np.float32(p["deltas"][0]["a0"]) == np.float32(2 * A[0, 0].item())
    p = lora_probe("model.blocks.0.attn.to_q", n, k, (meta, 1.0), (peft, -1.0))
    assert p["touches"] and [np.float32(x["scale"]) for x in p["deltas"]] == [np.float32(2.0), np.float32(-1.0)]
    # a factor whose shape disagrees with the weight is never returned
    p = lora_probe("blocks.0.attn.to_q", n + 1, k, (peft, 1.0))
    assert p["touches"] and p["deltas"] == []
    assert not lora_probe("blocks.0.attn.to_k", n, k, (peft, 1.0))["touches"]
    empty = C.lora_file(str(tmp_path / "none.safetensors"), {"x.weight": torch.zeros(2)})
    out = C.run("lora_probe", "t", 1, 1, "lora", empty, 1.0, check=False)
    assert out.returncode == 3 and "holds no A/B factor pairs" in out.stdout


def test_mutated_headers_under_sanitizers(tmp_path):
    """Bounded mutation fuzz of the header parser and layout rules: 300
    seeded corruptions of a valid two-family checkpoint (bytes flipped,
    JSON tokens and huge or negative numbers spliced in, spans deleted, the
    length field and the data section cut or overstated), each probed with
    st_tool built under AddressSanitizer and UndefinedBehaviorSanitizer.
    Every run ends with a result or a refusal (exit 0 or 3), and the
    sanitizers report nothing."""
    cdir = os.path.join(C.ROOT, "tests", "cpp")
    mk = subprocess.run(["make", "-C", cdir, "st_tool_asan"], capture_output=True, text=True)
    if mk.returncode != 0:
        pytest.skip("sanitizer build unavailable: " + mk.stderr[-200:])
    exe = os.path.join(cdir, "st_tool_asan")
    g = torch.Generator().manual_seed(9)
    base = C.write(str(tmp_path / "base.safetensors"), {
        "a.weight": torch.randint(-127, 128, (64, 256), generator=g, dtype=torch.int8),
        "a.weight_scale": torch.rand(64, generator=g),
        "a.comfy_quant": C.comfy_blob({"format": "int8_tensorwise"}),
        "b.weight": torch.randint(0, 255, (64, 128), generator=g, dtype=torch.uint8),
        "b.weight_scale": torch.rand(64, 2, generator=g).half(),
        "b.comfy_quant": C.comfy_blob({"format": "asym_w4a8_int8", "group_size": 128}),
    })
    raw = open(base, "rb").read()
    hlen = struct.unpack("<Q", raw[:8])[0]
    hdr, body = raw[8:8 + hlen], raw[8 + hlen:]
    tokens = [b'"', b"{", b"}", b"[", b"]", b",", b":", b"-1", b"99999999999999999999", b"18446744073709551615",
              b'"I4"', b'"F8_E4M3"', b'"float8_e4m3fn"', b"null", b"\\u0000", b"1e999", b'"data_offsets"',
              b'"shape"', b'"dtype"', b"0", b"4294967296"]
    rng = np.random.default_rng(17)
    logs = str(tmp_path / "san")
    env = dict(os.environ, ASAN_OPTIONS=f"detect_leaks=0:log_path={logs}",
               UBSAN_OPTIONS=f"print_stacktrace=1:log_path={logs}")
    p = tmp_path / "m.safetensors"
    for it in range(300):
        h = bytearray(hdr)
        for _ in range(int(rng.integers(1, 7))):
            pos, op = int(rng.integers(len(h))), rng.random()
            if op < 0.4:
                h[pos] = int(rng.integers(256))
            elif op < 0.8:
                h[pos:pos] = tokens[int(rng.integers(len(tokens)))]
            else:
                del h[pos:pos + int(rng.integers(1, 9))]
        b = body if rng.random() < 0.8 else body[:int(rng.integers(len(body) + 1))]
        n = len(h) if rng.random() < 0.9 else [0, 1, len(h) + 5, 2 ** 40, 2 ** 64 - 1][int(rng.integers(5))]
        p.write_bytes(struct.pack("<Q", n) + bytes(h) + b)
        out = subprocess.run([exe, "probe", str(p), "ab"[it % 2]], capture_output=True, env=env, timeout=60)
        reports = [f for f in os.listdir(tmp_path) if f.startswith("san")]
        assert out.returncode in (0, 3) and not reports, (it, out.returncode, out.stdout[-300:], reports)
