"""CPU checks of the C ABI boundary (no GPU needed).

* libphi_qlinear.so loads and exports every function include/*.h declares;
* libphi_media.so (the C++ host layer) loads and exports the reference-named
  dispatch entry points;
* contract violations are refused before any device work, with the status
  codes and the messages the reference's dispatchers raise
  (core/runtime/compute.cpp:552, :665-668; core/kernels/w4a8_expand.cpp:264-281).
"""
import ctypes
import glob
import os
import re
import subprocess

import pytest

import phi_qlinear as Q

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = ctypes.c_void_p(0x10000)  # a well-aligned address; never dereferenced on these paths


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(phi_hip_\w+)\s*\(", text))
    return names


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 12
    out = subprocess.run(["nm", "-D", "--defined-only", Q.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (phi_hip_\w+)", out))
    assert names <= exported, f"declared but not exported: {sorted(names - exported)}"
    assert set(Q.EXPORTS) == names
    for n in names:
        getattr(lib, n)


def test_abi_version(lib):
    assert lib.phi_hip_abi_version() == 1


def test_host_layer_library_exports_reference_names():
    assert os.path.exists(Q.MEDIA_LIB_PATH)
    ctypes.CDLL(Q.MEDIA_LIB_PATH)
    out = subprocess.run(["nm", "-DC", "--defined-only", Q.MEDIA_LIB_PATH], capture_output=True,
                         text=True).stdout
    for name in ("phi::media::dispatch_int8_gemm", "phi::media::dispatch_quant_convrot",
                 "phi::media::dispatch_w4a8_expand", "phi::media::linear_gemm",
                 "phi::media::ComputeContext::submit", "phi::media::dispatch_elem",
                 "phi::media::dispatch_silu_gate_fused", "phi::media::dispatch_int4_gemm",
                 "phi::media::dispatch_lora_rank_add", "phi::media::apply_lora_tail",
                 "phi::media::load_quant_linear", "phi::media::load_quant3_linear",
                 "phi::media::upload_quant_linear_i8", "phi::media::upload_quant_linear_w4a4",
                 "phi::media::load_lora_tail", "phi::media::LoraSet::add", "phi::media::LoraSet::touches",
                 "phi::media::LoraSet::deltas_for", "phi::media::GpuArena::alloc", "phi::media::GpuArena::rewind_to",
                 "phi::media::GpuCtx::walloc"):
        assert name in out, name


def status_and_msg(lib, rc):
    return rc, Q.last_error()


def test_quant_rotate_contract(lib):
    rc, msg = status_and_msg(lib, lib.phi_hip_quant_rotate(None, FAKE, Q.F32, 4, 300, 300, FAKE, 304,
                                                           FAKE, 127.0, 0, 1))
    assert rc == 2 and "K=300 is not a multiple of 256" in msg
    rc, msg = status_and_msg(lib, lib.phi_hip_quant_rotate(None, FAKE, Q.F32, 4, 256, 256, FAKE, 256,
                                                           FAKE, 127.5, 0, 1))
    assert rc == 1 and "qmax" in msg
    rc, msg = status_and_msg(lib, lib.phi_hip_quant_rotate(None, FAKE, Q.I8, 4, 256, 256, FAKE, 256,
                                                           FAKE, 127.0, 0, 1))
    assert rc == 1
    rc, msg = status_and_msg(lib, lib.phi_hip_quant_rotate(None, ctypes.c_void_p(0x10004), Q.F32, 4,
                                                           256, 256, FAKE, 256, FAKE, 127.0, 0, 1))
    assert rc == 3
    # rows == 0 is a no-op, as in dispatch_quant_convrot
    assert lib.phi_hip_quant_rotate(None, None, Q.F32, 0, 300, 300, None, 300, None, 127.0, 0, 1) == 0
    assert Q.last_error() == ""


def test_activation_contracts(lib):
    # unknown activation
    rc = lib.phi_hip_quant_rotate_act(None, FAKE, Q.F32, 4, 256, 512, 7, FAKE, 256, FAKE, 127.0, 0, 1)
    assert rc == 1 and "act" in Q.last_error()
    # the SiLU gate reads [gate | value]: ldx must cover 2K
    rc = lib.phi_hip_quant_rotate_act(None, FAKE, Q.F32, 4, 256, 256, Q.ACT_SILU_GATE, FAKE, 256, FAKE,
                                      127.0, 0, 1)
    assert rc == 2 and "2K" in Q.last_error()
    rc = lib.phi_hip_quant_rotate_act(None, FAKE, Q.F32, 4, 300, 600, Q.ACT_GELU_TANH, FAKE, 304, FAKE,
                                      127.0, 0, 1)
    assert rc == 2 and "K=300 is not a multiple of 256" in Q.last_error()
    rc = lib.phi_hip_silu_gate(None, FAKE, Q.F32, 4, 64, 100, ctypes.c_void_p(0x900000), Q.F32, 64)
    assert rc == 2
    # out overlapping gx
    rc = lib.phi_hip_silu_gate(None, FAKE, Q.F32, 4, 64, 128, ctypes.c_void_p(0x10000 + 256), Q.F32, 64)
    assert rc == 1 and "overlap" in Q.last_error()
    rc = lib.phi_hip_silu_gate(None, FAKE, Q.I8, 4, 64, 128, ctypes.c_void_p(0x900000), Q.F32, 64)
    assert rc == 1
    # in-place GELU only between equal dtypes
    rc = lib.phi_hip_gelu_tanh(None, FAKE, Q.BF16, FAKE, Q.F32, 64)
    assert rc == 1 and "in place" in Q.last_error()
    # empty problems are no-ops
    assert lib.phi_hip_silu_gate(None, None, Q.F32, 0, 64, 128, None, Q.F32, 64) == 0
    assert lib.phi_hip_quant_rotate_act(None, None, Q.F32, 0, 256, 512, Q.ACT_SILU_GATE, None, 256, None,
                                        127.0, 0, 1) == 0


def test_int4_gemm_contract(lib):
    rc = lib.phi_hip_i4_gemm(None, FAKE, 512, FAKE, 256, FAKE, FAKE, FAKE, Q.F32, 64, 0, 64, 512, None, 0)
    assert rc == 2 and Q.last_error() == "int4_gemm: empty problem"
    rc = lib.phi_hip_i4_gemm(None, FAKE, 768, FAKE, 384, FAKE, FAKE, FAKE, Q.F32, 64, 4, 64, 768, None, 0)
    assert rc == 2 and Q.last_error() == "int4_gemm: K=768 is not a multiple of 512"
    rc = lib.phi_hip_i4_gemm(None, FAKE, 512, FAKE, 200, FAKE, FAKE, FAKE, Q.F32, 64, 4, 64, 512, None, 0)
    assert rc == 2 and "nibble row" in Q.last_error()
    rc = lib.phi_hip_i4_gemm(None, FAKE, 512, FAKE, 256, None, FAKE, FAKE, Q.F32, 64, 4, 64, 512, None, 0)
    assert rc == 1 and "scales" in Q.last_error()
    assert lib.phi_hip_i4_workspace_bytes(511, 64, 512) == 0
    assert lib.phi_hip_i4_workspace_bytes(512, 64, 512) == 64 * 512
    assert lib.phi_hip_i4_workspace_bytes(512, 64, 768) == 0


def test_lora_contracts(lib):
    rc = lib.phi_hip_lora_rank_add(None, FAKE, FAKE, FAKE, Q.F32, 16, 0, 16, 4)
    assert rc == 2 and Q.last_error() == "lora_rank_add: empty problem"
    rc = lib.phi_hip_lora_rank_add(None, FAKE, FAKE, FAKE, Q.I8, 16, 4, 16, 4)
    assert rc == 1
    rc = lib.phi_hip_lora_down(None, FAKE, Q.F32, 100, 4, 256, FAKE, 8, FAKE)
    assert rc == 2 and "ldx" in Q.last_error()
    rc = lib.phi_hip_lora_tail(None, FAKE, Q.F32, 256, 4, 256, FAKE, FAKE, 8, 16, FAKE, Q.F32, 16, FAKE, 127)
    assert rc == 4 and "needs 128" in Q.last_error()
    # an inactive tail or no rows: a no-op
    assert lib.phi_hip_lora_tail(None, None, Q.F32, 256, 0, 256, None, None, 8, 16, None, Q.F32, 16, None, 0) == 0
    assert lib.phi_hip_lora_tail(None, None, Q.F32, 256, 4, 256, None, None, 0, 16, None, Q.F32, 16, None, 0) == 0


def test_gemm_contract(lib):
    g = lib.phi_hip_i8_gemm
    rc, msg = status_and_msg(lib, g(None, FAKE, 64, FAKE, 64, FAKE, FAKE, 0, None, 0, FAKE, Q.BF16, 64,
                                    0, 64, 64, None, 0))
    assert rc == 2 and "empty problem" in msg
    rc, msg = status_and_msg(lib, g(None, FAKE, 64, FAKE, 64, None, FAKE, 0, None, 0, FAKE, Q.BF16, 64,
                                    8, 64, 64, None, 0))
    assert rc == 1 and "scales" in msg
    # (K % 64 != 0 and unaligned operands are served by the any-K kernel, so
    # they are not contract errors; no case here may reach a launch.)
    rc, msg = status_and_msg(lib, g(None, FAKE, 64, FAKE, 64, FAKE, FAKE, 0, FAKE, Q.I8, FAKE, Q.BF16,
                                    64, 8, 64, 64, None, 0))
    assert rc == 1 and "bias" in msg
    rc, msg = status_and_msg(lib, g(None, FAKE, 64, FAKE, 64, FAKE, FAKE, 0, None, 0, FAKE, Q.F16, 64,
                                    8, 64, 64, None, 0))
    assert rc == 1 and "output dtype" in msg


def test_linear_requires_activation_scratch(lib):
    rc = lib.phi_hip_q8_linear(None, FAKE, Q.BF16, 256, 4, 256, FAKE, 256, FAKE, 1, None, 0, 64,
                               FAKE, Q.BF16, 64, None, None, 0, None, 0)
    assert rc == 1 and "activation scratch" in Q.last_error()


def w4(rows=4, k=128, group=32, layout=0, crb=64, cb=None):
    w = Q.W4a8Weight()
    w.codes = 0x10000
    w.codes_row_bytes = crb
    w.s_rel = 0x20000
    w.s_rel_dtype = Q.F32
    w.srel_row_bytes = 4 * max(1, k // max(group, 1))
    w.rows, w.k, w.group, w.layout = rows, k, group, layout
    w.codebook = cb
    return w


def test_w4a8_contract(lib):
    e = lib.phi_hip_w4a8_expand
    rc = e(None, ctypes.byref(w4(k=200, group=64)), FAKE, FAKE)
    assert rc == 2 and "K=200 is not a multiple of group=64" in Q.last_error()
    rc = e(None, ctypes.byref(w4(k=128, group=32, crb=50)), FAKE, FAKE)
    assert rc == 2 and "needs 64 packed bytes, got 50" in Q.last_error()
    rc = e(None, ctypes.byref(w4(k=128, group=2, layout=1, crb=96)), FAKE, FAKE)
    assert rc == 2 and "whole number of code groups" in Q.last_error()
    rc = e(None, ctypes.byref(w4(k=128, group=32, layout=1, crb=96, cb=0x30000)), FAKE, FAKE)
    assert rc == 1 and "codebook" in Q.last_error()
    rc = lib.phi_hip_w4a8_prepare(None, ctypes.byref(w4(k=128, group=32, layout=1, crb=96)), FAKE, FAKE)
    assert rc == 7
    # group must be a power of two >= 64 for the in-register GEMM
    rc = lib.phi_hip_w4a8_linear(None, FAKE, Q.BF16, 256, 4, 256, FAKE, 128, FAKE, 32, FAKE, None, 0,
                                 64, FAKE, Q.BF16, 64, FAKE, FAKE, 0, None, 0)
    assert rc == 2 and "group=32" in Q.last_error()


def test_gemv_contract(lib):
    items = (Q.GemvItem * 1)()
    items[0].W, items[0].sW, items[0].C, items[0].ldc = 0x10000, 0x20000, 0x30000, 64
    rc = lib.phi_hip_i8_gemv_batched(None, FAKE, FAKE, 9, 256, 64, items, 1, Q.F32, Q.BF16, None, 0)
    assert rc == 2 and "M=9" in Q.last_error()
    rc = lib.phi_hip_i8_gemv_batched(None, FAKE, FAKE, 1, 250, 64, items, 1, Q.F32, Q.BF16, None, 0)
    assert rc == 2
    items[0].ldc = 10
    rc = lib.phi_hip_i8_gemv_batched(None, FAKE, FAKE, 1, 256, 64, items, 1, Q.F32, Q.BF16, None, 0)
    assert rc == 2 and "ldc" in Q.last_error()
    assert lib.phi_hip_i8_gemv_batched(None, FAKE, FAKE, 1, 256, 64, items, 0, Q.F32, Q.BF16, None, 0) == 0


def test_weight_step_contracts(lib):
    """Load-time steps: argument checks that return before any launch."""
    rc = lib.phi_hip_convrot_rows(None, FAKE, 4, 300, 300, FAKE, 300)
    assert rc == 2 and "not a multiple of 256" in Q.last_error()
    rc = lib.phi_hip_convrot_rows(None, ctypes.c_void_p(0x10000), 4, 256, 256, ctypes.c_void_p(0x10400), 256)
    assert rc == 1 and "overlaps" in Q.last_error()
    assert lib.phi_hip_convrot_rows(None, None, 0, 256, 256, None, 256) == 0
    rc = lib.phi_hip_dequant_rows(None, FAKE, Q.I8, 4, 64, 64, None, 0, FAKE, 64)
    assert rc == 1 and "row scales" in Q.last_error()
    rc = lib.phi_hip_dequant_rows(None, FAKE, Q.U8_E4M3, 4, 64, 64, None, 0, FAKE, 64)
    assert rc == 1 and "src dtype" in Q.last_error()
    # nvfp4 rows: a block table too small for the rows asked is refused before a launch
    rc = lib.phi_hip_dequant_fp4_rows(None, FAKE, 512, 100, 100, 1024, FAKE, 128, 16, 16, None, 0, FAKE, 1024)
    assert rc == 2 and "block-scale table does not cover" in Q.last_error()
    rc = lib.phi_hip_dequant_fp4_rows(None, FAKE, 100, 0, 4, 1024, None, 0, 0, 16, None, 0, FAKE, 1024)
    assert rc == 2 and "leading dimension" in Q.last_error()
    rc = lib.phi_hip_dequant_rows(None, FAKE, Q.I4, 4, 64, 31, None, 0, FAKE, 64)
    assert rc == 2 and "leading dimension" in Q.last_error()
    rc = lib.phi_hip_lora_fold(None, FAKE, 30, 4, 64, FAKE, FAKE, 2, 1.0)
    assert rc == 2 and "ldw < k" in Q.last_error()
    assert lib.phi_hip_lora_fold(None, None, 64, 4, 64, None, None, 0, 1.0) == 0


def test_any_k_gemm_contract(lib):
    """Any K and any operand offset are served; empty problems and misaligned
    scale vectors are still refused."""
    rc = lib.phi_hip_i8_gemm(None, FAKE, 100, FAKE, 100, None, None, 0, None, Q.F32, FAKE, Q.I32, 4, 0, 4, 100,
                             None, 0)
    assert rc == 2 and "empty problem" in Q.last_error()
    rc = lib.phi_hip_i8_gemm(None, ctypes.c_void_p(0x10001), 100, FAKE, 100, ctypes.c_void_p(0x20002), FAKE, 1,
                             None, Q.F32, FAKE, Q.F32, 4, 4, 4, 100, None, 0)
    assert rc == 3 and "sA is misaligned" in Q.last_error()
    rc = lib.phi_hip_i8_gemm(None, FAKE, 50, FAKE, 100, None, None, 0, None, Q.F32, FAKE, Q.I32, 4, 4, 4, 100,
                             None, 0)
    assert rc == 2 and "leading dimension" in Q.last_error()


def test_k_tiled_contracts(lib):
    """The K-tiled entries take whole 256-deep K-steps, 16-byte aligned
    operands and whole 16-byte output pieces, and refuse anything else before
    any device work."""
    odd = ctypes.c_void_p(0x10008)
    rc = lib.phi_hip_pack_k_tiled(None, FAKE, 320, 4, 320, FAKE)
    assert rc == 2 and "not a multiple of 256" in Q.last_error()
    rc = lib.phi_hip_pack_k_tiled(None, odd, 512, 4, 512, FAKE)
    assert rc == 3 and "16-byte aligned" in Q.last_error()
    rc = lib.phi_hip_pack_k_tiled(None, FAKE, 520, 4, 512, FAKE)
    assert rc == 3 and "multiple of 16" in Q.last_error()
    rc = lib.phi_hip_pack_k_tiled(None, FAKE, 512, 0, 512, FAKE)
    assert rc == 2 and "empty" in Q.last_error()
    rc = lib.phi_hip_i8_gemm_kt(None, FAKE, FAKE, FAKE, FAKE, 1, None, Q.F32, FAKE, Q.BF16, 12, 4, 12, 512)
    assert rc == 7 and "16-byte output pieces" in Q.last_error()
    rc = lib.phi_hip_i8_gemm_kt(None, FAKE, odd, FAKE, FAKE, 1, None, Q.F32, FAKE, Q.BF16, 16, 4, 16, 512)
    assert rc == 3
    rc = lib.phi_hip_q8_linear_kt(None, FAKE, Q.BF16, 16384 + 256, 4, 16384 + 256, FAKE, FAKE, 1, None, Q.F32, 16,
                                  FAKE, Q.BF16, 16, FAKE, FAKE, 0)
    assert rc == 7 and "16384" in Q.last_error()
    rc = lib.phi_hip_q8_linear_kt(None, FAKE, Q.BF16, 512, 4, 512, FAKE, FAKE, 1, None, Q.F32, 16, FAKE, Q.BF16,
                                  16, None, FAKE, 0)
    assert rc == 1 and "activation scratch" in Q.last_error()
    rc = lib.phi_hip_quant_rotate_kt(None, FAKE, Q.BF16, 4, 300, 300, FAKE, FAKE, 127.0, 0)
    assert rc == 2
    rc = lib.phi_hip_quant_rotate_act_kt(None, FAKE, Q.BF16, 4, 512, 512, 9, FAKE, FAKE, 127.0, 0)
    assert rc == 1 and "act" in Q.last_error()
    rc = lib.phi_hip_quant_rotate_mod_kt(None, FAKE, Q.BF16, 4, 16640, 16640, FAKE, FAKE, FAKE, FAKE, 127.0, 0)
    assert rc == 7 and "16384" in Q.last_error()
    rc = lib.phi_hip_i8_gemm_residual_kt(None, FAKE, FAKE, FAKE, FAKE, 1, None, Q.F32, None, FAKE, 16, 4, 16, 512)
    assert rc == 1 and "gate" in Q.last_error()


def test_tile_plan(lib):
    """The persistent plan on 256 compute units (the CPU fallback): config 1
    up runs 16 tile-rows of 256 x 256 (three whole rounds) and the last 256
    rows as 128 x 128 tiles; config 1 down, one round of 204 256 x 256 tiles;
    config 0, 128 x 128 tiles only."""
    assert lib.phi_hip_big_tile_rows(4352, 12288) == 4096
    assert lib.phi_hip_big_tile_rows(4352, 3072) == 4352
    assert lib.phi_hip_big_tile_rows(256, 3072) == 0
    assert lib.phi_hip_big_tile_rows(0, 3072) == 0


def test_workspace_queries(lib):
    assert lib.phi_hip_workspace_bytes(4352, 12288, 3072) >= 0
    assert lib.phi_hip_gemv_workspace_bytes(60) >= 0


def test_binding_refuses_host_tensors():
    import torch

    with pytest.raises(ValueError):
        Q.quant_rotate(torch.zeros((2, 256)))


def test_noalloc_contract(lib):
    """The allocation-free linear refuses, before touching any device, a
    problem whose activation scratch does not fit its static array."""
    cap = lib.phi_hip_noalloc_scratch_bytes()
    assert cap == 64 << 20
    K = 4096
    rc = lib.phi_hip_q8_linear_noalloc(None, FAKE, Q.BF16, K, cap // K + 1, K, FAKE, K, FAKE, 1, None, Q.F32, 64,
                                       FAKE, Q.BF16, 64, 0)
    assert rc == 4 and "static scratch" in Q.last_error()
    rc = lib.phi_hip_q8_linear_noalloc(None, FAKE, Q.BF16, K, 0, K, FAKE, K, FAKE, 1, None, Q.F32, 64,
                                       FAKE, Q.BF16, 64, 0)
    assert rc == 2 and "empty problem" in Q.last_error()


def test_gemm_plan_table(lib):
    """The tuning table's C ABI without a device: entries set, read back,
    replaced and removed; malformed plans refused with the library's message."""
    Q.gemm_plan_clear()
    assert Q.gemm_plan_count() == 0
    Q.gemm_plan_set(4352, 12288, 3072, k_tiled=True, big_rows=4096, group_m=8, split=True)
    Q.gemm_plan_set(4352, 12288, 3072, k_tiled=False, big_rows=4352, group_m=2)
    assert Q.gemm_plan_count() == 2
    # The tile shape comes back resolved: with no device the cost model counts
    # 256 CUs, where 272 x 192 tiles fill config 1's rounds (K-tiled only).
    assert Q.gemm_plan_get(4352, 12288, 3072, k_tiled=True) == {"big_rows": 4096, "group_m": 8, "split": True,
                                                                "tile": Q.PLAN_TILE_272, "tuned": True}
    assert Q.gemm_plan_get(4352, 12288, 3072) == {"big_rows": 4352, "group_m": 2, "split": False,
                                                  "tile": Q.PLAN_TILE_272, "tuned": True}
    Q.gemm_plan_set(4352, 12288, 3072, k_tiled=True, big_rows=3840, group_m=4, tile=Q.PLAN_TILE_SQUARE)
    now = Q.gemm_plan_get(4352, 12288, 3072, k_tiled=True)
    assert now["big_rows"] == 3840 and now["tile"] == Q.PLAN_TILE_SQUARE and Q.gemm_plan_count() == 2
    Q.gemm_plan_set(4352, 12288, 3072, k_tiled=True, group_m=2, tile=Q.PLAN_TILE_272)
    assert Q.gemm_plan_get(4352, 12288, 3072, k_tiled=True)["tile"] == Q.PLAN_TILE_272
    for bad, msg in ((dict(big_rows=100), "big_rows=100"), (dict(big_rows=5000), "big_rows=5000"),
                     (dict(big_rows=-2), "big_rows=-2"), (dict(group_m=17), "group_m=17"),
                     (dict(tile=3), "tile=3"), (dict(tile=-1), "tile=-1")):
        with pytest.raises(Q.QLinearError, match=msg):
            Q.gemm_plan_set(4352, 12288, 3072, **bad)
    for kt in (True, False):
        with pytest.raises(Q.QLinearError, match="K % 512 == 0"):
            Q.gemm_plan_set(4352, 12288, 3328, k_tiled=kt, tile=Q.PLAN_TILE_272)
    # Unresolvable by 272 x 192 tiles (K % 512 != 0): the square plan.
    assert Q.gemm_plan_get(4352, 12288, 3328, k_tiled=True)["tile"] == Q.PLAN_TILE_SQUARE
    # The cost model (256 CUs): K-tiled, 272 x 192 tiles at the DiT shapes,
    # config 3's included (13 and 35 rounds against 10 and 27 square ones);
    # row-major, at config 1's whole rounds but not at config 3's; config 0's
    # 256 rows keep the square plan's 128 x 128 tiles.
    for M, N, K in ((4352, 3072, 12288), (4352, 9216, 3072), (32760, 5120, 5120), (32760, 13824, 5120)):
        assert Q.gemm_plan_get(M, N, K, k_tiled=True)["tile"] == Q.PLAN_TILE_272, (M, N, K)
    for M, N, K in ((4352, 3072, 12288), (4352, 12288, 3072)):
        assert Q.gemm_plan_get(M, N, K)["tile"] == Q.PLAN_TILE_272, (M, N, K)
    for M, N, K in ((32760, 5120, 5120), (32760, 13824, 5120)):
        assert Q.gemm_plan_get(M, N, K)["tile"] == Q.PLAN_TILE_SQUARE, (M, N, K)
    for kt in (True, False):
        assert Q.gemm_plan_get(256, 3072, 3072, k_tiled=kt)["tile"] == Q.PLAN_TILE_SQUARE
    with pytest.raises(Q.QLinearError, match="empty problem"):
        Q.gemm_plan_set(0, 1, 1)
    Q.gemm_plan_set(4352, 12288, 3072, k_tiled=True, remove=True)
    assert Q.gemm_plan_count() == 1
    Q.gemm_plan_clear()
    assert Q.gemm_plan_count() == 0
