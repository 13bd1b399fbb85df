#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-linear hot path.

Default workload (BASELINE.json metric): the W8A8 linear at M=4352, K=3072,
N=12288 (config 1's up-projection) -- one step is one fused linear: the
rotate+quantise prologue over the bf16 activations, then the int8 MFMA GEMM
with the scale/bias epilogue to bf16.  Inputs are resident in HBM before the
timed region.  Prints ONE JSON line.

  python bench.py [--steps K] [--warmup W] [--config c1_up|c1_down|c2|c3_attn|c3_mlp|c4|c0]
                  [--no-cpu-baseline] [--calibrate-copy MIB]

--calibrate-copy launches a plain device copy of MIB MiB (three times, after the
timed region) so a rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE run of this same
command can scale the counters to bytes; the measured HBM bytes per launch of
the dominant kernel are read back from profiles/traffic_<config>.json.

Only one GPU is used: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "phi-agent_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "W8A8 linear TOPS & % int8 MFMA peak at M=4352,K=3072,N=12288"
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, 8 TB/s
FP32_PEAK_TFLOPS = 157.3  # MI355X fp32 vector (published; counts packed-fp32 issue)
CPU_SAMPLE_ROWS = 4352    # rows of the reference CPU linear timed for the baseline (all of c1)

CONFIGS = {
    "c0": dict(kind="w8a8", M=256, K=3072, N=3072),
    "c1_up": dict(kind="w8a8", M=4352, K=3072, N=12288),
    "c1_down": dict(kind="w8a8", M=4352, K=12288, N=3072),
    "c2": dict(kind="w4a8", M=4352, K=3072, N=9216, group=128),
    "c3_attn": dict(kind="w8a8", M=32760, K=5120, N=5120),
    "c3_mlp": dict(kind="w8a8", M=32760, K=5120, N=13824),
    "c4": dict(kind="gemv", M=1, K=3072, N=18432, items=60),
    "c4_m2": dict(kind="gemv", M=2, K=3072, N=18432, items=60),
    # Config 1's MLP as a DiT sub-block: adaLN modulate -> up (bf16) -> GELU-tanh
    # -> down into the fp32 residual stream through the gate.
    "c1_block": dict(kind="block", M=4352, K=3072, N=12288),
    # The text encoder's convrot_w4a4 MLP up-projection (hidden 5120 -> 25600,
    # a 1024-token prompt): rotate + quantise with qmax 7, then the int4 GEMM.
    "c5_w4a4": dict(kind="w4a4", M=1024, K=5120, N=25600),
    # A rank-64 LoRA correction on config 1's up-projection output (fp32, as
    # the reference's apply_lora_tail runs it after the linear).
    "c1_lora": dict(kind="lora", M=4352, K=3072, N=12288, rank=64),
    # Ceilings, not a workload: int8 MFMAs with no data movement (zero, static
    # and rotating random operands) and the operand stream into LDS alone.
    "mfma_ceiling": dict(kind="ceiling"),
    # A reference point, not this library: the vendor int8 GEMM (hipBLASLt,
    # through torch._int_mm) on config 1's shapes, int32 out, no epilogue.
    "c1_up_vendor": dict(kind="vendor", M=4352, K=3072, N=12288),
    # The headline step with the GEMM's per-tile timeline recorded (the
    # pipeline rebuilt with its trace hooks in lib/libphi_probe.so).
    "c1_up_tiles": dict(kind="tiletrace", M=4352, K=3072, N=12288),
    "c1_down_tiles": dict(kind="tiletrace", M=4352, K=12288, N=3072),
    # The same for the 272 x 192 kernel the plan picks at these shapes
    # (i8_gemm_t272.hip rebuilt with its trace hooks in lib/libphi_probe.so).
    "c1_up_t272_tiles": dict(kind="t272trace", M=4352, K=3072, N=12288),
    "c1_down_t272_tiles": dict(kind="t272trace", M=4352, K=12288, N=3072),
    "c2_t272_tiles": dict(kind="t272trace", M=4352, K=3072, N=9216, group=128),
    # the same kernel on row-major operands (the drop-in's default layout)
    "c1_up_t272_tiles_row": dict(kind="t272trace", M=4352, K=3072, N=12288, layout="row"),
    "c1_down_t272_tiles_row": dict(kind="t272trace", M=4352, K=12288, N=3072, layout="row"),
    "c1_down_vendor": dict(kind="vendor", M=4352, K=12288, N=3072),
    # A reference point for the prologue: torch's bf16 -> int8 conversion of
    # the same activation tensor moves the prologue's bytes (2K in, K out a row).
    "c1_prologue_vendor": dict(kind="convref", M=4352, K=3072),
    # The prologue against the floor of its memory pattern (probe kernels).
    "c1_prologue_floor": dict(kind="qrfloor", M=4352, K=3072),
    "c1_down_prologue_floor": dict(kind="qrfloor", M=4352, K=12288),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def traffic_for(config: str):
    """HBM bytes per launch of the dominant kernel, measured by rocprofv3
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration) and
    committed as profiles/traffic_<config>.json; None when not measured."""
    path = os.path.join(ROOT, "profiles", f"traffic_{config}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return float(json.load(f)["hbm_bytes_per_launch"])


def calibrate_copy(mib: int) -> None:
    import torch

    n = mib * 1024 * 1024
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def cpu_baseline(cfg) -> dict | None:
    """The reference's CPU linear (convrot + quantise + naive gemm_int8,
    core/host/quant.cpp) on a bounded row sample, single thread."""
    import oracle

    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    rows = min(M, CPU_SAMPLE_ROWS)
    if oracle.ref_available():
        secs = oracle.ref_bench_q8(M, N, K, rows)
        kind = "reference"
    else:
        # The C restatement: same loops, timed the same way.
        import numpy as np

        from phi_qlinear import synth

        x = synth.activations(rows, K, seed=0)
        w = synth.int8_weight(N, K, seed=1).numpy()
        xb = x.view(__import__("torch").int16).numpy().view(np.uint16)
        t0 = time.perf_counter()
        q, s = oracle.quantize_rows(xb)
        oracle.gemm_i8_i32(q, w)
        secs = time.perf_counter() - t0
        kind = "port"
    tops = 2.0 * rows * N * K / secs / 1e12
    out = {"value": tops, "unit": "TOPS", "cores": 1, "kind": kind,
           "sample": f"{rows} of {M} rows x N={N} x K={K} (naive loop is linear in M), {secs:.2f} s"}
    if kind == "reference":
        # The same rows over the host's cores (one row per task from a shared
        # counter, as the reference's parallel_for), at most 16: the GPU box's share.
        threads = max(1, min(16, os.cpu_count() or 1))
        mt = oracle.ref_bench_q8_mt(M, N, K, rows, threads)
        out["parallel"] = {"value": 2.0 * rows * N * K / mt / 1e12, "unit": "TOPS", "cores": threads,
                           "seconds": round(mt, 3)}
    return out


def settle(seconds=1.0):
    """An idle pause with the device drained, so the next burst of launches
    meets the board's clocks as the first one did."""
    import torch

    torch.cuda.synchronize()
    time.sleep(seconds)


def bench_w8a8(cfg, steps, warmup, layout="kt", weights="uniform"):
    """One step: rotate + quantise the activations, then the GEMM with the
    dequant + bias epilogue to bf16.  layout "kt": the weight is packed into
    the K-tiled operand layout once, before timing (a load-time step, like
    the checkpoint's quantisation), and the prologue writes q8 K-tiled;
    "row": row-major operands (the reference's layout).  weights "uniform":
    int8 codes uniform on [-127, 127] with one scale; "gaussian": the
    reference benchmark's weights (core/bench/media_bench.cpp:224-231),
    N(0, 1) values rotated and quantised per row (this library's quantiser,
    the reference's quantize_weight), with the per-row scales."""
    import torch

    import phi_qlinear as Q
    from phi_qlinear import synth

    dev = torch.device("cuda:0")
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    x = synth.activations(M, K, seed=0, device=dev)
    if weights == "gaussian":
        g = torch.Generator(device=dev).manual_seed(11)
        W, sW = Q.quant_rotate(torch.randn((N, K), generator=g, device=dev))
    else:
        W = synth.int8_weight(N, K, seed=1, device=dev)
        sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=2, device=dev)
    q8 = torch.empty((M, K), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    if layout == "kt":
        Wk = Q.pack_k_tiled(W)
        qk = q8.view(-1)
        torch.cuda.synchronize()

    def linear():
        if layout == "kt":
            Q.q8_linear_kt(x, Wk, N, sW, b, q8=qk, s8=s8, C=y)
        else:
            Q.q8_linear(x, W, sW, b, q8=q8, s8=s8, C=y)

    def prologue():
        if layout == "kt":
            Q.quant_rotate_kt(x, q=qk, s=s8)
        else:
            Q.quant_rotate(x, q=q8, s=s8)

    def gemm():
        if layout == "kt":
            Q.i8_gemm_kt(qk, Wk, M, N, K, s8, sW, b, C=y)
        else:
            Q.i8_gemm(q8, W, s8, sW, b, C=y)

    for _ in range(warmup):
        linear()
    torch.cuda.synchronize()
    # The timed region: `steps` whole linears back to back, nothing recorded
    # between them (an event record costs ~4.5 us of stream time a step).
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        linear()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    # The roofline region: the same steps with an event pair around each GEMM
    # launch, on the launch stream, under the timed region's conditions.  The
    # board lowers its clock some launches into a burst and recovers only
    # after hundreds, so a region run straight after the timed one would sit
    # deeper in that dip than the launches it describes.  An idle second (the
    # clocks are back at idle levels within 0.4 s) and the same warm-up come
    # first, so the GEMM is timed at the same point of a burst.
    settle()
    for _ in range(warmup):
        linear()
    mids = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        prologue()
        mids[i].record()
        gemm()
        ends[i].record()
    torch.cuda.synchronize()
    gemm_ms = sum(m.elapsed_time(z) for m, z in zip(mids, ends)) / steps
    pro_ms = (sum(ends[i - 1].elapsed_time(mids[i]) for i in range(1, steps)) / (steps - 1)) if steps > 1 else None
    ops = 2.0 * M * N * K
    extra = {"prologue_us": None if pro_ms is None else pro_ms * 1e3, "gemm_us": gemm_ms * 1e3,
             "fused_linear_tops": ops / (ms * 1e-3) / 1e12}
    if layout == "kt":
        # The drop-in's own path (linear_gemm without K-tiled weights): the
        # row-major linear, timed like the headline region (idle second,
        # warm-up, then `steps` of them).
        settle()
        for _ in range(warmup):
            Q.q8_linear(x, W, sW, b, q8=q8, s8=s8, C=y)
        start.record()
        for _ in range(steps):
            Q.q8_linear(x, W, sW, b, q8=q8, s8=s8, C=y)
        end.record()
        torch.cuda.synchronize()
        row_ms = start.elapsed_time(end) / steps
        extra["row_major_linear_us"] = row_ms * 1e3
        extra["row_major_linear_tops"] = ops / (row_ms * 1e-3) / 1e12
        # What linear_gemm runs for a row-major weight: the same linear with
        # the activation scratch K-tiled where the 272 x 192 plan takes it
        # (phi_hip_q8_linear_kq), timed the same way.
        qk2 = torch.empty((M, K), dtype=torch.int8, device=dev)
        settle()
        for _ in range(warmup):
            Q.q8_linear_kq(x, W, sW, b, q8=qk2, s8=s8, C=y)
        start.record()
        for _ in range(steps):
            Q.q8_linear_kq(x, W, sW, b, q8=qk2, s8=s8, C=y)
        end.record()
        torch.cuda.synchronize()
        dl_ms = start.elapsed_time(end) / steps
        extra["drop_in_linear_us"] = dl_ms * 1e3
        extra["drop_in_linear_tops"] = ops / (dl_ms * 1e-3) / 1e12
    return {
        "value": ops / (ms * 1e-3) / 1e12, "ms": ms, "gemm_ms": gemm_ms, "prologue_ms": pro_ms,
        "roofline": {"bound": "mfma", "achieved": ops / (gemm_ms * 1e-3) / 1e12,
                     "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": ops / (gemm_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, "traffic": None},
        "dtype": "int8", "extra": extra,
    }


def bench_block(cfg, steps, warmup):
    """Config 1's MLP pair as the DiT runs it, fused against unfused.

    Fused: quant_rotate_mod -> GEMM up (bf16) -> quant_rotate with GELU-tanh
    in front (phi_hip_quant_rotate_act) -> GEMM down with the gated residual
    (phi_hip_i8_gemm_residual): four launches.  Unfused: the modulation, the
    GELU (bf16 out) and the residual update as separate elementwise passes,
    the projections as plain linears.  Reported: the fused block on K-tiled
    operands, with the row-major fused block and the unfused one beside it."""
    import torch

    import phi_qlinear as Q
    from phi_qlinear import synth

    dev = torch.device("cuda:0")
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    x = synth.activations(M, K, seed=0, device=dev)
    Wu = synth.int8_weight(N, K, seed=1, device=dev)
    Wd = synth.int8_weight(K, N, seed=2, device=dev)
    sW = synth.weight_scale(0.002, device=dev)
    bu = synth.bias(N, seed=3, device=dev)
    g = torch.Generator(device=dev).manual_seed(4)
    msc = torch.randn(K, generator=g, device=dev) * 0.1
    msh = torch.randn(K, generator=g, device=dev) * 0.1
    gate = torch.randn(K, generator=g, device=dev) * 0.1
    H = torch.randn(M, K, generator=g, device=dev)
    q8u = torch.empty((M, K), dtype=torch.int8, device=dev)
    s8u = torch.empty((M,), dtype=torch.float32, device=dev)
    q8d = torch.empty((M, N), dtype=torch.int8, device=dev)
    s8d = torch.empty((M,), dtype=torch.float32, device=dev)
    up = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    act = torch.empty_like(up)
    proj = torch.empty((M, K), dtype=torch.float32, device=dev)

    def fused():
        Q.quant_rotate(x, q=q8u, s=s8u, mod_scale=msc, mod_shift=msh)
        Q.i8_gemm(q8u, Wu, s8u, sW, bu, C=up)
        Q.quant_rotate(up, q=q8d, s=s8d, act="gelu_tanh")
        Q.i8_gemm_residual(q8d, Wd, s8d, sW, None, gate, H)

    # The same four launches on K-tiled operands (both weights packed once,
    # before timing).
    Wuk, Wdk = Q.pack_k_tiled(Wu), Q.pack_k_tiled(Wd)
    q8uk, q8dk = q8u.view(-1), q8d.view(-1)

    def fused_kt():
        Q.quant_rotate_kt(x, q=q8uk, s=s8u, mod_scale=msc, mod_shift=msh)
        Q.i8_gemm_kt(q8uk, Wuk, M, N, K, s8u, sW, bu, C=up)
        Q.quant_rotate_kt(up, q=q8dk, s=s8d, act="gelu_tanh")
        Q.i8_gemm_residual_kt(q8dk, Wdk, M, K, N, s8d, sW, None, gate, H)

    def unfused():
        xm = torch.addcmul(msh, x.float(), 1.0 + msc)  # the separate ModAdd pass
        Q.quant_rotate(xm, q=q8u, s=s8u)
        Q.i8_gemm(q8u, Wu, s8u, sW, bu, C=up)
        Q.gelu_tanh(up, out=act)
        Q.quant_rotate(act, q=q8d, s=s8d)
        Q.i8_gemm(q8d, Wd, s8d, sW, None, C=proj)
        H.addcmul_(proj, gate)  # the separate AddMul pass

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    ms_un = timed(unfused)
    ms_row = timed(fused)
    ms = timed(fused_kt)
    ops = 2 * 2.0 * M * N * K
    return {"value": ops / (ms * 1e-3) / 1e12, "ms": ms, "dtype": "int8",
            "roofline": {"bound": "mfma", "achieved": ops / (ms * 1e-3) / 1e12, "peak": INT8_PEAK_TOPS,
                         "unit": "TFLOP/s", "frac": ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS,
                         "traffic": None},
            "extra": {"fused_kt_us": ms * 1e3, "fused_row_major_us": ms_row * 1e3, "unfused_us": ms_un * 1e3}}


def bench_w4a8(cfg, steps, warmup):
    import torch

    import phi_qlinear as Q
    from phi_qlinear import synth

    dev = torch.device("cuda:0")
    M, K, N, group = cfg["M"], cfg["K"], cfg["N"], cfg["group"]
    x = synth.activations(M, K, seed=0, device=dev)
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=3, device=dev)
    lut, sw = Q.w4a8_prepare(codes, s_rel, Q.F16, sch, k=K, group=group, correction=corr)
    q8 = torch.empty((M, K), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def run(ws):
        for _ in range(warmup):
            Q.w4a8_linear(x, codes, lut, sw, group=group, q8=q8, s8=s8, C=y, workspace=ws)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            Q.w4a8_linear(x, codes, lut, sw, group=group, q8=q8, s8=s8, C=y, workspace=ws)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    # The in-register expansion (no workspace) and, when the library asks for
    # one, the expand-once path with a caller workspace; then the in-LDS
    # expansion from the band-packed weight (packed once, before timing).
    # The fastest is reported.
    ms_reg = run(None)
    ws = Q.w4a8_workspace(M, N, K, group, dev)
    ms_ws = run(ws) if ws is not None else None
    ms_band = None
    if K % 1024 == 0:
        banded = Q.w4a8_pack_banded(codes, lut, k=K, group=group)
        qk = q8.view(-1)
        for _ in range(warmup):
            Q.w4a8_linear_banded(x, banded, sw, N=N, group=group, q8=qk, s8=s8, C=y)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            Q.w4a8_linear_banded(x, banded, sw, N=N, group=group, q8=qk, s8=s8, C=y)
        end.record()
        torch.cuda.synchronize()
        ms_band = start.elapsed_time(end) / steps
    ms = min(t for t in (ms_reg, ms_ws, ms_band) if t is not None)
    ops = 2.0 * M * N * K
    return {"value": ops / (ms * 1e-3) / 1e12, "ms": ms, "dtype": "int8",
            "roofline": {"bound": "mfma", "achieved": ops / (ms * 1e-3) / 1e12, "peak": INT8_PEAK_TOPS,
                         "unit": "TFLOP/s", "frac": ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS,
                         "traffic": None},
            "extra": {"in_register_us": ms_reg * 1e3,
                      "expand_once_us": None if ms_ws is None else ms_ws * 1e3,
                      "in_lds_banded_us": None if ms_band is None else ms_band * 1e3}}


def bench_w4a4(cfg, steps, warmup):
    """One step: phi_hip_quant_rotate (qmax 7) then phi_hip_i4_gemm (fp32 out,
    as the reference), with and without the expand-once workspace; the faster
    is reported."""
    import torch

    import phi_qlinear as Q
    from phi_qlinear import synth

    dev = torch.device("cuda:0")
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    x = synth.activations(M, K, seed=0, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    B = torch.randint(0, 256, (N, K // 2), generator=g, device=dev, dtype=torch.uint8)
    sB = torch.rand(N, generator=g, device=dev) * 0.01 + 0.001
    q8 = torch.empty((M, K), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)

    def run(ws):
        def once():
            Q.quant_rotate(x, q=q8, s=s8, qmax=7.0)
            Q.i4_gemm(q8, B, s8, sB, C=y, workspace=ws)
        for _ in range(warmup):
            once()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            once()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    ms_reg = run(None)
    ws = Q.i4_workspace(M, N, K, dev)
    ms_ws = run(ws) if ws is not None else None
    ms = min(ms_reg, ms_ws) if ms_ws is not None else ms_reg
    ops = 2.0 * M * N * K
    return {"value": ops / (ms * 1e-3) / 1e12, "ms": ms, "dtype": "int8",
            "roofline": {"bound": "mfma", "achieved": ops / (ms * 1e-3) / 1e12, "peak": INT8_PEAK_TOPS,
                         "unit": "TFLOP/s", "frac": ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS,
                         "traffic": None},
            "extra": {"in_register_us": ms_reg * 1e3,
                      "expand_once_us": None if ms_ws is None else ms_ws * 1e3}}


def bench_lora(cfg, steps, warmup):
    """One step: phi_hip_lora_tail, out [M, N] fp32 += (x A^T) B^T with exact
    fp32 fma chains.  Throughput in TFLOP/s of fp32 fma work (2 (M R K + M N R)),
    against MI355X's fp32 vector peak."""
    import torch

    import phi_qlinear as Q

    dev = torch.device("cuda:0")
    M, K, N, R = cfg["M"], cfg["K"], cfg["N"], cfg["rank"]
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(M, K, generator=g, device=dev)
    A = torch.randn(R, K, generator=g, device=dev) * 0.02
    B = torch.randn(N, R, generator=g, device=dev) * 0.02
    out = torch.randn(M, N, generator=g, device=dev)
    h = torch.empty((M, R), dtype=torch.float32, device=dev)
    for _ in range(warmup):
        Q.lora_tail(x, A, B, out, h=h)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        Q.lora_tail(x, A, B, out, h=h)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    flops = 2.0 * (M * R * K + M * N * R)
    tf = flops / (ms * 1e-3) / 1e12
    return {"value": tf, "ms": ms, "dtype": "f32", "unit": "TFLOP/s",
            "roofline": {"bound": "valu", "achieved": tf, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": tf / FP32_PEAK_TFLOPS, "traffic": None}}


def bench_gemv(cfg, steps, warmup):
    import torch

    import phi_qlinear as Q
    from phi_qlinear import synth

    dev = torch.device("cuda:0")
    M, K, N, n = cfg["M"], cfg["K"], cfg["N"], cfg["items"]
    x = synth.activations(M, K, seed=0, device=dev)
    q8, s8 = Q.quant_rotate(x)
    Ws = [synth.int8_weight(N, K, seed=200 + i, device=dev) for i in range(n)]
    sc = [synth.weight_scale(0.002, device=dev) for _ in range(n)]
    outs = [torch.empty((M, N), dtype=torch.bfloat16, device=dev) for _ in range(n)]
    for _ in range(warmup):
        Q.gemv_batched(q8, s8, Ws, sc, outs=outs)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        Q.gemv_batched(q8, s8, Ws, sc, outs=outs)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    wbytes = float(n) * N * K
    gbs = wbytes / (ms * 1e-3) / 1e9
    return {"value": gbs, "ms": ms, "dtype": "int8", "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None}}


def bench_vendor(cfg, steps, warmup):
    """torch._int_mm (hipBLASLt's int8 GEMM) on the shape: A [M, K] row-major
    times B [N, K] row-major (the checkpoint layout, a column-major [K, N]
    view), int32 out.  Timed like the W8A8 bench's timed region."""
    import torch

    from phi_qlinear import synth

    dev = torch.device("cuda:0")
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    A = synth.int8_weight(M, K, seed=0, device=dev)
    B = synth.int8_weight(N, K, seed=1, device=dev)
    for _ in range(warmup):
        torch._int_mm(A, B.t())
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        torch._int_mm(A, B.t())
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"value": tops, "ms": ms, "dtype": "int8", "unit": "TOPS",
            "roofline": {"bound": "mfma", "achieved": tops, "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                         "frac": tops / INT8_PEAK_TOPS, "traffic": None}}


def bench_tiletrace(cfg, steps, warmup):
    """The headline step (K-tiled quantiser, then the GEMM) with the GEMM
    launched from the traced build of the pipeline (phi_probe_tile_trace):
    the same kernel code plus stamps per workgroup at each tile's start,
    K-loop end and epilogue end, in the 100 MHz real-time clock and in shader
    clock cycles.  The record of the last timed launch gives where a
    workgroup's time goes, averaged over workgroups.  With the bf16 output the
    tiles' transitions are fused: a tile's first K-step runs inside the
    previous tile's epilogue (the first tile's before its start stamp), so a
    K-loop span holds K/64 - 1 K-steps."""
    import ctypes

    import torch

    import phi_qlinear as Q
    from phi_qlinear import synth

    lib = ctypes.CDLL(os.path.join(PKG, "lib", "libphi_probe.so"))
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.phi_probe_tile_trace.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, P, ctypes.c_longlong]
    dev = torch.device("cuda:0")
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    x = synth.activations(M, K, seed=0, device=dev)
    W = synth.int8_weight(N, K, seed=1, device=dev)
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=2, device=dev)
    Wk = Q.pack_k_tiled(W)
    q8 = torch.empty((M * K,), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    slots = 1024 * 128
    rec = torch.zeros(slots, dtype=torch.int64, device=dev)
    # The library's plan: whole rounds of 256 x 256 tiles, the rest 128 x 128.
    big_rows = Q.big_tile_rows(M, N)
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        Q.quant_rotate_kt(x, q=q8, s=s8)
        rc = lib.phi_probe_tile_trace(stream, q8.data_ptr(), Wk.data_ptr(), s8.data_ptr(), sW.data_ptr(),
                                      b.data_ptr(), y.data_ptr(), M, N, K, big_rows, 1, rec.data_ptr(), slots)
        if rc != 0:
            raise RuntimeError(f"phi_probe_tile_trace failed ({rc})")

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    r = rec.view(-1, 128).cpu().tolist()
    used = [w for w in r if w[24] != 0]
    t0 = min(w[24] for w in used)
    us = lambda t: (t - t0) / 100.0  # 100 MHz real-time clock
    fused = K > 256  # the bf16 output without a gate at K > 256
    ksteps = K // 64 - (1 if fused else 0)

    def tiles(w, base, c=0):
        out = []
        for i in range(8):
            a, k, e = w[c + base + 3 * i], w[c + base + 3 * i + 1], w[c + base + 3 * i + 2]
            if w[base + 3 * i] == 0:
                break
            out.append(((k - a) / (100.0 if c == 0 else 1.0), (e - k) / (100.0 if c == 0 else 1.0)))
        return out

    big = [t for w in used for t in tiles(w, 0)]
    small = [t for w in used for t in tiles(w, 26)]
    big_c = [t for w in used for t in tiles(w, 0, 64)]
    small_c = [t for w in used for t in tiles(w, 26, 64)]
    by_round = {}
    for w in used:
        for i, t in enumerate(tiles(w, 0)):
            by_round.setdefault(i, []).append(t[0])
    per_wg = {}
    for w in used:
        n = len(tiles(w, 0))
        per_wg[n] = per_wg.get(n, 0) + 1
    mean = lambda v: sum(v) / len(v) if v else None
    first = [us(w[0] if w[0] else w[26]) for w in used if w[0] or w[26]]
    bigdone = [us(w[25]) for w in used if w[25]]
    ends = [us(w[50]) for w in used]
    cycles = [w[64 + 50] - w[64 + 24] for w in used]
    clock = [(w[64 + 50] - w[64 + 24]) / ((w[50] - w[24]) * 10.0) for w in used if w[50] > w[24]]  # GHz
    per_xcd = {}
    for w in used:
        d = per_xcd.setdefault(int(w[60]), [])
        d.append(us(w[25]) if w[25] else us(w[50]))
    ops = 2.0 * M * N * K
    extra = {
        "big_rows": big_rows, "workgroups": len(used), "ksteps_per_kloop": ksteps,
        "big_tiles": len(big), "big_kloop_us": mean([t[0] for t in big]), "big_epilogue_us": mean([t[1] for t in big]),
        "big_kloop_cycles_per_kstep": mean([t[0] / ksteps for t in big_c]) if big_c else None,
        "big_epilogue_cycles": mean([t[1] for t in big_c]),
        "small_tiles": len(small), "small_kloop_us": mean([t[0] for t in small]),
        "small_epilogue_us": mean([t[1] for t in small]),
        "small_kloop_cycles_per_kstep": mean([t[0] / ksteps for t in small_c]) if small_c else None,
        "small_epilogue_cycles": mean([t[1] for t in small_c]),
        "workgroup_cycles": {"mean": mean(cycles), "max": max(cycles)},
        "shader_clock_ghz": mean(clock),
        "first_tile_start_us": mean(first),
        "workgroup_start_us": {"min": min(us(w[24]) for w in used), "mean": mean([us(w[24]) for w in used]),
                               "max": max(us(w[24]) for w in used)},
        "workgroup_setup_us": mean([(w[0] if w[0] else w[26]) / 100.0 - w[24] / 100.0 for w in used if w[0] or w[26]]),
        "big_phase_end_us": {"min": min(bigdone), "mean": mean(bigdone), "max": max(bigdone)} if bigdone else None,
        "kernel_end_us": {"min": min(ends), "mean": mean(ends), "max": max(ends)},
        "big_phase_end_by_xcd_us": {str(k): round(mean(v), 2) for k, v in sorted(per_xcd.items())},
        "big_kloop_by_tile_us": {str(k): round(mean(v), 2) for k, v in sorted(by_round.items())},
        "workgroups_by_big_tiles": {str(k): v for k, v in sorted(per_wg.items())},
    }
    log("bench: tile trace " + json.dumps(extra))
    return {"value": ops / (ms * 1e-3) / 1e12, "ms": ms, "dtype": "int8", "unit": "TOPS",
            "roofline": {"bound": "mfma", "achieved": ops / (ms * 1e-3) / 1e12, "peak": INT8_PEAK_TOPS,
                         "unit": "TFLOP/s", "frac": ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, "traffic": None},
            "extra": extra}


def bench_t272trace(cfg, steps, warmup):
    """The headline step (K-tiled quantiser, then the GEMM) with the GEMM
    launched from the traced build of the 272 x 192 kernel
    (phi_probe_t272_trace): the same kernel code plus shader-clock stamps per
    workgroup at each tile's start, K-loop end and epilogue end.  The record
    of the last timed launch gives where a workgroup's time goes: clocks a
    K-step against the 816 of MFMA issue (51 MFMAs of 16 clocks), the
    epilogue, and the set-up before the first tile."""
    import ctypes

    import torch

    import phi_qlinear as Q
    from phi_qlinear import synth

    lib = ctypes.CDLL(os.path.join(PKG, "lib", "libphi_probe.so"))
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.phi_probe_t272_trace.argtypes = [P, P, P, P, P, P, P, I, I, I, P, ctypes.c_longlong, I]
    lib.phi_probe_t272w4_trace.argtypes = [P, P, P, ctypes.c_longlong, P, I, P, P, P, P, I, I, I, P,
                                           ctypes.c_longlong]
    dev = torch.device("cuda:0")
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    group = cfg.get("group")  # W4A8: the codes expanded in LDS (i8_gemm_t272w4_kernel)
    kt = cfg.get("layout", "kt") == "kt"  # row: the activations and the weight row-major
    x = synth.activations(M, K, seed=0, device=dev)
    b = synth.bias(N, seed=2, device=dev)
    if group:
        codes, s_rel, sch, corr = synth.w4a8_weight(N, K, group, seed=3, device=dev)
        lut, sW = Q.w4a8_prepare(codes, s_rel, Q.F16, sch, k=K, group=group, correction=corr)
    else:
        W = synth.int8_weight(N, K, seed=1, device=dev)
        sW = synth.weight_scale(0.002, device=dev)
        Wk = Q.pack_k_tiled(W) if kt else W
    q8 = torch.empty((M * K,), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    slots = 1024 * 64
    rec = torch.zeros(slots, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        if kt:
            Q.quant_rotate_kt(x, q=q8, s=s8)
        else:
            Q.quant_rotate(x, q=q8.view(M, K), s=s8)
        if group:
            rc = lib.phi_probe_t272w4_trace(stream, q8.data_ptr(), codes.data_ptr(), codes.stride(0),
                                            lut.data_ptr(), group, s8.data_ptr(), sW.data_ptr(), b.data_ptr(),
                                            y.data_ptr(), M, N, K, rec.data_ptr(), slots)
        else:
            rc = lib.phi_probe_t272_trace(stream, q8.data_ptr(), Wk.data_ptr(), s8.data_ptr(), sW.data_ptr(),
                                          b.data_ptr(), y.data_ptr(), M, N, K, rec.data_ptr(), slots, 1 if kt else 0)
        if rc != 0:
            raise RuntimeError(f"phi_probe_t272_trace failed ({rc})")

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    used = [w for w in rec.view(-1, 64).cpu().tolist() if w[0] != 0]
    ksteps = K // 64
    kl, ep, setup = [], [], []
    for w in used:
        setup.append(w[1] - w[0])
        for i in range(16):
            a, k, e = w[1 + 3 * i], w[2 + 3 * i], w[3 + 3 * i]
            if a == 0:
                break
            kl.append(k - a)
            ep.append(e - k)
    cycles = [w[49] - w[0] for w in used]
    clock = [(w[49] - w[0]) / ((w[52] - w[51]) * 10.0) for w in used if w[52] > w[51]]  # GHz
    t0 = min(w[51] for w in used)
    per_xcd = {}
    for w in used:
        per_xcd.setdefault(int(w[50]), []).append((w[52] - t0) / 100.0)
    mean = lambda v: sum(v) / len(v) if v else None
    extra = {
        "workgroups": len(used), "tiles": len(kl), "ksteps_per_tile": ksteps,
        "kloop_cycles_per_kstep": mean(kl) / ksteps, "mfma_issue_cycles_per_kstep": 51 * 16,
        "epilogue_cycles": mean(ep), "setup_cycles": mean(setup),
        "workgroup_cycles": {"mean": mean(cycles), "max": max(cycles)},
        "mfma_issue_share": 51 * 16 * ksteps * len(kl) / len(used) / mean(cycles),
        "shader_clock_ghz": mean(clock),
        "kernel_end_by_xcd_us": {str(k): round(mean(v), 2) for k, v in sorted(per_xcd.items())},
    }
    log("bench: t272 tile trace " + json.dumps(extra))
    ops = 2.0 * M * N * K
    return {"value": ops / (ms * 1e-3) / 1e12, "ms": ms, "dtype": "int8", "unit": "TOPS",
            "roofline": {"bound": "mfma", "achieved": ops / (ms * 1e-3) / 1e12, "peak": INT8_PEAK_TOPS,
                         "unit": "TFLOP/s", "frac": ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, "traffic": None},
            "extra": extra}


def bench_convref(cfg, steps, warmup):
    """torch's elementwise bf16 -> int8 conversion over the prologue's
    activation tensor: the prologue's HBM bytes with none of its work."""
    import torch

    from phi_qlinear import synth

    dev = torch.device("cuda:0")
    M, K = cfg["M"], cfg["K"]
    x = synth.activations(M, K, seed=0, device=dev)
    q = torch.empty((M, K), dtype=torch.int8, device=dev)
    for _ in range(warmup):
        q.copy_(x)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        q.copy_(x)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    gbs = 3.0 * M * K / (ms * 1e-3) / 1e9
    # A plain bf16 copy of the same tensor (4K bytes a row moved).
    x2 = torch.empty_like(x)
    for _ in range(warmup):
        x2.copy_(x)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        x2.copy_(x)
    end.record()
    torch.cuda.synchronize()
    ms_copy = start.elapsed_time(end) / steps
    return {"value": gbs, "ms": ms, "dtype": "bf16", "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None},
            "extra": {"convert_us": ms * 1e3, "copy_us": ms_copy * 1e3,
                      "copy_gbs": 4.0 * M * K / (ms_copy * 1e-3) / 1e9}}


def bench_prologue_floor(cfg, steps, warmup):
    """The rotate+quantise prologue (quant_rotate_kt, K-tiled codes) against
    what its memory pattern alone costs: phi_probe_prologue_stream loads the
    same bf16 rows and stores the same 16-byte code chunks on the same launch
    shape, without the rotation and quantisation (mode 0, K-tiled and
    row-major stores), and with the LDS round trips and barrier added (mode
    1); and torch's bf16 -> int8 conversion of the tensor.  Interleaved
    rounds in one process, median per variant."""
    import ctypes
    import statistics

    import torch

    import phi_qlinear as Q
    from phi_qlinear import synth

    dev = torch.device("cuda:0")
    M, K = cfg["M"], cfg["K"]
    G = K // 256
    x = synth.activations(M, K, seed=0, device=dev)
    q = torch.empty((M * K,), dtype=torch.int8, device=dev)
    s = torch.empty((M,), dtype=torch.float32, device=dev)
    q2 = torch.empty((M, K), dtype=torch.int8, device=dev)
    lib = ctypes.CDLL(os.path.join(PKG, "lib", "libphi_probe.so"))
    lib.phi_probe_prologue_stream.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int]
    stream = torch.cuda.current_stream().cuda_stream

    def probe(mode, kt, run=0):
        def go():
            rc = lib.phi_probe_prologue_stream(stream, x.data_ptr(), M, G, q.data_ptr(), s.data_ptr(), mode, kt, run)
            if rc != 0:
                raise RuntimeError(f"prologue stream probe failed ({rc})")
        return go

    # The prologue variants call the C ABI directly, with the A/B switches set
    # once per variant (setup), so that the host keeps ahead of ~10 us
    # launches: under a kernel tracer, where host calls are slower, the launches
    # sit ~20 us apart while each runs ~10 us.
    qlib = Q.load()

    def prologue(lg_run=3, rounds=0):
        def go():
            rc = qlib.phi_hip_quant_rotate_kt(stream, x.data_ptr(), Q.BF16, M, K, K, q.data_ptr(), s.data_ptr(),
                                              127.0, Q.ROUND_HALF_AWAY)
            if rc != 0:
                raise RuntimeError(f"quant_rotate_kt failed ({rc})")

        def setup():
            os.environ["PHI_QR_RUN"] = str(lg_run)
            os.environ["PHI_QR_ROUNDS"] = str(rounds)
        go.setup = setup
        return go

    variants = {
        "prologue": prologue(),
        "prologue_run1": prologue(0),
        **{f"prologue_r{r}": prologue(3, r) for r in range(1, 6)},
        "stream_kt": probe(0, 1),
        "stream_kt_run2": probe(0, 1, 2),
        "stream_kt_run4": probe(0, 1, 4),
        "stream_kt_run8": probe(0, 1, 8),
        "stream_row_major": probe(0, 0),
        "stream_lds_kt": probe(1, 1),
        "torch_convert": lambda: q2.copy_(x),
    }
    times = {k: [] for k in variants}
    same = {}
    variants["prologue"].setup()
    variants["prologue"]()
    torch.cuda.synchronize()
    q_ref, s_ref = q.clone(), s.clone()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for rnd in range(3):
        for name, fn in variants.items():
            if name.startswith("prologue"):
                q.zero_()
                s.zero_()
                fn.setup()
            if name == "prologue":
                # The round's first prologue variant follows lighter kernels
                # (the stream probes, torch's copy).  A kernel trace shows the
                # board's clock transient there: launches 1-50 fast, then
                # 25 % slower, recovering over some hundreds of launches.
                # Without 1000 untimed launches first, this variant measured
                # 6-8 % slower than the identical forced-R variant after it.
                for _ in range(max(3 * warmup, 1000)):
                    fn()
            for _ in range(warmup):
                fn()
            start.record()
            for _ in range(steps):
                fn()
            end.record()
            torch.cuda.synchronize()
            times[name].append(start.elapsed_time(end) / steps * 1e3)
            if name.startswith("prologue"):
                same[name] = bool(torch.equal(q, q_ref) and torch.equal(s, s_ref)) and same.get(name, True)
    os.environ.pop("PHI_QR_RUN", None)
    os.environ.pop("PHI_QR_ROUNDS", None)
    us = {k: statistics.median(v) for k, v in times.items()}
    nbytes = 3.0 * M * K + 4.0 * M
    gbs = nbytes / (us["prologue"] * 1e-6) / 1e9
    return {"value": gbs, "ms": us["prologue"] * 1e-3, "dtype": "bf16", "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None},
            "extra": {"us": {k: round(v, 2) for k, v in us.items()}, "codes_equal": same,
                      "gbs": {k: round(nbytes / (v * 1e-6) / 1e9, 1) for k, v in us.items()},
                      "rounds_us": {k: [round(t, 2) for t in v] for k, v in times.items()}}}


def bench_ceiling(steps, warmup):
    """The two ceilings the headline GEMM is argued against, from the probe
    kernels of lib/libphi_probe.so: every wave of every CU issues int8 MFMAs
    back to back on 16 accumulators (zero operands; one static random fragment
    pair; the GEMM's 8 + 8 random fragments, changed every K-step), and every
    wave streams operands into LDS the way the GEMM's pipeline does (no
    MFMAs), from a window that fits the MALL and one that does not."""
    import ctypes

    import torch

    lib = ctypes.CDLL(os.path.join(PKG, "lib", "libphi_probe.so"))
    lib.phi_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_int]
    lib.phi_probe_lds_dma.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_int]
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator(device=dev).manual_seed(7)
    ops = torch.randint(-127, 128, (64 * 1024,), generator=g, device=dev, dtype=torch.int8)
    sink = torch.zeros(cus * 4, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def timed(launch):
        for _ in range(warmup):
            launch()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            launch()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps * 1e-3

    iters = 2000  # 64000 MFMAs a wave, about 1 ms a launch
    tops = {}
    for mode, name in ((0, "zero"), (1, "static"), (2, "rotating"), (6, "zero_16x16x64"),
                       (5, "rotating_16x16x64")):
        def launch(mode=mode):
            rc = lib.phi_probe_mfma(stream, ctypes.c_void_p(ops.data_ptr()), mode, iters,
                                    ctypes.c_void_p(sink.data_ptr()), cus)
            if rc != 0:
                raise RuntimeError(f"mfma probe launch failed ({rc})")
        secs = timed(launch)
        tops[name] = cus * 4 * iters * 32 * 65536 / secs / 1e12
        log(f"bench: mfma ceiling ({name} operands) {tops[name]:.0f} TOPS")
    dma = {}
    for label, window in (("mall", 32 << 20), ("hbm", 1536 << 20)):
        buf = torch.randint(-127, 128, (window,), generator=g, device=dev, dtype=torch.int8)
        dma_iters = 4000

        def launch(buf=buf, window=window):
            rc = lib.phi_probe_lds_dma(stream, ctypes.c_void_p(buf.data_ptr()), window, dma_iters,
                                       ctypes.c_void_p(sink.data_ptr()), cus)
            if rc != 0:
                raise RuntimeError(f"lds dma probe launch failed ({rc})")
        secs = timed(launch)
        dma[label] = cus * 4 * dma_iters * 8 * 1024 / secs / 1e9
        log(f"bench: LDS DMA stream ({label} window) {dma[label]:.0f} GB/s")
        del buf
    # VALU work beside the MFMAs: V v_perm_b32 after every MFMA (the W4 table
    # lookup's instruction), the rotating operands of mode 2.
    lib.phi_probe_mfma_valu.argtypes = lib.phi_probe_mfma.argtypes
    beside = {}
    for v in (0, 1, 2, 3, 4, 6, 8):
        def launch(v=v):
            rc = lib.phi_probe_mfma_valu(stream, ctypes.c_void_p(ops.data_ptr()), v, iters,
                                         ctypes.c_void_p(sink.data_ptr()), cus)
            if rc != 0:
                raise RuntimeError(f"mfma+valu probe launch failed ({rc})")
        secs = timed(launch)
        beside[str(v)] = cus * 4 * iters * 32 * 65536 / secs / 1e12
        log(f"bench: mfma with {v} VALU ops beside each: {beside[str(v)]:.0f} TOPS")
    # The same MFMA-only loop (rotating 16x16x64 operands) in the driver's
    # window: after an idle second, 25 launches of about one headline GEMM's
    # length (170 iterations), each timed by its own events; launches 6-25 are
    # the ones `--steps 20 --warmup 5` times.
    win_iters = 170
    window = []
    for _ in range(2):
        torch.cuda.synchronize()
        time.sleep(1.0)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(26)]
        ev[0].record()
        for i in range(25):
            rc = lib.phi_probe_mfma(stream, ctypes.c_void_p(ops.data_ptr()), 5, win_iters,
                                    ctypes.c_void_p(sink.data_ptr()), cus)
            if rc != 0:
                raise RuntimeError(f"mfma probe launch failed ({rc})")
            ev[i + 1].record()
        torch.cuda.synchronize()
        us = [ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(25)]
        w_ops = cus * 4 * win_iters * 32 * 65536
        w_tops = w_ops / (sum(us[5:25]) / 20 * 1e-6) / 1e12
        window.append({"launch_us": [round(u, 1) for u in us], "tops_launches_6_25": w_tops,
                       "frac_launches_6_25": w_tops / INT8_PEAK_TOPS})
        log(f"bench: mfma ceiling in the driver's window (rotating_16x16x64, launches 6-25) {w_tops:.0f} TOPS "
            f"({w_tops / INT8_PEAK_TOPS:.3f}); per launch us {[round(u) for u in us]}")
    value = tops["rotating"]
    return {"value": value, "ms": None, "dtype": "int8", "unit": "TOPS",
            "roofline": {"bound": "mfma", "achieved": value, "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                         "frac": value / INT8_PEAK_TOPS, "traffic": None},
            "extra": {"mfma_tops": tops, "lds_dma_gbs": dma, "mfma_tops_with_valu_per_mfma": beside,
                      "cus": cus, "mfma_per_wave_per_launch": iters * 32,
                      "rotating_16x16x64_in_driver_window": window}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 300 warm-up steps (about 70 ms of GPU work at the headline shape) bring
    # the clocks to their steady state; 10 leave the GEMM ~10 % slower.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--config", default="c1_up", choices=sorted(CONFIGS))
    ap.add_argument("--layout", default="kt", choices=["kt", "row"],
                    help="W8A8 operands: K-tiled (weight packed before timing) or row-major")
    ap.add_argument("--weights", default="uniform", choices=["uniform", "gaussian"],
                    help="W8A8 weight codes: uniform int8, or the reference benchmark's rotated, "
                         "per-row quantised N(0, 1) weights")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU (one MI355X); multi-GPU runs are not part of it",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    cfg = CONFIGS[args.config]
    log(f"bench: config {args.config} {cfg}, warmup {args.warmup}, steps {args.steps}")
    if cfg["kind"] == "w8a8":
        r = bench_w8a8(cfg, args.steps, args.warmup, args.layout, args.weights)
    elif cfg["kind"] == "block":
        r = bench_block(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "w4a8":
        r = bench_w4a8(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "w4a4":
        r = bench_w4a4(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "lora":
        r = bench_lora(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "tiletrace":
        r = bench_tiletrace(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "t272trace":
        r = bench_t272trace(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "convref":
        r = bench_convref(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "qrfloor":
        r = bench_prologue_floor(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "vendor":
        r = bench_vendor(cfg, args.steps, args.warmup)
    elif cfg["kind"] == "ceiling":
        r = bench_ceiling(min(args.steps, 20), min(args.warmup, 20))
    else:
        r = bench_gemv(cfg, args.steps, args.warmup)
    if r["ms"] is not None:
        log(f"bench: {r['ms'] * 1e3:.1f} us per step")
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
    r["roofline"]["traffic"] = traffic_for(args.config)

    cpu = None
    if not args.no_cpu_baseline and cfg["kind"] == "w8a8":
        log("bench: timing the reference CPU path on a row sample ...")
        cpu = cpu_baseline(cfg)
    unit = r.get("unit", "TOPS")
    workload = {"c1_up": "W8A8 linear M=4352 K=3072 N=12288 (config 1 up-projection)"}.get(
        args.config, f"{args.config} {cfg}")
    line = {
        "metric": METRIC if args.config == "c1_up" else f"{args.config} {unit}",
        "value": r["value"], "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": r["ms"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": r["dtype"],
        "data": "synthetic (seeded: bf16 N(0,1) activations with 0.1% x20 outlier channels, "
                + ("N(0,1) weights rotated and quantised per row to int8 with per-row scales "
                   "(the reference benchmark's weights)" if args.weights == "gaussian"
                   else "int8 U[-127,127] weights, scale 0.002") + ", bf16 N(0,0.02) bias)",
        "config": {"workload": workload, **{k: v for k, v in cfg.items() if k != "kind"},
                   **({"operand_layout": "k-tiled" if args.layout == "kt" else "row-major",
                       "weights": args.weights} if cfg["kind"] == "w8a8" else {}),
                   "parallelism": "single GPU"},
        "roofline": r["roofline"], "cpu_baseline": cpu,
    }
    if "extra" in r:
        line["extra"] = r["extra"]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
