"""CPU oracle for the quantized-linear hot path -- TEST INFRASTRUCTURE ONLY.

numpy front end over ``liboracle.so`` (this repo's C restatement of the
reference's host arithmetic, ``oracle/oracle.c``) and over ``_ref/phiref``
(the reference's own ``core/host/quant.cpp`` compiled from its sources).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package; the product library never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_EXE = os.path.join(HERE, "_ref", "phiref")

F32, BF16, F16, I32, I8, F8_E4M3, F8_E5M2, U8_E4M3 = range(8)
ROUND_HALF_AWAY, ROUND_HALF_EVEN, ROUND_DEVICE_FLOOR = 0, 1, 2

_lib = None


def build(quiet: bool = True) -> None:
    """Compile liboracle.so (and _ref/phiref when the reference is mounted)."""
    out = subprocess.run(["make", "-C", HERE], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.orc_quantize_rows.argtypes = [P, I, I64, I64, I64, I, ctypes.c_float, I, P, P]
        L.orc_quantize_rows.restype = I
        L.orc_convrot_rows.argtypes = [P, P, I64, I64]
        L.orc_gemm_i8_i32.argtypes = [P, I64, P, I64, I64, I64, I64, P]
        L.orc_epilogue.argtypes = [P, I64, I64, P, P, I, P, I, I, P, I]
        L.orc_w4a8_expand.argtypes = [P, I64, P, I, I64, P, I, P, P, I64, I64, I64, I, P, P, P]
        L.orc_w4a8_expand.restype = I
        L.orc_gelu_tanh.argtypes = [P, P, I64]
        L.orc_silu_gate.argtypes = [P, P, I64, I64]
        L.orc_lora_down.argtypes = [P, I64, P, P, I64, I64, I64]
        L.orc_lora_rank_add.argtypes = [P, P, P, I64, I64, I64, I64]
        L.orc_quantize_convrot_w4a4.argtypes = [P, I64, I64, P, P]
        L.orc_quantize_convrot_w4a4.restype = I
        L.orc_int4_gemm.argtypes = [P, I64, P, I64, P, P, I64, I64, I64, P, I64]
        L.orc_mod_add.argtypes = [P, P, P, P, I64, I64]
        L.orc_add_mul.argtypes = [P, P, P, P, I64, I64]
        L.orc_f32_to_bf16_n.argtypes = [P, P, I64]
        L.orc_bf16_to_f32_n.argtypes = [P, P, I64]
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f8_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_f8_e4m3_to_f32.restype = ctypes.c_float
        L.orc_f8_e5m2_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_f8_e5m2_to_f32.restype = ctypes.c_float
        L.orc_scale_at.argtypes = [P, I, I64]
        L.orc_scale_at.restype = ctypes.c_float
        L.orc_dequant_fp8_rows.argtypes = [P, I64, I64, I64, I, P, P]
        L.orc_dequant_fp4_rows.argtypes = [P, I64, I64, I64, I64, P, I, I64, I64, I64, P, P]
        L.orc_round_forms_differ.argtypes = [P, I64]
        L.orc_round_forms_differ.restype = I64
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- conversions
def f32_to_bf16(x) -> np.ndarray:
    """fp32 -> bf16 bits (uint16), RNE by the reference's carry rule."""
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_p(x), _p(y), x.size)
    return y


def bf16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_f32_n(_p(h), _p(y), h.size)
    return y


def scale_table_to_f32(table: np.ndarray, dtype: int) -> np.ndarray:
    """Decode a scale table stored as f32/f16/bf16/e4m3/e5m2/u8-e4m3."""
    t = np.ascontiguousarray(table)
    return np.array([lib().orc_scale_at(_p(t), dtype, i) for i in range(t.size)],
                    np.float32).reshape(t.shape)


# ---------------------------------------------------------------- A1 / A2
def convrot(x) -> np.ndarray:
    x = _c(x, np.float32)
    rows, cols = x.shape
    assert cols % 256 == 0
    y = np.empty_like(x)
    lib().orc_convrot_rows(_p(x), _p(y), rows, cols)
    return y


def quantize_rows(x, *, rotate=True, qmax=127.0, round_mode=ROUND_HALF_AWAY, x_is_bf16=None):
    """Rotate (optionally) and quantise rows -> (q int8 [rows, cols], s f32 [rows]).

    ``x`` is float32, or uint16 bf16 bits (``x_is_bf16`` defaults to the dtype).
    """
    x = np.ascontiguousarray(x)
    if x_is_bf16 is None:
        x_is_bf16 = x.dtype == np.uint16
    x = _c(x, np.uint16 if x_is_bf16 else np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows,), np.float32)
    rc = lib().orc_quantize_rows(_p(x), BF16 if x_is_bf16 else F32, rows, cols, cols,
                                 1 if rotate else 0, float(qmax), round_mode, _p(q), _p(s))
    if rc != 0:
        raise ValueError(f"quantize_rows: cols={cols} is not a multiple of 256")
    return q, s


def dequant_fp8_rows(codes, dtype, scale=None) -> np.ndarray:
    """fp8 weight rows in fp32: f8(code) * scale[r] (dequant_fp8_row,
    core/host/quant.cpp:433-439).  codes uint8 [rows, k]; dtype F8_E4M3 or
    F8_E5M2; scale None or float32 [rows]."""
    codes = _c(codes, np.uint8)
    rows, k = codes.shape
    sc = None if scale is None else _c(np.broadcast_to(np.asarray(scale, np.float32).reshape(-1), (rows,)), np.float32)
    out = np.empty((rows, k), np.float32)
    lib().orc_dequant_fp8_rows(_p(codes), k, rows, k, dtype, _p(sc), _p(out))
    return out


def dequant_fp4_rows(codes, k, table=None, table_dtype=F8_E4M3, block=16, global_scale=None, row0=0) -> np.ndarray:
    """nvfp4 / mxfp4 weight rows row0 .. row0 + rows - 1 in fp32
    (dequant_nvfp4_row, core/host/quant.cpp:390-431): codes uint8 [rows, >= k/2]
    (even column in the high nibble), table the stored 2-D block-scale table
    (cuBLAS tiled layout) as raw elements of table_dtype (uint8 for the fp8
    spellings, uint16 bits for f16/bf16, float32), global_scale None or float32
    [rows] / [1]."""
    codes = _c(codes, np.uint8)
    rows, ld = codes.shape
    if table is not None:
        table = np.ascontiguousarray(table)
        t_rows, t_cols = table.shape if table.ndim == 2 else (1, table.size)
    else:
        t_rows = t_cols = 0
    g = None if global_scale is None else _c(np.broadcast_to(np.asarray(global_scale, np.float32).reshape(-1),
                                                             (rows,)), np.float32)
    out = np.empty((rows, k), np.float32)
    lib().orc_dequant_fp4_rows(_p(codes), ld, row0, rows, k, _p(table), table_dtype, t_rows, t_cols, block, _p(g),
                               _p(out))
    return out


def round_forms_differ(cap: int = 16) -> tuple[int, np.ndarray]:
    """Every fp32 d with |d| <= 128 where the host rule (ROUND_HALF_AWAY, double
    arithmetic, core/host/quant.cpp:163-166) and the reference device kernel's
    fp32 floorf(d + 0.5f) form (ROUND_DEVICE_FLOOR, core/kernels/int8_gemm.cpp:777-780)
    give different codes: (count, the first `cap` of them)."""
    out = np.zeros(cap, np.float32)
    n = lib().orc_round_forms_differ(_p(out), cap)
    return int(n), out[:min(n, cap)]


# ---------------------------------------------------------------- A4 / A5
def gemm_i8_i32(a, b) -> np.ndarray:
    a = _c(a, np.int8)
    b = _c(b, np.int8)
    M, K = a.shape
    N = b.shape[0]
    acc = np.empty((M, N), np.int32)
    lib().orc_gemm_i8_i32(_p(a), K, _p(b), K, M, N, K, _p(acc))
    return acc


def gemm_i8_i32_fast(a, b) -> np.ndarray:
    """Same integer product via a float64 BLAS matmul (a library routine).

    Exact: every partial sum is an integer below K * 127^2 < 2^53."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape[1] * 127 * 127 < 2 ** 53
    return (a @ b.T).astype(np.int64).astype(np.int32)


def epilogue(acc, sa, sb, bias=None, *, out="bf16", fused=True):
    """((float)acc*sa[m]) * sb[n] (+ bias[n]) -> bf16 bits (uint16) or f32.

    ``sb`` of size 1 is a per-tensor scale.  ``bias`` is float32, or uint16
    bf16 bits.  ``fused`` selects fma(t, sb, bias) (the reference device
    epilogue) over separately rounded (t*sb)+bias.
    """
    acc = _c(acc, np.int32)
    M, N = acc.shape
    sa = _c(sa, np.float32)
    sb = _c(sb, np.float32).reshape(-1)
    bdt = -1
    if bias is not None:
        bias = np.ascontiguousarray(bias)
        bdt = BF16 if bias.dtype == np.uint16 else F32
        bias = _c(bias, np.uint16 if bdt == BF16 else np.float32)
    if out == "bf16":
        y = np.empty((M, N), np.uint16)
        odt = BF16
    else:
        y = np.empty((M, N), np.float32)
        odt = F32
    lib().orc_epilogue(_p(acc), M, N, _p(sa), _p(sb), 1 if sb.size == 1 else 0, _p(bias), bdt,
                       1 if fused else 0, _p(y), odt)
    return y


def q8_linear(x, w, sw, bias=None, *, out="bf16", round_mode=ROUND_HALF_AWAY):
    """The full W8A8 linear: rotate+quantise x, int8 GEMM, epilogue.

    Returns (y, q, s, acc)."""
    q, s = quantize_rows(x, rotate=True, round_mode=round_mode)
    acc = gemm_i8_i32_fast(q, w)
    y = epilogue(acc, s, sw, bias, out=out)
    return y, q, s, acc


# ---------------------------------------------------------------- A7
def w4a8_expand(codes, s_rel, s_rel_dtype, s_channel, *, k, group, codebook=None,
                correction=None, layout=0, srel_row_bytes=None, codes_row_bytes=None,
                return_values=False):
    """Decode a grouped 4-bit (layout 0) / 6-bit (layout 1) weight and requantise
    each row -> (q int8 [rows, k], s f32 [rows]) [, values f32 [rows, k]]."""
    codes = _c(codes, np.uint8)
    rows = codes.shape[0]
    crb = codes_row_bytes or codes.shape[1]
    s_rel = np.ascontiguousarray(s_rel) if s_rel is not None else None
    srb = srel_row_bytes or (s_rel.strides[0] if s_rel is not None else 0)
    sch = None if s_channel is None else _c(s_channel, np.float32).reshape(-1)
    cb = None if codebook is None else _c(codebook, np.float32)
    corr = None if correction is None else _c(correction, np.float32)
    q = np.empty((rows, k), np.int8)
    s = np.empty((rows,), np.float32)
    vals = np.empty((rows, k), np.float32) if return_values else None
    rc = lib().orc_w4a8_expand(_p(codes), crb, _p(s_rel), s_rel_dtype, srb, _p(sch),
                               1 if (sch is not None and sch.size == 1) else 0, _p(cb),
                               _p(corr), rows, k, group, layout, _p(q), _p(s), _p(vals))
    if rc != 0:
        raise ValueError("w4a8_expand: bad geometry")
    return (q, s, vals) if return_values else (q, s)


def mod_add(a, b, c) -> np.ndarray:
    """adaLN ModAdd per column: fma(a, 1 + b[col], c[col]) (b, c may be None)."""
    a = _c(a, np.float32)
    rows, cols = a.shape
    b = None if b is None else _c(b, np.float32).reshape(-1)
    c = None if c is None else _c(c, np.float32).reshape(-1)
    y = np.empty_like(a)
    lib().orc_mod_add(_p(a), _p(b), _p(c), _p(y), rows, cols)
    return y


def add_mul(a, b, c) -> np.ndarray:
    """Gated residual AddMul per column: fma(b, c[col], a)."""
    a = _c(a, np.float32)
    rows, cols = a.shape
    b = _c(b, np.float32)
    c = _c(c, np.float32).reshape(-1)
    y = np.empty_like(a)
    lib().orc_add_mul(_p(a), _p(b), _p(c), _p(y), rows, cols)
    return y


def gelu_tanh(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_gelu_tanh(_p(x), _p(y), x.size)
    return y


def quantize_convrot_w4a4(w):
    """Signed-int4 weight packer (core/host/quant.cpp:247-272): (packed u8 [rows, cols/2], scales f32 [rows])."""
    w = _c(w, np.float32)
    rows, cols = w.shape
    packed = np.empty((rows, cols // 2), dtype=np.uint8)
    scales = np.empty(rows, dtype=np.float32)
    if lib().orc_quantize_convrot_w4a4(_p(w), rows, cols, _p(packed), _p(scales)) != 0:
        raise ValueError("quantize_convrot_w4a4: cols is not a multiple of 256")
    return packed, scales


def int4_gemm(a, b_packed, sa, sb) -> np.ndarray:
    """C = ((float)(A . unpack(B)^T) * sa) * sb, fp32 (core/kernels/h3_kernels.cpp:546-635)."""
    a, b = _c(a, np.int8), _c(b_packed, np.uint8)
    M, K = a.shape
    N = b.shape[0]
    c = np.empty((M, N), dtype=np.float32)
    lib().orc_int4_gemm(_p(a), K, _p(b), b.shape[1], _p(_c(sa, np.float32)), _p(_c(sb, np.float32)),
                        M, N, K, _p(c), N)
    return c


def lora_down(x, a) -> np.ndarray:
    """h [M, R] = x [M, K] . a [R, K]^T as k-ordered fp32 fma chains (fp32 x)."""
    x, a = _c(x, np.float32), _c(a, np.float32)
    M, K = x.shape
    R = a.shape[0]
    h = np.empty((M, R), dtype=np.float32)
    lib().orc_lora_down(_p(x), K, _p(a), _p(h), M, K, R)
    return h


def lora_rank_add(h, b, c) -> np.ndarray:
    """c + h . b^T as r-ordered fp32 fma chains starting from c (returns a new array)."""
    h, b = _c(h, np.float32), _c(b, np.float32)
    out = np.array(c, dtype=np.float32, copy=True, order="C")
    M, N = out.shape
    lib().orc_lora_rank_add(_p(h), _p(b), _p(out), N, M, N, h.shape[1])
    return out


def silu_gate(gx) -> np.ndarray:
    """silu(gx[:, :cols]) * gx[:, cols:] for gx [rows, 2 cols], fp32."""
    gx = _c(gx, np.float32)
    rows, two = gx.shape
    out = np.empty((rows, two // 2), dtype=np.float32)
    lib().orc_silu_gate(_p(gx), _p(out), rows, two // 2)
    return out


# ---------------------------------------------------------------- _ref driver
def ref_available() -> bool:
    return os.path.exists(REF_EXE)


def _ref_run(args):
    out = subprocess.run([REF_EXE] + [str(a) for a in args], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"phiref {args[0]} failed: {out.stderr}")
    return out.stdout


def ref_convrot(x) -> np.ndarray:
    x = _c(x, np.float32)
    with tempfile.TemporaryDirectory() as d:
        fi, fo = os.path.join(d, "x"), os.path.join(d, "y")
        x.tofile(fi)
        _ref_run(["convrot", x.shape[0], x.shape[1], fi, fo])
        return np.fromfile(fo, np.float32).reshape(x.shape)


def ref_quantize(x, rotate=True):
    x = _c(x, np.float32)
    with tempfile.TemporaryDirectory() as d:
        fi, fq, fs = (os.path.join(d, n) for n in ("x", "q", "s"))
        x.tofile(fi)
        _ref_run(["quant", x.shape[0], x.shape[1], 1 if rotate else 0, fi, fq, fs])
        return (np.fromfile(fq, np.int8).reshape(x.shape), np.fromfile(fs, np.float32))


def ref_gemm(a, sa, b, sb) -> np.ndarray:
    a, b = _c(a, np.int8), _c(b, np.int8)
    sa, sb = _c(sa, np.float32), _c(sb, np.float32)
    M, K = a.shape
    N = b.shape[0]
    with tempfile.TemporaryDirectory() as d:
        names = [os.path.join(d, n) for n in ("a", "sa", "b", "sb", "y")]
        for arr, n in zip((a, sa, b, sb), names):
            arr.tofile(n)
        _ref_run(["gemm", M, N, K] + names)
        return np.fromfile(names[-1], np.float32).reshape(M, N)


def ref_grouped_decode(codes, s_rel_f32, s_channel, *, k, group, codebook=None,
                       correction=None, six=False) -> np.ndarray:
    codes = _c(codes, np.uint8)
    rows = codes.shape[0]
    with tempfile.TemporaryDirectory() as d:
        fc, fr, fs, fcb, fco, fo = (os.path.join(d, n) for n in ("c", "r", "s", "cb", "co", "o"))
        codes.tofile(fc)
        _c(s_rel_f32, np.float32).tofile(fr)
        _c(s_channel, np.float32).tofile(fs)
        if codebook is not None:
            _c(codebook, np.float32).tofile(fcb)
        if correction is not None:
            _c(correction, np.float32).tofile(fco)
        hc = 1 if correction is not None else 0
        if six:
            _ref_run(["w6", rows, k, group, hc, fc, fr, fs, fco, fo])
        else:
            _ref_run(["w4", rows, k, group, 1 if codebook is not None else 0, hc, fc, fr, fs,
                      fcb, fco, fo])
        return np.fromfile(fo, np.float32).reshape(rows, k)


def ref_w4a4pack(w):
    """The reference's own quantize_convrot_w4a4 (group 256) on w [rows, cols]."""
    w = _c(w, np.float32)
    rows, cols = w.shape
    with tempfile.TemporaryDirectory() as d:
        fw, fp, fs = (os.path.join(d, n) for n in ("w", "p", "s"))
        w.tofile(fw)
        _ref_run(["w4a4pack", rows, cols, fw, fp, fs])
        return (np.fromfile(fp, np.uint8).reshape(rows, cols // 2), np.fromfile(fs, np.float32))


def ref_bench_q8(M, N, K, rows) -> float:
    """Seconds the reference CPU path takes for ``rows`` rows of an MxNxK linear."""
    return float(_ref_run(["bench_q8", M, N, K, rows]).split()[0])


def ref_bench_q8_mt(M, N, K, rows, threads) -> float:
    """The same rows spread over ``threads`` threads, one row per task."""
    return float(_ref_run(["bench_q8_mt", M, N, K, rows, threads]).split()[0])
