"""Python front end of the gfx950 quantized-linear library.

Thin ctypes bindings over the C ABI in ``include/phi_qlinear.h``
(``lib/libphi_qlinear.so``).  PyTorch provides device memory and the stream;
every computation runs in the HIP kernels.  There is no fallback: if the
library is missing or the device is absent the calls raise.

Names and argument meaning follow the reference's dispatchers:
``quant_rotate`` is ``dispatch_quant_convrot`` (core/runtime/compute.cpp:663-684),
``i8_gemm`` is ``dispatch_int8_gemm`` (:551-661), ``q8_linear`` is
``linear_gemm``'s int8 branch (core/models/model_common.cpp:1363-1412) and
``w4a8_expand`` is ``dispatch_w4a8_expand`` (core/kernels/w4a8_expand.cpp:263-303).
"""
from __future__ import annotations

import ctypes
import os

import torch

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(os.path.dirname(PKG_DIR), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libphi_qlinear.so")
MEDIA_LIB_PATH = os.path.join(LIB_DIR, "libphi_media.so")
INCLUDE_DIR = os.path.join(os.path.dirname(os.path.dirname(PKG_DIR)), "include")

# phi_dtype
F32, BF16, F16, I32, I8, F8_E4M3, F8_E5M2, U8_E4M3, I4 = range(9)
# phi_round
ROUND_HALF_AWAY, ROUND_HALF_EVEN = 0, 1
ACT_GELU_TANH, ACT_SILU_GATE = 1, 2
# phi_status
STATUS = {0: "PHI_OK", 1: "PHI_ERR_ARG", 2: "PHI_ERR_SHAPE", 3: "PHI_ERR_ALIGN",
          4: "PHI_ERR_WORKSPACE", 5: "PHI_ERR_HIP", 6: "PHI_ERR_DEVICE_LOST",
          7: "PHI_ERR_UNSUPPORTED"}


class QLinearError(RuntimeError):
    """A failing library call: ``status`` is the phi_status, the message is the
    library's own (the reference raises MediaError with the same text)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


class W4a8Weight(ctypes.Structure):
    _fields_ = [("codes", ctypes.c_void_p), ("codes_row_bytes", ctypes.c_int64),
                ("s_rel", ctypes.c_void_p), ("s_rel_dtype", ctypes.c_int),
                ("srel_row_bytes", ctypes.c_int64), ("s_channel", ctypes.c_void_p),
                ("sch_scalar", ctypes.c_int), ("codebook", ctypes.c_void_p),
                ("correction", ctypes.c_void_p), ("rows", ctypes.c_int64),
                ("k", ctypes.c_int64), ("group", ctypes.c_int64), ("layout", ctypes.c_int)]


PLAN_TILE_AUTO, PLAN_TILE_SQUARE, PLAN_TILE_272 = 0, 1, 2


class GemmPlan(ctypes.Structure):
    """phi_gemm_plan: big_rows (-1: the cost model), group_m (0: 4), split,
    tile (PLAN_TILE_AUTO / _SQUARE / _272), reserved (0)."""
    _fields_ = [("big_rows", ctypes.c_int64), ("group_m", ctypes.c_int32), ("split", ctypes.c_int32),
                ("tile", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class GemvItem(ctypes.Structure):
    _fields_ = [("W", ctypes.c_void_p), ("sW", ctypes.c_void_p), ("sw_scalar", ctypes.c_int),
                ("bias", ctypes.c_void_p), ("C", ctypes.c_void_p), ("ldc", ctypes.c_int64)]


EXPORTS = ["phi_hip_last_error", "phi_hip_abi_version", "phi_hip_quant_rotate", "phi_hip_i8_gemm",
           "phi_hip_workspace_bytes", "phi_hip_q8_linear", "phi_hip_w4a8_expand",
           "phi_hip_w4a8_prepare", "phi_hip_w4a8_linear", "phi_hip_i8_gemv_batched",
           "phi_hip_gemv_workspace_bytes", "phi_hip_gelu_tanh", "phi_hip_w4a8_workspace_bytes",
           "phi_hip_quant_rotate_mod", "phi_hip_i8_gemm_residual", "phi_hip_quant_rotate_act",
           "phi_hip_silu_gate", "phi_hip_i4_gemm", "phi_hip_i4_workspace_bytes", "phi_hip_lora_tail",
           "phi_hip_lora_down", "phi_hip_lora_rank_add", "phi_hip_dequant_rows", "phi_hip_convrot_rows",
           "phi_hip_lora_fold", "phi_hip_q8_linear_noalloc", "phi_hip_noalloc_scratch_bytes",
           "phi_hip_pack_k_tiled", "phi_hip_i8_gemm_kt", "phi_hip_q8_linear_kt", "phi_hip_q8_linear_kq",
           "phi_hip_quant_rotate_kt", "phi_hip_big_tile_rows",
           "phi_hip_quant_rotate_mod_kt", "phi_hip_quant_rotate_act_kt", "phi_hip_i8_gemm_residual_kt",
           "phi_hip_dequant_fp4_rows", "phi_hip_gemm_plan_set", "phi_hip_gemm_plan_get", "phi_hip_gemm_plan_count",
           "phi_hip_gemm_plan_clear", "phi_hip_w4a8_banded_bytes", "phi_hip_w4a8_pack_banded",
           "phi_hip_w4a8_linear_banded"]

_lib = None


def load() -> ctypes.CDLL:
    """Load lib/libphi_qlinear.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C phi-agent_amd)")
    L = ctypes.CDLL(LIB_PATH)
    P, I64, I, F, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    L.phi_hip_last_error.restype = ctypes.c_char_p
    L.phi_hip_abi_version.restype = I
    L.phi_hip_quant_rotate.argtypes = [P, P, I, I64, I64, I64, P, I64, P, F, I, I]
    L.phi_hip_i8_gemm.argtypes = [P, P, I64, P, I64, P, P, I, P, I, P, I, I64, I64, I64, I64, P, SZ]
    L.phi_hip_workspace_bytes.argtypes = [I64, I64, I64]
    L.phi_hip_workspace_bytes.restype = SZ
    L.phi_hip_q8_linear.argtypes = [P, P, I, I64, I64, I64, P, I64, P, I, P, I, I64, P, I, I64, P, P,
                                    I, P, SZ]
    L.phi_hip_w4a8_expand.argtypes = [P, ctypes.POINTER(W4a8Weight), P, P]
    L.phi_hip_w4a8_prepare.argtypes = [P, ctypes.POINTER(W4a8Weight), P, P]
    L.phi_hip_w4a8_linear.argtypes = [P, P, I, I64, I64, I64, P, I64, P, I64, P, P, I, I64, P, I,
                                      I64, P, P, I, P, SZ]
    L.phi_hip_i8_gemv_batched.argtypes = [P, P, P, I64, I64, I64, ctypes.POINTER(GemvItem), I, I,
                                          I, P, SZ]
    L.phi_hip_quant_rotate_mod.argtypes = [P, P, I, I64, I64, I64, P, P, P, I64, P, ctypes.c_float, I, I]
    L.phi_hip_i8_gemm_residual.argtypes = [P, P, I64, P, I64, P, P, I, P, I, P, P, I64, I64, I64, I64, P, SZ]
    L.phi_hip_w4a8_workspace_bytes.argtypes = [I64, I64, I64, I64]
    L.phi_hip_w4a8_workspace_bytes.restype = SZ
    L.phi_hip_gemv_workspace_bytes.argtypes = [I]
    L.phi_hip_gemv_workspace_bytes.restype = SZ
    L.phi_hip_gelu_tanh.argtypes = [P, P, I, P, I, I64]
    L.phi_hip_quant_rotate_act.argtypes = [P, P, I, I64, I64, I64, I, P, I64, P, F, I, I]
    L.phi_hip_silu_gate.argtypes = [P, P, I, I64, I64, I64, P, I, I64]
    L.phi_hip_i4_gemm.argtypes = [P, P, I64, P, I64, P, P, P, I, I64, I64, I64, I64, P, SZ]
    L.phi_hip_i4_workspace_bytes.argtypes = [I64, I64, I64]
    L.phi_hip_lora_tail.argtypes = [P, P, I, I64, I64, I64, P, P, I64, I64, P, I, I64, P, SZ]
    L.phi_hip_lora_down.argtypes = [P, P, I, I64, I64, I64, P, I64, P]
    L.phi_hip_lora_rank_add.argtypes = [P, P, P, P, I, I64, I64, I64, I64]
    L.phi_hip_i4_workspace_bytes.restype = SZ
    L.phi_hip_dequant_rows.argtypes = [P, P, I, I64, I64, I64, P, I, P, I64]
    L.phi_hip_convrot_rows.argtypes = [P, P, I64, I64, I64, P, I64]
    L.phi_hip_dequant_fp4_rows.argtypes = [P, P, I64, I64, I64, I64, P, I64, I64, I64, P, I, P, I64]
    L.phi_hip_gemm_plan_set.argtypes = [I64, I64, I64, I, ctypes.POINTER(GemmPlan)]
    L.phi_hip_gemm_plan_get.argtypes = [I64, I64, I64, I, ctypes.POINTER(GemmPlan), ctypes.POINTER(ctypes.c_int)]
    L.phi_hip_gemm_plan_count.restype = I64
    L.phi_hip_gemm_plan_clear.restype = None
    L.phi_hip_lora_fold.argtypes = [P, P, I64, I64, I64, P, P, I64, F]
    L.phi_hip_q8_linear_noalloc.argtypes = [P, P, I, I64, I64, I64, P, I64, P, I, P, I, I64, P, I, I64, I]
    L.phi_hip_noalloc_scratch_bytes.argtypes = []
    L.phi_hip_noalloc_scratch_bytes.restype = SZ
    L.phi_hip_pack_k_tiled.argtypes = [P, P, I64, I64, I64, P]
    L.phi_hip_quant_rotate_kt.argtypes = [P, P, I, I64, I64, I64, P, P, F, I]
    L.phi_hip_quant_rotate_mod_kt.argtypes = [P, P, I, I64, I64, I64, P, P, P, P, F, I]
    L.phi_hip_quant_rotate_act_kt.argtypes = [P, P, I, I64, I64, I64, I, P, P, F, I]
    L.phi_hip_i8_gemm_residual_kt.argtypes = [P, P, P, P, P, I, P, I, P, P, I64, I64, I64, I64]
    L.phi_hip_big_tile_rows.argtypes = [I64, I64]
    L.phi_hip_big_tile_rows.restype = I64
    L.phi_hip_i8_gemm_kt.argtypes = [P, P, P, P, P, I, P, I, P, I, I64, I64, I64, I64]
    L.phi_hip_q8_linear_kt.argtypes = [P, P, I, I64, I64, I64, P, P, I, P, I, I64, P, I, I64, P, P, I]
    L.phi_hip_q8_linear_kq.argtypes = [P, P, I, I64, I64, I64, P, I64, P, I, P, I, I64, P, I, I64, P, P,
                                       I, P, SZ]
    L.phi_hip_w4a8_banded_bytes.argtypes = [I64, I64, I64]
    L.phi_hip_w4a8_banded_bytes.restype = SZ
    L.phi_hip_w4a8_pack_banded.argtypes = [P, P, I64, P, I64, I64, I64, P]
    L.phi_hip_w4a8_linear_banded.argtypes = [P, P, I, I64, I64, I64, P, I64, P, P, I, I64, P, I, I64, P, P, I]
    for name in EXPORTS:
        f = getattr(L, name)
        if f.restype is None:
            f.restype = I
    _lib = L
    return L


def last_error() -> str:
    return load().phi_hip_last_error().decode()


def _check(status: int) -> None:
    if status != 0:
        raise QLinearError(status, last_error())


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _dt(t: torch.Tensor) -> int:
    return {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int32: I32,
            torch.int8: I8}[t.dtype]


def _require_device(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("phi_qlinear operates on device tensors")


# ---------------------------------------------------------------- A1-A3
def quant_rotate(x: torch.Tensor, *, qmax: float = 127.0, round_mode: int = ROUND_HALF_AWAY,
                 rotate: bool = True, q: torch.Tensor | None = None,
                 s: torch.Tensor | None = None, mod_scale: torch.Tensor | None = None,
                 mod_shift: torch.Tensor | None = None, act: str | None = None, stream=None):
    """Rotate (256-wide convrot) and quantise rows of x [rows, K] (f32/bf16).

    mod_scale / mod_shift ([K] fp32): the adaLN modulation fma(x, 1 + scale,
    shift) applied first (phi_hip_quant_rotate_mod).
    act: "gelu_tanh" applies GELU-tanh first; "silu_gate" takes x [rows, 2K]
    and quantises silu(x[:, :K]) * x[:, K:] (phi_hip_quant_rotate_act).
    Returns (q int8 [rows, K], s f32 [rows])."""
    _require_device(x, mod_scale, mod_shift)
    rows, K = x.shape
    if act is not None:
        if mod_scale is not None or mod_shift is not None:
            raise ValueError("quant_rotate: act and modulation are exclusive")
        code = {"gelu_tanh": ACT_GELU_TANH, "silu_gate": ACT_SILU_GATE}[act]
        if act == "silu_gate":
            if K % 2:
                raise ValueError("quant_rotate: silu_gate needs an even number of columns")
            K //= 2
        if q is None:
            q = torch.empty((rows, K), dtype=torch.int8, device=x.device)
        if s is None:
            s = torch.empty((rows,), dtype=torch.float32, device=x.device)
        _check(load().phi_hip_quant_rotate_act(_stream(stream), _ptr(x), _dt(x), rows, K, x.stride(0), code,
                                               _ptr(q), q.stride(0), _ptr(s), float(qmax), round_mode,
                                               1 if rotate else 0))
        return q, s
    if q is None:
        q = torch.empty((rows, K), dtype=torch.int8, device=x.device)
    if s is None:
        s = torch.empty((rows,), dtype=torch.float32, device=x.device)
    if mod_scale is None and mod_shift is None:
        _check(load().phi_hip_quant_rotate(_stream(stream), _ptr(x), _dt(x), rows, K, x.stride(0),
                                           _ptr(q), q.stride(0), _ptr(s), float(qmax), round_mode,
                                           1 if rotate else 0))
    else:
        _check(load().phi_hip_quant_rotate_mod(_stream(stream), _ptr(x), _dt(x), rows, K,
                                               x.stride(0), _ptr(mod_scale), _ptr(mod_shift),
                                               _ptr(q), q.stride(0), _ptr(s), float(qmax),
                                               round_mode, 1 if rotate else 0))
    return q, s


# ---------------------------------------------------------------- A4-A6
def _ws(workspace):
    if workspace is None:
        return None, 0
    _require_device(workspace)
    return _ptr(workspace), workspace.numel() * workspace.element_size()


def i8_gemm(A: torch.Tensor, B: torch.Tensor, sA: torch.Tensor | None, sB: torch.Tensor | None,
            bias: torch.Tensor | None = None, *, out_dtype=torch.bfloat16,
            C: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
            stream=None) -> torch.Tensor:
    """C = fma((float)(A . B^T) * sA, sB, bias) in out_dtype (int32: raw acc)."""
    _require_device(A, B, sA, sB, bias, C)
    M, K = A.shape
    N = B.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=A.device)
    sb_scalar = 1 if (sB is not None and sB.numel() == 1) else 0
    wp, wn = _ws(workspace)
    _check(load().phi_hip_i8_gemm(_stream(stream), _ptr(A), A.stride(0), _ptr(B), B.stride(0),
                                  _ptr(sA), _ptr(sB), sb_scalar, _ptr(bias),
                                  _dt(bias) if bias is not None else F32, _ptr(C), _dt(C),
                                  C.stride(0), M, N, K, wp, wn))
    return C


def i8_gemm_residual(A: torch.Tensor, B: torch.Tensor, sA: torch.Tensor, sB: torch.Tensor,
                     bias: torch.Tensor | None, gate: torch.Tensor, H: torch.Tensor,
                     stream=None) -> torch.Tensor:
    """H = fma(fma((float)(A . B^T) * sA, sB, bias), gate, H) in place (fp32 H)."""
    _require_device(A, B, sA, sB, bias, gate, H)
    M, K = A.shape
    N = B.shape[0]
    sb_scalar = 1 if sB.numel() == 1 else 0
    _check(load().phi_hip_i8_gemm_residual(_stream(stream), _ptr(A), A.stride(0), _ptr(B),
                                           B.stride(0), _ptr(sA), _ptr(sB), sb_scalar, _ptr(bias),
                                           _dt(bias) if bias is not None else F32, _ptr(gate),
                                           _ptr(H), H.stride(0), M, N, K, None, 0))
    return H


def q8_linear(x: torch.Tensor, W: torch.Tensor, sW: torch.Tensor,
              bias: torch.Tensor | None = None, *, out_dtype=torch.bfloat16,
              q8: torch.Tensor | None = None, s8: torch.Tensor | None = None,
              C: torch.Tensor | None = None, round_mode: int = ROUND_HALF_AWAY,
              workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """The W8A8 linear: rotate+quantise x into q8/s8, int8 GEMM, epilogue."""
    _require_device(x, W, sW, bias, q8, s8, C)
    M, K = x.shape
    N = W.shape[0]
    if q8 is None:
        q8 = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if s8 is None:
        s8 = torch.empty((M,), dtype=torch.float32, device=x.device)
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=x.device)
    wp, wn = _ws(workspace)
    _check(load().phi_hip_q8_linear(_stream(stream), _ptr(x), _dt(x), x.stride(0), M, K, _ptr(W),
                                    W.stride(0), _ptr(sW), 1 if sW.numel() == 1 else 0,
                                    _ptr(bias), _dt(bias) if bias is not None else F32, N,
                                    _ptr(C), _dt(C), C.stride(0), _ptr(q8), _ptr(s8), round_mode,
                                    wp, wn))
    return C


def q8_linear_kq(x: torch.Tensor, W: torch.Tensor, sW: torch.Tensor,
                 bias: torch.Tensor | None = None, *, out_dtype=torch.bfloat16,
                 q8: torch.Tensor | None = None, s8: torch.Tensor | None = None,
                 C: torch.Tensor | None = None, round_mode: int = ROUND_HALF_AWAY,
                 workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """q8_linear on a row-major weight with the activation scratch q8 written
    K-tiled where the 272 x 192 plan takes the problem (phi_hip_q8_linear_kq):
    C and s8 are q8_linear's, bit for bit; q8 is scratch."""
    _require_device(x, W, sW, bias, q8, s8, C)
    M, K = x.shape
    N = W.shape[0]
    if q8 is None:
        q8 = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if s8 is None:
        s8 = torch.empty((M,), dtype=torch.float32, device=x.device)
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=x.device)
    wp, wn = _ws(workspace)
    _check(load().phi_hip_q8_linear_kq(_stream(stream), _ptr(x), _dt(x), x.stride(0), M, K, _ptr(W),
                                       W.stride(0), _ptr(sW), 1 if sW.numel() == 1 else 0,
                                       _ptr(bias), _dt(bias) if bias is not None else F32, N,
                                       _ptr(C), _dt(C), C.stride(0), _ptr(q8), _ptr(s8), round_mode,
                                       wp, wn))
    return C


def q8_linear_noalloc(x: torch.Tensor, W: torch.Tensor, sW: torch.Tensor,
                      bias: torch.Tensor | None = None, *, out_dtype=torch.bfloat16,
                      C: torch.Tensor | None = None, round_mode: int = ROUND_HALF_AWAY,
                      stream=None) -> torch.Tensor:
    """q8_linear with the activation scratch in the library's static device
    array (phi_hip_q8_linear_noalloc): no caller scratch, nothing allocated
    by the library.  Calls that overlap on one GPU race on that array."""
    _require_device(x, W, sW, bias, C)
    M, K = x.shape
    N = W.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=x.device)
    _check(load().phi_hip_q8_linear_noalloc(_stream(stream), _ptr(x), _dt(x), x.stride(0), M, K, _ptr(W),
                                            W.stride(0), _ptr(sW), 1 if sW.numel() == 1 else 0, _ptr(bias),
                                            _dt(bias) if bias is not None else F32, N, _ptr(C), _dt(C),
                                            C.stride(0), round_mode))
    return C


# ---------------------------------------------------------------- A7
def _w4a8_desc(codes, s_rel, s_rel_dtype, s_channel, codebook, correction, k, group, layout):
    _require_device(codes, s_rel, s_channel, codebook, correction)
    w = W4a8Weight()
    w.codes = codes.data_ptr()
    w.codes_row_bytes = codes.stride(0)
    w.s_rel = s_rel.data_ptr() if s_rel is not None else None
    w.s_rel_dtype = s_rel_dtype
    w.srel_row_bytes = (s_rel.stride(0) * s_rel.element_size()) if s_rel is not None else 0
    w.s_channel = s_channel.data_ptr() if s_channel is not None else None
    w.sch_scalar = 1 if (s_channel is not None and s_channel.numel() == 1) else 0
    w.codebook = codebook.data_ptr() if codebook is not None else None
    w.correction = correction.data_ptr() if correction is not None else None
    w.rows = codes.shape[0]
    w.k = k
    w.group = group
    w.layout = layout
    return w


def w4a8_expand(codes, s_rel, s_rel_dtype, s_channel=None, *, k, group, codebook=None,
                correction=None, layout=0, stream=None):
    """Decode a grouped 4-bit / 6-bit weight to (q int8 [N, k], s f32 [N])."""
    w = _w4a8_desc(codes, s_rel, s_rel_dtype, s_channel, codebook, correction, k, group, layout)
    q = torch.empty((w.rows, k), dtype=torch.int8, device=codes.device)
    s = torch.empty((w.rows,), dtype=torch.float32, device=codes.device)
    _check(load().phi_hip_w4a8_expand(_stream(stream), ctypes.byref(w), _ptr(q), _ptr(s)))
    return q, s


def w4a8_prepare(codes, s_rel, s_rel_dtype, s_channel=None, *, k, group, codebook=None,
                 correction=None, stream=None):
    """Per-(row, group) 16-entry int8 tables + row scales for the in-register GEMM."""
    w = _w4a8_desc(codes, s_rel, s_rel_dtype, s_channel, codebook, correction, k, group, 0)
    lut = torch.empty((w.rows, k // group, 16), dtype=torch.int8, device=codes.device)
    s = torch.empty((w.rows,), dtype=torch.float32, device=codes.device)
    _check(load().phi_hip_w4a8_prepare(_stream(stream), ctypes.byref(w), _ptr(lut), _ptr(s)))
    return lut, s


def w4a8_linear(x, codes, lut, s_w, *, group, bias=None, out_dtype=torch.bfloat16, q8=None,
                s8=None, C=None, round_mode=ROUND_HALF_AWAY, workspace=None, stream=None):
    """W4A8 linear; workspace (phi_hip_w4a8_workspace_bytes bytes) lets a call
    with many rows expand the codes once instead of per tile."""
    _require_device(x, codes, lut, s_w, bias, q8, s8, C)
    M, K = x.shape
    N = codes.shape[0]
    if q8 is None:
        q8 = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if s8 is None:
        s8 = torch.empty((M,), dtype=torch.float32, device=x.device)
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=x.device)
    _check(load().phi_hip_w4a8_linear(_stream(stream), _ptr(x), _dt(x), x.stride(0), M, K,
                                      _ptr(codes), codes.stride(0), _ptr(lut), group, _ptr(s_w),
                                      _ptr(bias), _dt(bias) if bias is not None else F32, N,
                                      _ptr(C), _dt(C), C.stride(0), _ptr(q8), _ptr(s8),
                                      round_mode, *_ws(workspace)))
    return C


def w4a8_pack_banded(codes: torch.Tensor, lut: torch.Tensor, *, k: int, group: int,
                     stream=None) -> torch.Tensor:
    """The W4A8 weight (codes [N, >= k/2] nibbles, lut from w4a8_prepare)
    packed in bands of 192 rows for the in-LDS expansion
    (phi_hip_w4a8_pack_banded): a uint8 buffer of phi_hip_w4a8_banded_bytes."""
    _require_device(codes, lut)
    N = codes.shape[0]
    n = load().phi_hip_w4a8_banded_bytes(N, k, group)
    if not n:
        raise ValueError(f"no band layout for a {N} x {k} weight with group {group}")
    out = torch.empty(n, dtype=torch.uint8, device=codes.device)
    _check(load().phi_hip_w4a8_pack_banded(_stream(stream), _ptr(codes), codes.stride(0), _ptr(lut), N, k, group,
                                           _ptr(out)))
    return out


def w4a8_linear_banded(x, banded, s_w, *, N: int, group: int, bias=None, out_dtype=torch.bfloat16, q8=None,
                       s8=None, C=None, round_mode=ROUND_HALF_AWAY, stream=None):
    """w4a8_linear on a band-packed weight (phi_hip_w4a8_linear_banded): the
    codes expanded in LDS, no workspace; q8 (M * K bytes) is written K-tiled."""
    _require_device(x, banded, s_w, bias, q8, s8, C)
    M, K = x.shape
    if q8 is None:
        q8 = torch.empty((M * K,), dtype=torch.int8, device=x.device)
    if s8 is None:
        s8 = torch.empty((M,), dtype=torch.float32, device=x.device)
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=x.device)
    _check(load().phi_hip_w4a8_linear_banded(_stream(stream), _ptr(x), _dt(x), x.stride(0), M, K, _ptr(banded),
                                             group, _ptr(s_w), _ptr(bias), _dt(bias) if bias is not None else F32,
                                             N, _ptr(C), _dt(C), C.stride(0), _ptr(q8), _ptr(s8), round_mode))
    return C


def w4a8_workspace(M: int, N: int, K: int, group: int, device) -> torch.Tensor | None:
    """A buffer of phi_hip_w4a8_workspace_bytes bytes (None when 0)."""
    n = load().phi_hip_w4a8_workspace_bytes(M, N, K, group)
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


# ---------------------------------------------------------------- GEMV
def gemv_batched(q8: torch.Tensor, s8: torch.Tensor, weights, scales, *, biases=None,
                 outs=None, out_dtype=torch.bfloat16, stream=None):
    """C_i = epilogue(q8 . W_i^T) for every weight (M = q8.shape[0] <= 8)."""
    _require_device(q8, s8)
    M, K = q8.shape
    N = weights[0].shape[0]
    n = len(weights)
    if outs is None:
        outs = [torch.empty((M, N), dtype=out_dtype, device=q8.device) for _ in range(n)]
    items = (GemvItem * n)()
    bias_dt = F32
    for i in range(n):
        items[i].W = weights[i].data_ptr()
        items[i].sW = scales[i].data_ptr() if scales is not None else None
        items[i].sw_scalar = 1 if (scales is not None and scales[i].numel() == 1) else 0
        b = biases[i] if biases is not None else None
        if b is not None:
            bias_dt = _dt(b)
        items[i].bias = b.data_ptr() if b is not None else None
        items[i].C = outs[i].data_ptr()
        items[i].ldc = outs[i].stride(0)
    _check(load().phi_hip_i8_gemv_batched(_stream(stream), _ptr(q8), _ptr(s8), M, K, N, items, n,
                                          bias_dt, _dt(outs[0]), None, 0))
    return outs


def gelu_tanh(x: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """GELU-tanh of a contiguous x into out (x's shape; f32 or bf16)."""
    _require_device(x, out)
    if out is None:
        out = torch.empty_like(x)
    if not x.is_contiguous() or not out.is_contiguous() or out.numel() != x.numel():
        raise ValueError("gelu_tanh: x and out must be contiguous and equally sized")
    _check(load().phi_hip_gelu_tanh(_stream(stream), _ptr(x), _dt(x), _ptr(out), _dt(out),
                                    x.numel()))
    return out


def silu_gate(gx: torch.Tensor, out: torch.Tensor | None = None, *, out_dtype=None,
              stream=None) -> torch.Tensor:
    """out [rows, cols] = silu(gx[:, :cols]) * gx[:, cols:] for gx [rows, 2*cols]
    (phi_hip_silu_gate; dispatch_silu_gate_fused core/kernels/h3_kernels.hpp:116-129)."""
    _require_device(gx, out)
    rows, two = gx.shape
    if two % 2:
        raise ValueError("silu_gate: gx needs an even number of columns")
    cols = two // 2
    if out is None:
        out = torch.empty((rows, cols), dtype=out_dtype or gx.dtype, device=gx.device)
    _check(load().phi_hip_silu_gate(_stream(stream), _ptr(gx), _dt(gx), rows, cols, gx.stride(0), _ptr(out),
                                    _dt(out), out.stride(0)))
    return out


def i4_workspace(M: int, N: int, K: int, device) -> torch.Tensor | None:
    """The optional expand-once buffer of i4_gemm (None when the shape takes none)."""
    n = load().phi_hip_i4_workspace_bytes(M, N, K)
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


def i4_gemm(A: torch.Tensor, B: torch.Tensor, sA: torch.Tensor | None, sB: torch.Tensor | None, *,
            out_dtype=torch.float32, C: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
            stream=None) -> torch.Tensor:
    """convrot_w4a4 GEMM: C = ((float)(A . w^T) * sA) * sB, B uint8 [N, K/2] of signed
    nibbles (low nibble = even column); int32 out_dtype gives the accumulators."""
    _require_device(A, B, sA, sB, C)
    M, K = A.shape
    N = B.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=A.device)
    ws, wsb = _ws(workspace)
    _check(load().phi_hip_i4_gemm(_stream(stream), _ptr(A), A.stride(0), _ptr(B), B.stride(0), _ptr(sA),
                                  _ptr(sB), _ptr(C), _dt(C), C.stride(0), M, N, K, ws, wsb))
    return C


def lora_down(x: torch.Tensor, A: torch.Tensor, h: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """h [M, R] = x [M, K] . A [R, K]^T in fp32, k-ordered fma chains (phi_hip_lora_down)."""
    _require_device(x, A, h)
    M, K = x.shape
    R = A.shape[0]
    if h is None:
        h = torch.empty((M, R), dtype=torch.float32, device=x.device)
    _check(load().phi_hip_lora_down(_stream(stream), _ptr(x), _dt(x), x.stride(0), M, K, _ptr(A), R, _ptr(h)))
    return h


def lora_rank_add(h: torch.Tensor, B: torch.Tensor, C: torch.Tensor, stream=None) -> torch.Tensor:
    """C [M, N] += h [M, R] . B [N, R]^T in place, r-ordered fma chains from C (phi_hip_lora_rank_add)."""
    _require_device(h, B, C)
    M, N = C.shape
    R = h.shape[1]
    _check(load().phi_hip_lora_rank_add(_stream(stream), _ptr(h), _ptr(B), _ptr(C), _dt(C), C.stride(0), M, N, R))
    return C


def lora_tail(x: torch.Tensor, At: torch.Tensor, Bt: torch.Tensor, out: torch.Tensor,
              h: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """out += (x . At^T) . Bt^T in place (phi_hip_lora_tail; apply_lora_tail
    core/models/model_common.cpp:1667-1700); h is the [M, R] fp32 scratch."""
    _require_device(x, At, Bt, out, h)
    M, K = x.shape
    R = At.shape[0]
    N = out.shape[1]
    if h is None:
        h = torch.empty((M, R), dtype=torch.float32, device=x.device)
    _check(load().phi_hip_lora_tail(_stream(stream), _ptr(x), _dt(x), x.stride(0), M, K, _ptr(At), _ptr(Bt), R, N,
                                    _ptr(out), _dt(out), out.stride(0), _ptr(h), h.numel() * h.element_size()))
    return out


def dequant_rows(src: torch.Tensor, dtype: int, cols: int, row_scale: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """phi_hip_dequant_rows: a stored tensor's rows in fp32.  src holds the raw
    elements [rows, lds] (uint8 for I4 and the fp8 codes); dtype one of I8, I4,
    F8_E4M3, F8_E5M2, F16, BF16, F32; row_scale [rows] or [1]."""
    _require_device(src, row_scale, out)
    rows = src.shape[0]
    if out is None:
        out = torch.empty((rows, cols), dtype=torch.float32, device=src.device)
    _check(load().phi_hip_dequant_rows(_stream(stream), _ptr(src), dtype, rows, cols, src.stride(0), _ptr(row_scale),
                                       1 if row_scale is not None and row_scale.numel() == 1 else 0, _ptr(out),
                                       out.stride(0)))
    return out


def dequant_fp4_rows(codes: torch.Tensor, k: int, block_scale: torch.Tensor | None = None, *, block: int = 16,
                     global_scale: torch.Tensor | None = None, row0: int = 0, out: torch.Tensor | None = None,
                     stream=None) -> torch.Tensor:
    """phi_hip_dequant_fp4_rows: nvfp4 / mxfp4 weight rows row0 .. row0 +
    rows - 1 in fp32.  codes uint8 [rows, >= k/2]; block_scale the 2-D tiled
    table already in fp32; global_scale [rows] or [1]."""
    _require_device(codes, block_scale, global_scale, out)
    rows = codes.shape[0]
    if out is None:
        out = torch.empty((rows, k), dtype=torch.float32, device=codes.device)
    tr, tc = (block_scale.shape if block_scale is not None else (0, 0))
    _check(load().phi_hip_dequant_fp4_rows(_stream(stream), _ptr(codes), codes.stride(0), row0, rows, k,
                                           _ptr(block_scale), tr, tc, block, _ptr(global_scale),
                                           1 if global_scale is not None and global_scale.numel() == 1 else 0,
                                           _ptr(out), out.stride(0)))
    return out


def gemm_plan_set(M: int, N: int, K: int, *, k_tiled: bool = False, big_rows: int = -1, group_m: int = 0,
                  split: bool = False, tile: int = PLAN_TILE_AUTO, remove: bool = False) -> None:
    """phi_hip_gemm_plan_set: the tuning table's plan for one GEMM shape
    (remove=True drops the entry)."""
    plan = None if remove else ctypes.byref(GemmPlan(big_rows, group_m, 1 if split else 0, tile, 0))
    _check(load().phi_hip_gemm_plan_set(M, N, K, 1 if k_tiled else 0, plan))


def gemm_plan_get(M: int, N: int, K: int, *, k_tiled: bool = False) -> dict:
    """The plan a GEMM of this shape runs: {big_rows, group_m, split, tile,
    tuned}, the tile shape resolved (PLAN_TILE_SQUARE or PLAN_TILE_272)."""
    plan, tuned = GemmPlan(), ctypes.c_int(0)
    _check(load().phi_hip_gemm_plan_get(M, N, K, 1 if k_tiled else 0, ctypes.byref(plan), ctypes.byref(tuned)))
    return {"big_rows": plan.big_rows, "group_m": plan.group_m, "split": bool(plan.split), "tile": plan.tile,
            "tuned": bool(tuned.value)}


def gemm_plan_clear() -> None:
    load().phi_hip_gemm_plan_clear()


def gemm_plan_count() -> int:
    return int(load().phi_hip_gemm_plan_count())


def pack_k_tiled(W: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """An int8 [rows, K] matrix (row pitch a multiple of 16) in the K-tiled
    operand layout of the persistent GEMM (phi_hip_pack_k_tiled): a flat
    int8 tensor of rows * K bytes."""
    _require_device(W, out)
    rows, K = W.shape
    if out is None:
        out = torch.empty((rows * K,), dtype=torch.int8, device=W.device)
    if out.numel() < rows * K:
        raise ValueError(f"pack_k_tiled: out holds {out.numel()} bytes, needs {rows * K}")
    _check(load().phi_hip_pack_k_tiled(_stream(stream), _ptr(W), W.stride(0), rows, K, _ptr(out)))
    return out


def big_tile_rows(M: int, N: int) -> int:
    """Rows of an M x N GEMM the persistent plan runs as 256 x 256 tiles on
    the current device (phi_hip_big_tile_rows)."""
    return int(load().phi_hip_big_tile_rows(M, N))


def quant_rotate_kt(x: torch.Tensor, q: torch.Tensor | None = None, s: torch.Tensor | None = None,
                    qmax: float = 127.0, round_mode: int = ROUND_HALF_AWAY, *, mod_scale=None, mod_shift=None,
                    act: str | None = None, stream=None):
    """quant_rotate with q (rows * K bytes) written K-tiled
    (phi_hip_quant_rotate_kt / _mod_kt / _act_kt).  For act="silu_gate" x is
    [rows, 2K] (gate then value halves)."""
    _require_device(x, q, s, mod_scale, mod_shift)
    rows = x.shape[0]
    K = x.shape[1] // 2 if act == "silu_gate" else x.shape[1]
    if q is None:
        q = torch.empty((rows * K,), dtype=torch.int8, device=x.device)
    if s is None:
        s = torch.empty((rows,), dtype=torch.float32, device=x.device)
    if q.numel() < rows * K:
        raise ValueError(f"quant_rotate_kt: q holds {q.numel()} bytes, needs {rows * K}")
    L = load()
    if act is not None:
        code = {"gelu_tanh": ACT_GELU_TANH, "silu_gate": ACT_SILU_GATE}[act]
        _check(L.phi_hip_quant_rotate_act_kt(_stream(stream), _ptr(x), _dt(x), rows, K, x.stride(0), code,
                                             _ptr(q), _ptr(s), qmax, round_mode))
    elif mod_scale is not None or mod_shift is not None:
        _check(L.phi_hip_quant_rotate_mod_kt(_stream(stream), _ptr(x), _dt(x), rows, K, x.stride(0),
                                             _ptr(mod_scale), _ptr(mod_shift), _ptr(q), _ptr(s), qmax, round_mode))
    else:
        _check(L.phi_hip_quant_rotate_kt(_stream(stream), _ptr(x), _dt(x), rows, K, x.stride(0), _ptr(q),
                                         _ptr(s), qmax, round_mode))
    return q, s


def i8_gemm_residual_kt(A: torch.Tensor, B: torch.Tensor, M: int, N: int, K: int, sA: torch.Tensor,
                        sB: torch.Tensor, bias: torch.Tensor | None, gate: torch.Tensor, H: torch.Tensor,
                        stream=None) -> torch.Tensor:
    """phi_hip_i8_gemm_residual_kt: H = fma(linear, gate, H) in place, A and B K-tiled."""
    _require_device(A, B, sA, sB, bias, gate, H)
    for name, t, rows in (("A", A, M), ("B", B, N)):
        if t.numel() < rows * K:
            raise ValueError(f"i8_gemm_residual_kt: {name} holds {t.numel()} bytes, needs {rows * K}")
    _check(load().phi_hip_i8_gemm_residual_kt(_stream(stream), _ptr(A), _ptr(B), _ptr(sA), _ptr(sB),
                                              1 if sB.numel() == 1 else 0, _ptr(bias),
                                              _dt(bias) if bias is not None else F32, _ptr(gate), _ptr(H),
                                              H.stride(0), M, N, K))
    return H


def i8_gemm_kt(A: torch.Tensor, B: torch.Tensor, M: int, N: int, K: int, sA: torch.Tensor | None,
               sB: torch.Tensor | None, bias: torch.Tensor | None = None, *, out_dtype=torch.bfloat16,
               C: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """phi_hip_i8_gemm_kt: A [M, K] and B [N, K] given K-tiled (pack_k_tiled)."""
    _require_device(A, B, sA, sB, bias, C)
    for name, t, rows in (("A", A, M), ("B", B, N)):
        if t.numel() < rows * K:
            raise ValueError(f"i8_gemm_kt: {name} holds {t.numel()} bytes, needs {rows * K}")
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=A.device)
    _check(load().phi_hip_i8_gemm_kt(_stream(stream), _ptr(A), _ptr(B), _ptr(sA), _ptr(sB),
                                     1 if sB is not None and sB.numel() == 1 else 0, _ptr(bias),
                                     _dt(bias) if bias is not None else F32, _ptr(C), _dt(C), C.stride(0),
                                     M, N, K))
    return C


def q8_linear_kt(x: torch.Tensor, Wkt: torch.Tensor, N: int, sW: torch.Tensor,
                 bias: torch.Tensor | None = None, *, out_dtype=torch.bfloat16,
                 q8: torch.Tensor | None = None, s8: torch.Tensor | None = None,
                 C: torch.Tensor | None = None, round_mode: int = ROUND_HALF_AWAY,
                 stream=None) -> torch.Tensor:
    """q8_linear with the weight packed K-tiled (pack_k_tiled, N rows): q8
    (M * K bytes) is written K-tiled; C is bit-identical to q8_linear's."""
    _require_device(x, Wkt, sW, bias, q8, s8, C)
    M, K = x.shape
    if Wkt.numel() < N * K:
        raise ValueError(f"q8_linear_kt: the packed weight holds {Wkt.numel()} bytes, needs {N * K}")
    if q8 is None:
        q8 = torch.empty((M * K,), dtype=torch.int8, device=x.device)
    if s8 is None:
        s8 = torch.empty((M,), dtype=torch.float32, device=x.device)
    if q8.numel() < M * K:
        raise ValueError(f"q8_linear_kt: q8 holds {q8.numel()} bytes, needs {M * K}")
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=x.device)
    _check(load().phi_hip_q8_linear_kt(_stream(stream), _ptr(x), _dt(x), x.stride(0), M, K, _ptr(Wkt),
                                       _ptr(sW), 1 if sW.numel() == 1 else 0, _ptr(bias),
                                       _dt(bias) if bias is not None else F32, N, _ptr(C), _dt(C),
                                       C.stride(0), _ptr(q8), _ptr(s8), round_mode))
    return C
