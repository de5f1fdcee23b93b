"""hipgemm_amd -- MI355X (gfx950) FP8 e4m3 GEMM with bf16 output.

Host side of the library.  The compute path is libhipgemm.so (hand-written
HIP kernels for CDNA4 behind the C ABI of include/hipgemm.h); this module
binds that ABI with ctypes and, for convenience, accepts torch tensors, whose
device memory and current stream it passes through as plain pointers.

There is no CPU or library fallback: if libhipgemm.so is missing or fails to
load, every entry point raises HipGemmError.

Reference (nirw4nna/hipgemm) interface mirrored here:
  fp8_gemm_4wave_256x256x128(A, B_T, C)  -- the kernel of fp8_4wave.hpp:334-338
      as launched at test.cpp:79 / bench.cpp:78: C (M x N bf16) = A (M x K
      e4m3) . B_T (N x K e4m3)^T.
  fp8_gemm_bf16(...)                      -- the same with runtime strides,
      per-tensor scales, a stream and a schedule choice (C ABI
      hipgemm_fp8_gemm_bf16).
Argument errors raise HipGemmError (the C ABI returns hipErrorInvalidValue);
the reference has no error path (fp8_4wave.hpp has no shape checks).
"""
from __future__ import annotations

import ctypes
import os
import re
from typing import Optional

__all__ = [
    "HipGemmError", "lib", "lib_path", "fp8_gemm_bf16", "fp8_gemm",
    "fp8_gemm_4wave_256x256x128", "gemm_raw", "select_variant", "split_columns",
    "variant_name", "version", "tile_order", "lds_slot", "lds_slot_kpair",
    "lds_stage_slot",
    "VARIANTS",
    "declared_symbols", "gemm_raw_ws", "workspace_size",
    "fp8_gemm_bf16_rowcol", "gemm_raw_rowcol", "GemmDesc", "gemm_desc_raw",
    "gemm", "gemm_desc_noalloc_raw", "FMT_E4M3", "FMT_E5M2", "FMT_FP6_E2M3",
    "FMT_FP6_E3M2", "FMT_FP4_E2M1", "OUT_BF16", "OUT_F16", "OUT_F32",
    "OUT_FP8_E4M3", "ACTIVATIONS",
    "mx_scales_bytes", "mx_pack_scales",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_HERE)
_LIB_PATH = os.path.join(_HERE, "libhipgemm.so")
_HEADER = os.path.join(_ROOT, "include", "hipgemm.h")

VARIANTS = {"auto": 0, "4wave": 1, "4wave_mfma16": 2, "skinny": 3, "8wave": 4,
            "tile128": 5, "strip": 6}

# include/hipgemm.h codes
FMT_E4M3, FMT_E5M2, FMT_FP6_E2M3, FMT_FP6_E3M2, FMT_FP4_E2M1 = 0, 1, 2, 3, 4
OUT_BF16, OUT_F16, OUT_F32, OUT_FP8_E4M3 = 0, 1, 2, 3
ACTIVATIONS = {None: 0, "none": 0, "relu": 1, "gelu_tanh": 2, "silu": 3}

hipSuccess = 0
hipErrorInvalidValue = 1


class GemmDesc(ctypes.Structure):
    """hipgemm_gemm_desc (include/hipgemm.h)."""
    _fields_ = [("size", ctypes.c_size_t),
                ("A", ctypes.c_void_p), ("B_T", ctypes.c_void_p),
                ("C", ctypes.c_void_p),
                ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
                ("lda", ctypes.c_int), ("ldb", ctypes.c_int),
                ("ldc", ctypes.c_int),
                ("a_format", ctypes.c_int), ("b_format", ctypes.c_int),
                ("out_dtype", ctypes.c_int), ("activation", ctypes.c_int),
                ("scale_a", ctypes.c_void_p), ("scale_b", ctypes.c_void_p),
                ("scale_rows", ctypes.c_void_p),
                ("scale_cols", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("variant", ctypes.c_int),
                ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_size_t),
                ("mx_scale_a", ctypes.c_void_p),
                ("mx_scale_b", ctypes.c_void_p),
                ("scale_out", ctypes.c_void_p)]

    def __init__(self, **kw):
        super().__init__()
        self.size = ctypes.sizeof(GemmDesc)
        for k, v in kw.items():
            setattr(self, k, v or (None if k in _PTR_FIELDS else 0))


_PTR_FIELDS = {"A", "B_T", "C", "scale_a", "scale_b", "scale_rows",
               "scale_cols", "bias", "workspace", "mx_scale_a", "mx_scale_b",
               "scale_out"}


class HipGemmError(RuntimeError):
    """Raised for a missing library, bad arguments or a failed launch."""

    def __init__(self, msg: str, code: int = -1):
        super().__init__(msg)
        self.code = code


_lib: Optional[ctypes.CDLL] = None


def lib_path() -> str:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Load libhipgemm.so (once).  Raises HipGemmError if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise HipGemmError(
            f"{_LIB_PATH} is not built; run `python -m hipgemm_amd.build` "
            "(or __graft_entry__.build()).  There is no fallback path.")
    try:
        L = ctypes.CDLL(_LIB_PATH)
    except OSError as e:  # pragma: no cover - depends on the machine
        raise HipGemmError(f"cannot load {_LIB_PATH}: {e}") from e
    vp, ci = ctypes.c_void_p, ctypes.c_int
    L.hipgemm_fp8_gemm_bf16.argtypes = [vp, vp, vp, ci, ci, ci, ci, ci, ci,
                                        vp, vp, ci, vp]
    L.hipgemm_fp8_gemm_bf16.restype = ci
    L.hipgemm_fp8_gemm_bf16_ws.argtypes = [vp, vp, vp, ci, ci, ci, ci, ci,
                                           ci, vp, vp, ci, vp, ctypes.c_size_t,
                                           vp]
    L.hipgemm_fp8_gemm_bf16_ws.restype = ci
    L.hipgemm_fp8_gemm_bf16_rowcol.argtypes = [vp, vp, vp, ci, ci, ci, ci, ci,
                                               ci, vp, vp, ci, vp,
                                               ctypes.c_size_t, vp]
    L.hipgemm_fp8_gemm_bf16_rowcol.restype = ci
    L.hipgemm_gemm.argtypes = [ctypes.POINTER(GemmDesc), vp]
    L.hipgemm_gemm.restype = ci
    L.hipgemm_gemm_noalloc.argtypes = [ctypes.POINTER(GemmDesc), vp]
    L.hipgemm_gemm_noalloc.restype = ci
    L.hipgemm_mx_scales_bytes.argtypes = [ci, ci]
    L.hipgemm_mx_scales_bytes.restype = ctypes.c_size_t
    L.hipgemm_mx_pack_scales.argtypes = [vp, ci, ci, ci, vp, vp]
    L.hipgemm_mx_pack_scales.restype = ci
    L.hipgemm_workspace_size.argtypes = [ci, ci, ci, ci]
    L.hipgemm_workspace_size.restype = ctypes.c_size_t
    L.hipgemm_fp8_gemm_4wave_256x256x128.argtypes = [vp, vp, vp, ci, ci, ci,
                                                     vp]
    L.hipgemm_fp8_gemm_4wave_256x256x128.restype = ci
    L.hipgemm_select_variant.argtypes = [ci, ci, ci]
    L.hipgemm_select_variant.restype = ci
    L.hipgemm_split_columns.argtypes = [ci, ci, ci]
    L.hipgemm_split_columns.restype = ci
    L.hipgemm_gemm_workspace_size.argtypes = [ctypes.c_void_p]
    L.hipgemm_gemm_workspace_size.restype = ctypes.c_size_t
    L.hipgemm_variant_name.argtypes = [ci]
    L.hipgemm_variant_name.restype = ctypes.c_char_p
    L.hipgemm_version.argtypes = []
    L.hipgemm_version.restype = ci
    L.hipgemm_tile_order.argtypes = [ci, ci, ci, ci, vp, vp, ci]
    L.hipgemm_tile_order.restype = ci
    L.hipgemm_lds_slot.argtypes = [ci, ci]
    L.hipgemm_lds_slot.restype = ci
    L.hipgemm_lds_slot_kpair.argtypes = [ci, ci]
    L.hipgemm_lds_slot_kpair.restype = ci
    L.hipgemm_lds_stage_slot.argtypes = [ci, ci]
    L.hipgemm_lds_stage_slot.restype = ci
    _lib = L
    return L


def declared_symbols() -> list:
    """Function names declared in include/hipgemm.h."""
    with open(_HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hipgemm_[a-z0-9_]+)\s*\(", text)))


def _check(code: int, what: str) -> None:
    if code != hipSuccess:
        raise HipGemmError(f"{what} failed with hipError {code}", code)


def gemm_raw(a_ptr: int, b_ptr: int, c_ptr: int, M: int, N: int, K: int,
             lda: int, ldb: int, ldc: int, scale_a_ptr: int = 0,
             scale_b_ptr: int = 0, variant: int = 0, stream: int = 0) -> int:
    """Call hipgemm_fp8_gemm_bf16 on raw device pointers; returns hipError_t."""
    return int(lib().hipgemm_fp8_gemm_bf16(
        a_ptr or None, b_ptr or None, c_ptr or None, M, N, K, lda, ldb, ldc,
        scale_a_ptr or None, scale_b_ptr or None, variant, stream or None))


def gemm_raw_ws(a_ptr: int, b_ptr: int, c_ptr: int, M: int, N: int, K: int,
                lda: int, ldb: int, ldc: int, scale_a_ptr: int, scale_b_ptr: int,
                variant: int, ws_ptr: int, ws_bytes: int,
                stream: int = 0) -> int:
    """Call hipgemm_fp8_gemm_bf16_ws on raw device pointers."""
    return int(lib().hipgemm_fp8_gemm_bf16_ws(
        a_ptr or None, b_ptr or None, c_ptr or None, M, N, K, lda, ldb, ldc,
        scale_a_ptr or None, scale_b_ptr or None, variant, ws_ptr or None,
        ws_bytes, stream or None))


def gemm_raw_rowcol(a_ptr: int, b_ptr: int, c_ptr: int, M: int, N: int,
                    K: int, lda: int, ldb: int, ldc: int, rows_ptr: int,
                    cols_ptr: int, variant: int = 0, ws_ptr: int = 0,
                    ws_bytes: int = 0, stream: int = 0) -> int:
    """Call hipgemm_fp8_gemm_bf16_rowcol on raw device pointers (rows_ptr: M
    floats, cols_ptr: N floats, 0 = all ones)."""
    return int(lib().hipgemm_fp8_gemm_bf16_rowcol(
        a_ptr or None, b_ptr or None, c_ptr or None, M, N, K, lda, ldb, ldc,
        rows_ptr or None, cols_ptr or None, variant, ws_ptr or None, ws_bytes,
        stream or None))


def gemm_desc_raw(desc: "GemmDesc", stream: int = 0) -> int:
    """Call hipgemm_gemm; returns hipError_t."""
    return int(lib().hipgemm_gemm(ctypes.byref(desc), stream or None))


def gemm_desc_noalloc_raw(desc: "GemmDesc", stream: int = 0) -> int:
    """Call hipgemm_gemm_noalloc (the library's static per-GPU scratch
    instead of a workspace; desc.workspace must be 0); returns hipError_t."""
    return int(lib().hipgemm_gemm_noalloc(ctypes.byref(desc), stream or None))


def mx_scales_bytes(rows: int, K: int) -> int:
    """Bytes of the packed MX scale layout (hipgemm_mx_scales_bytes)."""
    return int(lib().hipgemm_mx_scales_bytes(rows, K))


def mx_pack_scales(scales, K: int, stream=None):
    """Packs E8M0 block scales (a uint8 device tensor rows x ceil(K/32),
    unit column stride) into the device layout hipgemm_gemm reads."""
    torch = _torch()
    if scales.dtype != torch.uint8 or scales.dim() != 2 or not scales.is_cuda \
            or (scales.numel() and scales.stride(1) != 1):
        raise HipGemmError("scales must be a 2-D uint8 device tensor with unit "
                           "column stride", hipErrorInvalidValue)
    rows = scales.shape[0]
    if scales.shape[1] != (K + 31) // 32:
        raise HipGemmError("scales must have ceil(K/32) columns",
                           hipErrorInvalidValue)
    stream = stream or torch.cuda.current_stream(scales.device)
    out = torch.empty(max(mx_scales_bytes(rows, K), 1), dtype=torch.uint8,
                      device=scales.device)
    ld = scales.stride(0) if rows > 1 else scales.shape[1]
    _check(int(lib().hipgemm_mx_pack_scales(
        scales.data_ptr() or None, rows, K, ld, out.data_ptr(),
        stream.cuda_stream or None)), "hipgemm_mx_pack_scales")
    return out


def workspace_size(M: int, N: int, K: int, variant: int = 0) -> int:
    """Workspace bytes hipgemm_fp8_gemm_bf16_ws needs (0 = none)."""
    return int(lib().hipgemm_workspace_size(M, N, K, variant))


def select_variant(M: int, N: int, K: int) -> int:
    return int(lib().hipgemm_select_variant(M, N, K))


def split_columns(M: int, N: int, K: int) -> int:
    """Columns of C that AUTO runs on the 4-wave schedule when it splits C
    between the 4-wave and 128 x 128 schedules; 0 when it does not."""
    return int(lib().hipgemm_split_columns(M, N, K))


def variant_name(v: int) -> Optional[str]:
    r = lib().hipgemm_variant_name(v)
    return r.decode() if r is not None else None


def version() -> int:
    return int(lib().hipgemm_version())


def tile_order(grid: int, tiles_m: int, tiles_n: int, group_m: int = 0):
    """(tile_m, tile_n) lists in the order the kernel's workgroups visit
    tiles (host-side view, no GPU)."""
    cap = tiles_m * tiles_n
    tm = (ctypes.c_int * cap)()
    tn = (ctypes.c_int * cap)()
    n = lib().hipgemm_tile_order(grid, tiles_m, tiles_n, group_m,
                                 ctypes.cast(tm, ctypes.c_void_p),
                                 ctypes.cast(tn, ctypes.c_void_p), cap)
    return list(tm[:n]), list(tn[:n])


def lds_slot(row: int, chunk: int) -> int:
    return int(lib().hipgemm_lds_slot(row, chunk))


def lds_slot_kpair(row: int, chunk: int) -> int:
    """Slot of K-chunk `chunk` of LDS row `row` in the instruction K order
    (hipgemm_lds_slot_kpair)."""
    return int(lib().hipgemm_lds_slot_kpair(row, chunk))


def lds_stage_slot(row: int, piece: int) -> int:
    """8-byte slot of 8-byte piece `piece` of row `row` of the 4-wave
    schedule's epilogue stage (hipgemm_lds_stage_slot)."""
    return int(lib().hipgemm_lds_stage_slot(row, piece))


# -- torch convenience layer ----------------------------------------------


def _torch():
    import torch  # noqa: WPS433 - torch is optional for the raw ABI
    return torch


def _as_bytes_2d(t, name):
    torch = _torch()
    if t.dim() != 2:
        raise HipGemmError(f"{name} must be 2-D, got {tuple(t.shape)}",
                           hipErrorInvalidValue)
    if t.dtype not in (torch.uint8, torch.float8_e4m3fn):
        raise HipGemmError(f"{name} must be float8_e4m3fn or uint8 bytes, got "
                           f"{t.dtype}", hipErrorInvalidValue)
    if not t.is_cuda:
        raise HipGemmError(f"{name} must be a device tensor",
                           hipErrorInvalidValue)
    if t.stride(1) != 1:
        raise HipGemmError(f"{name} must have unit stride along K",
                           hipErrorInvalidValue)
    return t


def _scale_ptr(s, name):
    if s is None:
        return 0
    torch = _torch()
    if not (isinstance(s, torch.Tensor) and s.is_cuda and
            s.dtype == torch.float32 and s.numel() == 1):
        raise HipGemmError(f"{name} must be a 1-element float32 device tensor",
                           hipErrorInvalidValue)
    return s.data_ptr()


def _vector_ptr(s, n, name):
    if s is None:
        return 0
    torch = _torch()
    if not (isinstance(s, torch.Tensor) and s.is_cuda and
            s.dtype == torch.float32 and s.dim() == 1 and s.numel() == n and
            (n <= 1 or s.stride(0) == 1)):
        raise HipGemmError(f"{name} must be a contiguous float32 device vector "
                           f"of {n} elements", hipErrorInvalidValue)
    return s.data_ptr()


def _mx_ptr(t, rows, K, name):
    if t is None:
        return 0
    torch = _torch()
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.uint8
            and t.numel() >= mx_scales_bytes(rows, K)):
        raise HipGemmError(f"{name} must be a packed uint8 device tensor "
                           "(mx_pack_scales)", hipErrorInvalidValue)
    return t.data_ptr()


def _gemm_operands(a, b_t, out, variant, stream, out_dtype=None):
    """Shared argument handling of the torch entry points: shapes, strides,
    output (out_dtype, default bfloat16), stream and workspace."""
    torch = _torch()
    out_dtype = out_dtype or torch.bfloat16
    a = _as_bytes_2d(a, "a")
    b_t = _as_bytes_2d(b_t, "b_t")
    M, K = a.shape
    N, K2 = b_t.shape
    if K2 != K:
        raise HipGemmError(f"K mismatch: a has {K}, b_t has {K2}",
                           hipErrorInvalidValue)
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    elif (out.dtype != out_dtype or tuple(out.shape) != (M, N) or
          (M > 0 and N > 0 and out.stride(1) != 1)):
        raise HipGemmError(f"out must be a (M, N) {out_dtype} tensor with unit "
                           "column stride", hipErrorInvalidValue)
    if stream is None:
        stream = torch.cuda.current_stream(a.device)
    lda = a.stride(0) if (M > 1 and K > 0) else max(K, 16)
    ldb = b_t.stride(0) if (N > 1 and K > 0) else max(K, 16)
    ldc = out.stride(0) if M > 1 else max(N, 1)
    nbytes = workspace_size(M, N, K, variant) if M > 0 and N > 0 else 0
    ws = _workspace(a.device, stream, nbytes) if nbytes else None
    if ws is None:
        nbytes = 0
    return (a, b_t, out, M, N, K, lda, ldb, ldc,
            ws.data_ptr() if ws is not None else 0, nbytes, stream)


def fp8_gemm_bf16(a, b_t, scale_a=None, scale_b=None, out=None,
                  variant: int = 0, stream=None):
    """out[M, N] (bf16) = scale_a * scale_b * a[M, K] @ b_t[N, K].T.

    a, b_t: device tensors of dtype float8_e4m3fn (or uint8 holding e4m3
    bytes) with unit stride along K.  scale_a / scale_b: optional 1-element
    float32 device tensors.  out: optional bf16 device tensor with unit column
    stride; allocated if None.  Runs on `stream` (a torch.cuda.Stream) or the
    current stream.
    """
    a, b_t, out, M, N, K, lda, ldb, ldc, ws, nbytes, stream = _gemm_operands(
        a, b_t, out, variant, stream)
    if not ws:
        # No workspace (none needed, or the stream is being captured): the
        # entry point that takes none.
        code = gemm_raw(a.data_ptr(), b_t.data_ptr(), out.data_ptr(), M, N, K,
                        lda, ldb, ldc, _scale_ptr(scale_a, "scale_a"),
                        _scale_ptr(scale_b, "scale_b"), variant,
                        stream.cuda_stream)
        _check(code, "hipgemm_fp8_gemm_bf16")
        return out
    code = gemm_raw_ws(a.data_ptr(), b_t.data_ptr(), out.data_ptr(), M, N, K,
                       lda, ldb, ldc, _scale_ptr(scale_a, "scale_a"),
                       _scale_ptr(scale_b, "scale_b"), variant, ws, nbytes,
                       stream.cuda_stream)
    _check(code, "hipgemm_fp8_gemm_bf16_ws")
    return out


def gemm(a, b_t, *, a_format: int = FMT_E4M3, b_format: int = FMT_E4M3,
         out_dtype=None, scale_a=None, scale_b=None, scale_rows=None,
         scale_cols=None, bias=None, activation=None, out=None,
         variant: int = 0, stream=None, mx_scale_a=None, mx_scale_b=None,
         scale_out=None):
    """The general entry point (hipgemm_gemm): out[m, n] =
    round(act(fma(acc, scale_rows[m] * (scale_cols[n] * (scale_a *
    scale_b)), bias[n]))), acc = a @ b_t.T with a in a_format and b_t in
    b_format (FMT_E4M3 / FMT_E5M2; float8_e4m3fn / float8_e5m2 tensors set
    it from their dtype; FMT_FP4_E2M1 for both, or float4_e2m1fn_x2
    tensors: K / 2 bytes per row, element 2i in the low nibble).  out_dtype: torch.bfloat16 (default),
    torch.float16, torch.float32 or torch.float8_e4m3fn (saturating; then
    scale_out, a 1-element float32 device tensor, multiplies the activated
    value before the conversion).  activation: None, "relu", "gelu_tanh" or
    "silu".
    scale_a / scale_b: 1-element float32 device tensors; scale_rows (M),
    scale_cols (N), bias (N): float32 device vectors; any may be None.
    mx_scale_a / mx_scale_b: MX block scales packed by mx_pack_scales
    (both or neither)."""
    torch = _torch()
    fmts = {torch.float8_e4m3fn: FMT_E4M3, torch.float8_e5m2: FMT_E5M2,
            torch.float4_e2m1fn_x2: FMT_FP4_E2M1}
    a_format = fmts.get(a.dtype, a_format)
    b_format = fmts.get(b_t.dtype, b_format)
    if a.dtype == torch.float4_e2m1fn_x2:
        a = a.view(torch.uint8)
    if b_t.dtype == torch.float4_e2m1fn_x2:
        b_t = b_t.view(torch.uint8)
    out_dtype = out_dtype or (out.dtype if out is not None else torch.bfloat16)
    codes = {torch.bfloat16: OUT_BF16, torch.float16: OUT_F16,
             torch.float32: OUT_F32, torch.float8_e4m3fn: OUT_FP8_E4M3}
    if out_dtype not in codes:
        raise HipGemmError("out_dtype must be bfloat16, float16, float32 or "
                           "float8_e4m3fn", hipErrorInvalidValue)
    if activation not in ACTIVATIONS:
        raise HipGemmError(f"activation must be one of {sorted(k for k in ACTIVATIONS if k)}",
                           hipErrorInvalidValue)
    if out is not None and out.dtype != out_dtype:
        raise HipGemmError("out has the wrong dtype", hipErrorInvalidValue)
    a, b_t, out, M, N, K, lda, ldb, ldc, ws, nbytes, stream = _gemm_operands(
        a.view(torch.uint8) if a.dtype == torch.float8_e5m2 else a,
        b_t.view(torch.uint8) if b_t.dtype == torch.float8_e5m2 else b_t,
        out, variant, stream, out_dtype)
    if a_format == FMT_FP4_E2M1 or b_format == FMT_FP4_E2M1:
        K *= 2  # elements: two per byte
    elif a_format in (FMT_FP6_E2M3, FMT_FP6_E3M2):
        if K % 3:
            raise HipGemmError("fp6 operands hold 4 elements per 3 bytes: the "
                               "row length in bytes must be a multiple of 3",
                               hipErrorInvalidValue)
        K = K // 3 * 4  # elements: four per three bytes
    d = GemmDesc(A=a.data_ptr(), B_T=b_t.data_ptr(), C=out.data_ptr(), M=M,
                 N=N, K=K, lda=lda, ldb=ldb, ldc=ldc, a_format=a_format,
                 b_format=b_format,
                 out_dtype=codes[out_dtype],
                 activation=ACTIVATIONS[activation],
                 scale_a=_scale_ptr(scale_a, "scale_a"),
                 scale_b=_scale_ptr(scale_b, "scale_b"),
                 scale_rows=_vector_ptr(scale_rows, M, "scale_rows"),
                 scale_cols=_vector_ptr(scale_cols, N, "scale_cols"),
                 bias=_vector_ptr(bias, N, "bias"), variant=variant,
                 workspace=ws, workspace_bytes=nbytes,
                 mx_scale_a=_mx_ptr(mx_scale_a, M, K, "mx_scale_a"),
                 mx_scale_b=_mx_ptr(mx_scale_b, N, K, "mx_scale_b"),
                 scale_out=_scale_ptr(scale_out, "scale_out"))
    need = int(lib().hipgemm_gemm_workspace_size(ctypes.byref(d)))
    if need != nbytes:  # the formats and MX scales decide the schedule
        w = _workspace(a.device, stream, need) if need else None
        d.workspace = w.data_ptr() if w is not None else None
        d.workspace_bytes = need if w is not None else 0
    _check(gemm_desc_raw(d, stream.cuda_stream), "hipgemm_gemm")
    return out


def fp8_gemm_bf16_rowcol(a, b_t, scale_rows=None, scale_cols=None, out=None,
                         variant: int = 0, stream=None):
    """out[m, n] (bf16) = scale_rows[m] * scale_cols[n] * (a @ b_t.T)[m, n].

    As fp8_gemm_bf16, with per-row scales of a (a float32 device vector of M
    elements) and per-column scales of the output (one per row of b_t: N
    elements); either may be None for all ones.  variant 1 (the 32x32x64
    schedule) is not available here.
    """
    a, b_t, out, M, N, K, lda, ldb, ldc, ws, nbytes, stream = _gemm_operands(
        a, b_t, out, variant, stream)
    code = gemm_raw_rowcol(a.data_ptr(), b_t.data_ptr(), out.data_ptr(), M, N,
                           K, lda, ldb, ldc,
                           _vector_ptr(scale_rows, M, "scale_rows"),
                           _vector_ptr(scale_cols, N, "scale_cols"), variant,
                           ws, nbytes, stream.cuda_stream)
    _check(code, "hipgemm_fp8_gemm_bf16_rowcol")
    return out


# Workspaces of the split-K schedules, one per (device, stream): calls on one
# stream are ordered, so they may share one (include/hipgemm.h: the counter
# region is zero between calls whatever schedule ran last).  A workspace is
# never freed once created: a CUDA graph captured with it keeps its address,
# so a smaller one stays alive (in _retired) when a larger one replaces it.
# Growth at least doubles the size, which bounds the retired bytes by the
# live ones.  None is created or grown while the stream is being captured
# (the allocation and its zero fill would only be recorded, not run): the
# call then goes to the C ABI without one, which runs a schedule that would
# split K unsplit (include/hipgemm.h).
_workspaces: dict = {}
_retired: list = []


def _workspace(device, stream, nbytes: int):
    """The stream's workspace of at least nbytes, or None while `stream` is
    being captured and has none that large."""
    torch = _torch()
    key = (device.index, stream.cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        # The capture status of `stream` itself (it need not be the current
        # stream).
        with torch.cuda.stream(stream):
            capturing = torch.cuda.is_current_stream_capturing()
        if capturing:
            return None
        size = nbytes if ws is None else max(nbytes, 2 * ws.numel())
        with torch.cuda.stream(stream):
            new = torch.zeros(size, dtype=torch.uint8, device=device)
        if ws is not None:
            _retired.append(ws)
        _workspaces[key] = ws = new
    return ws


fp8_gemm = fp8_gemm_bf16


def fp8_gemm_4wave_256x256x128(A, B_T, C, stream=None):
    """Mirror of the reference launch (test.cpp:79): C = A @ B_T.T with packed
    strides (lda = ldb = K, ldc = N), no scales, the 4-wave schedule."""
    torch = _torch()
    A = _as_bytes_2d(A, "A")
    B_T = _as_bytes_2d(B_T, "B_T")
    M, K = A.shape
    N = B_T.shape[0]
    if not (A.is_contiguous() and B_T.is_contiguous() and C.is_contiguous()):
        raise HipGemmError("A, B_T and C must be contiguous",
                           hipErrorInvalidValue)
    if C.dtype != torch.bfloat16 or tuple(C.shape) != (M, N):
        raise HipGemmError("C must be a contiguous (M, N) bfloat16 tensor",
                           hipErrorInvalidValue)
    if stream is None:
        stream = torch.cuda.current_stream(A.device)
    code = int(lib().hipgemm_fp8_gemm_4wave_256x256x128(
        A.data_ptr(), B_T.data_ptr(), C.data_ptr(), M, N, K,
        stream.cuda_stream or None))
    _check(code, "hipgemm_fp8_gemm_4wave_256x256x128")
    return C
