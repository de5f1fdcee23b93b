"""ctypes bindings for the hipgemm CPU oracle.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, always as the checker.  The product
package ``hipgemm_amd`` never imports this module.

Libraries (built by ``oracle/Makefile``):
  liboracle.so        C restatement of the reference path (oracle.c,
                      reftest_rng.cpp); see oracle.h for what pins each part.
  libpin_hipconv.so   HIP-header conversions, for the exhaustive codec pin.
  _ref/libref_test.so the reference's own test.cpp (gemm_cpu, init_random,
                      validate_matrix) built from its sources; optional.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

UNIFORM = 0
NORMAL = 1
# hg_gemm_ex codes (oracle.h; the values of include/hipgemm.h's)
FMT_E4M3, FMT_E5M2, FMT_FP6_E2M3, FMT_FP6_E3M2, FMT_FP4 = 0, 1, 2, 3, 4
FP6 = (FMT_FP6_E2M3, FMT_FP6_E3M2)


def k_elements(fmt: int, row_bytes: int) -> int:
    """Elements in a packed row of row_bytes bytes: fp4 two per byte, fp6
    four per three bytes, the 8-bit formats one per byte."""
    if fmt == FMT_FP4:
        return 2 * row_bytes
    if fmt in FP6:
        assert row_bytes % 3 == 0
        return row_bytes * 4 // 3
    return row_bytes
OUT_BF16, OUT_F16, OUT_F32, OUT_FP8 = 0, 1, 2, 3
ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3

_c_u8p = ctypes.POINTER(ctypes.c_uint8)
_vp = ctypes.c_void_p


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


class Oracle:
    """Thin wrapper over liboracle.so."""

    def __init__(self, path: Optional[str] = None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} missing: build it with `make -C oracle` "
                "(or __graft_entry__.build())")
        self.lib = L = ctypes.CDLL(path)
        L.hg_f32_to_e4m3.restype = ctypes.c_uint8
        L.hg_f32_to_e4m3.argtypes = [ctypes.c_float]
        L.hg_e4m3_to_f32.restype = ctypes.c_float
        L.hg_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.hg_f32_to_bf16.restype = ctypes.c_uint16
        L.hg_f32_to_bf16.argtypes = [ctypes.c_float]
        L.hg_bf16_to_f32.restype = ctypes.c_float
        L.hg_bf16_to_f32.argtypes = [ctypes.c_uint16]
        for name in ("hg_f32_to_e4m3_n", "hg_e4m3_to_f32_n",
                     "hg_f32_to_bf16_n", "hg_bf16_to_f32_n",
                     "hg_e5m2_to_f32_n", "hg_f32_to_e5m2_n",
                     "hg_f32_to_f16_n"):
            getattr(L, name).argtypes = [_vp, _vp, ctypes.c_size_t]
            getattr(L, name).restype = None
        L.hg_fp4_to_f32.argtypes = [ctypes.c_uint8]
        L.hg_fp4_to_f32.restype = ctypes.c_float
        for name in ("hg_fp6_e2m3_to_f32", "hg_fp6_e3m2_to_f32"):
            getattr(L, name).argtypes = [ctypes.c_uint8]
            getattr(L, name).restype = ctypes.c_float
        L.hg_rand64.restype = ctypes.c_uint64
        L.hg_rand64.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.hg_fill_e4m3.argtypes = [_vp, ctypes.c_size_t, ctypes.c_uint64,
                                   ctypes.c_int, ctypes.c_double,
                                   ctypes.c_double]
        L.hg_fill_e4m3.restype = None
        L.hg_fill_e4m3_reftest.argtypes = [_vp, ctypes.c_size_t,
                                           ctypes.c_uint64]
        L.hg_fill_e4m3_reftest.restype = None
        L.hg_draw_scale.restype = ctypes.c_float
        L.hg_draw_scale.argtypes = [ctypes.c_uint64, ctypes.c_double,
                                    ctypes.c_double]
        gemm_args = [_vp, _vp, _vp] + [ctypes.c_int] * 6 + [ctypes.c_float] * 2
        for name in ("hg_gemm_ref", "hg_gemm_fast"):
            getattr(L, name).argtypes = gemm_args
            getattr(L, name).restype = None
        L.hg_gemm_rowcol.argtypes = [_vp, _vp, _vp] + [ctypes.c_int] * 6 + \
            [_vp, _vp]
        L.hg_gemm_rowcol.restype = None
        L.hg_gemm_ex.argtypes = [_vp, _vp, _vp] + [ctypes.c_int] * 10 + \
            [ctypes.c_float] * 2 + [_vp, _vp, _vp, ctypes.c_float]
        L.hg_gemm_ex.restype = None
        L.hg_gemm_mx.argtypes = [_vp, _vp, _vp] + [ctypes.c_int] * 8 + \
            [_vp, ctypes.c_int, _vp, ctypes.c_int] + [ctypes.c_float] * 2
        L.hg_gemm_mx.restype = None
        L.hg_gemm_rows.argtypes = [_vp, _vp, _vp, _vp] + [ctypes.c_int] * 5 + \
            [ctypes.c_float] * 2
        L.hg_gemm_rows.restype = None
        for name in ("hg_gemm_rows_acc", "hg_gemm_rows_f64"):
            getattr(L, name).argtypes = [_vp, _vp, _vp, _vp] + [ctypes.c_int] * 5
            getattr(L, name).restype = None
        L.hg_num_threads.restype = ctypes.c_int

    # -- codecs ------------------------------------------------------------
    def f32_to_e4m3(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint8)
        self.lib.hg_f32_to_e4m3_n(_ptr(x), _ptr(out), x.size)
        return out

    def e4m3_to_f32(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.uint8)
        out = np.empty(x.shape, np.float32)
        self.lib.hg_e4m3_to_f32_n(_ptr(x), _ptr(out), x.size)
        return out

    def f32_to_bf16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.hg_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
        return out

    def bf16_to_f32(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.uint16)
        out = np.empty(x.shape, np.float32)
        self.lib.hg_bf16_to_f32_n(_ptr(x), _ptr(out), x.size)
        return out

    def e5m2_to_f32(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.uint8)
        out = np.empty(x.shape, np.float32)
        self.lib.hg_e5m2_to_f32_n(_ptr(x), _ptr(out), x.size)
        return out

    def f32_to_e5m2(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint8)
        self.lib.hg_f32_to_e5m2_n(_ptr(x), _ptr(out), x.size)
        return out

    def f32_to_f16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.hg_f32_to_f16_n(_ptr(x), _ptr(out), x.size)
        return out

    def fp4_to_f32(self, nibbles: np.ndarray) -> np.ndarray:
        """OCP E2M1 values of nibble codes 0..15 (hg_fp4_to_f32)."""
        return np.array([self.lib.hg_fp4_to_f32(int(v) & 15) for v in
                         np.asarray(nibbles).reshape(-1)],
                        np.float32).reshape(np.shape(nibbles))

    def fp6_to_f32(self, codes: np.ndarray, fmt: int) -> np.ndarray:
        """OCP FP6 values of 6-bit codes 0..63 (hg_fp6_e2m3_to_f32 /
        hg_fp6_e3m2_to_f32)."""
        fn = (self.lib.hg_fp6_e2m3_to_f32 if fmt == FMT_FP6_E2M3
              else self.lib.hg_fp6_e3m2_to_f32)
        return np.array([fn(int(v) & 63) for v in np.asarray(codes).reshape(-1)],
                        np.float32).reshape(np.shape(codes))

    def decode(self, x: np.ndarray, fmt: int) -> np.ndarray:
        """fp32 values of 8-bit operands in format fmt (FMT_E4M3 / FMT_E5M2)."""
        return self.e5m2_to_f32(x) if fmt == FMT_E5M2 else self.e4m3_to_f32(x)

    # -- generators --------------------------------------------------------
    def fill(self, shape: Sequence[int], seed: int, dist: int = UNIFORM,
             p0: float = -1.0, p1: float = 1.0) -> np.ndarray:
        out = np.empty(tuple(shape), np.uint8)
        self.lib.hg_fill_e4m3(_ptr(out), out.size, seed, dist, p0, p1)
        return out

    def fill_reftest(self, shape: Sequence[int], seed: int) -> np.ndarray:
        out = np.empty(tuple(shape), np.uint8)
        self.lib.hg_fill_e4m3_reftest(_ptr(out), out.size, seed)
        return out

    def draw_scale(self, seed: int, lo: float = 0.5, hi: float = 2.0) -> float:
        return float(self.lib.hg_draw_scale(seed, lo, hi))

    # -- GEMM --------------------------------------------------------------
    @staticmethod
    def _check(A, B, M, N, K, lda, ldb):
        assert A.dtype == np.uint8 and B.dtype == np.uint8
        assert A.size >= (M - 1) * lda + K if M > 0 else True
        assert B.size >= (N - 1) * ldb + K if N > 0 else True

    def gemm(self, A: np.ndarray, B: np.ndarray, scale_a: float = 1.0,
             scale_b: float = 1.0, faithful: bool = False) -> np.ndarray:
        """bf16 bits of scale_a*scale_b * A @ B.T, A: M x K, B: N x K."""
        A = np.ascontiguousarray(A)
        B = np.ascontiguousarray(B)
        M, K = A.shape
        N = B.shape[0]
        assert B.shape[1] == K
        C = np.empty((M, N), np.uint16)
        fn = self.lib.hg_gemm_ref if faithful else self.lib.hg_gemm_fast
        fn(_ptr(A), _ptr(B), _ptr(C), M, N, K, K, K, N, scale_a, scale_b)
        return C

    def gemm_rowcol(self, A: np.ndarray, B: np.ndarray,
                    scale_rows: Optional[np.ndarray] = None,
                    scale_cols: Optional[np.ndarray] = None) -> np.ndarray:
        """bf16 bits of (scale_rows[m] * scale_cols[n]) * (A @ B.T)[m, n];
        either vector may be None (1.0)."""
        A = np.ascontiguousarray(A)
        B = np.ascontiguousarray(B)
        M, K = A.shape
        N = B.shape[0]
        assert B.shape[1] == K
        sr = None if scale_rows is None else np.ascontiguousarray(scale_rows, np.float32)
        sc = None if scale_cols is None else np.ascontiguousarray(scale_cols, np.float32)
        assert sr is None or sr.shape == (M,)
        assert sc is None or sc.shape == (N,)
        C = np.empty((M, N), np.uint16)
        self.lib.hg_gemm_rowcol(_ptr(A), _ptr(B), _ptr(C), M, N, K, K, K, N,
                                None if sr is None else _ptr(sr),
                                None if sc is None else _ptr(sc))
        return C

    def gemm_ex(self, A: np.ndarray, B: np.ndarray, a_fmt: int = FMT_E4M3,
                b_fmt: int = FMT_E4M3, out: int = OUT_BF16, act: int = ACT_NONE,
                scale_a: float = 1.0, scale_b: float = 1.0,
                scale_rows: Optional[np.ndarray] = None,
                scale_cols: Optional[np.ndarray] = None,
                bias: Optional[np.ndarray] = None,
                scale_out: float = 1.0) -> np.ndarray:
        """Output bits of the hipgemm_gemm semantics (oracle.h: hg_gemm_ex):
        uint16 (bf16 / f16), uint32 (fp32 bits) or uint8 (e4m3).  fp4
        operands (a_fmt = b_fmt = FMT_FP4): A and B hold K / 2 bytes per
        row, two elements per byte; fp6 operands (both in FP6, either
        variant): 3 K / 4 bytes per row, packed LSB first."""
        A = np.ascontiguousarray(A)
        B = np.ascontiguousarray(B)
        M, Kb = A.shape
        N = B.shape[0]
        assert B.shape[1] == Kb
        assert (a_fmt == FMT_FP4) == (b_fmt == FMT_FP4)
        assert (a_fmt in FP6) == (b_fmt in FP6)
        K = k_elements(a_fmt, Kb)

        def vec(v, n):
            if v is None:
                return None
            v = np.ascontiguousarray(v, np.float32)
            assert v.shape == (n,)
            return v
        sr, sc, bb = vec(scale_rows, M), vec(scale_cols, N), vec(bias, N)
        C = np.empty((M, N), {OUT_F32: np.uint32, OUT_FP8: np.uint8}.get(out, np.uint16))
        self.lib.hg_gemm_ex(_ptr(A), _ptr(B), _ptr(C), M, N, K, Kb, Kb, N,
                            a_fmt, b_fmt, out, act, scale_a, scale_b,
                            None if sr is None else _ptr(sr),
                            None if sc is None else _ptr(sc),
                            None if bb is None else _ptr(bb), scale_out)
        return C

    def gemm_mx(self, A: np.ndarray, B: np.ndarray, sa: np.ndarray,
                sb: np.ndarray, a_fmt: int = FMT_E4M3, b_fmt: int = FMT_E4M3,
                scale_a: float = 1.0, scale_b: float = 1.0) -> np.ndarray:
        """bf16 bits of the MX-scaled product (oracle.h: hg_gemm_mx); sa: M x
        ceil(K/32) E8M0 bytes, sb: N x ceil(K/32), K in elements (fp4: A and
        B hold K / 2 bytes per row)."""
        A = np.ascontiguousarray(A)
        B = np.ascontiguousarray(B)
        M, Kb = A.shape
        N = B.shape[0]
        assert (a_fmt == FMT_FP4) == (b_fmt == FMT_FP4)
        assert (a_fmt in FP6) == (b_fmt in FP6)
        K = k_elements(a_fmt, Kb)
        kb = (K + 31) // 32
        sa = np.ascontiguousarray(sa, np.uint8)
        sb = np.ascontiguousarray(sb, np.uint8)
        assert B.shape[1] == Kb and sa.shape == (M, kb) and sb.shape == (N, kb)
        C = np.empty((M, N), np.uint16)
        self.lib.hg_gemm_mx(_ptr(A), _ptr(B), _ptr(C), M, N, K, Kb, Kb, N,
                            a_fmt, b_fmt, _ptr(sa), kb, _ptr(sb), kb,
                            scale_a, scale_b)
        return C

    def gemm_rows(self, A: np.ndarray, B: np.ndarray, rows: Sequence[int],
                  scale_a: float = 1.0, scale_b: float = 1.0) -> np.ndarray:
        A = np.ascontiguousarray(A)
        B = np.ascontiguousarray(B)
        K = A.shape[1]
        N = B.shape[0]
        r = np.ascontiguousarray(np.asarray(rows, dtype=np.int32))
        assert r.size == 0 or (r.min() >= 0 and r.max() < A.shape[0])
        C = np.empty((r.size, N), np.uint16)
        self.lib.hg_gemm_rows(_ptr(A), _ptr(B), _ptr(C), _ptr(r), r.size, N, K,
                              K, K, scale_a, scale_b)
        return C

    def gemm_rows_acc(self, A, B, rows) -> np.ndarray:
        A = np.ascontiguousarray(A)
        B = np.ascontiguousarray(B)
        r = np.ascontiguousarray(np.asarray(rows, dtype=np.int32))
        out = np.empty((r.size, B.shape[0]), np.float32)
        self.lib.hg_gemm_rows_acc(_ptr(A), _ptr(B), _ptr(out), _ptr(r), r.size,
                                  B.shape[0], A.shape[1], A.shape[1],
                                  A.shape[1])
        return out

    def gemm_rows_f64(self, A, B, rows) -> np.ndarray:
        A = np.ascontiguousarray(A)
        B = np.ascontiguousarray(B)
        r = np.ascontiguousarray(np.asarray(rows, dtype=np.int32))
        out = np.empty((r.size, B.shape[0]), np.float64)
        self.lib.hg_gemm_rows_f64(_ptr(A), _ptr(B), _ptr(out), _ptr(r), r.size,
                                  B.shape[0], A.shape[1], A.shape[1],
                                  A.shape[1])
        return out

    def num_threads(self) -> int:
        return int(self.lib.hg_num_threads())


class HipConvPin:
    """HIP-header host conversions (libpin_hipconv.so)."""

    def __init__(self, path: Optional[str] = None):
        path = path or os.path.join(HERE, "libpin_hipconv.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = L = ctypes.CDLL(path)
        L.hg_pin_hip_f32_to_e4m3.restype = ctypes.c_uint8
        L.hg_pin_hip_f32_to_e4m3.argtypes = [ctypes.c_float]
        L.hg_pin_hip_e4m3_to_f32.restype = ctypes.c_float
        L.hg_pin_hip_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.hg_pin_hip_f32_to_bf16.restype = ctypes.c_uint16
        L.hg_pin_hip_f32_to_bf16.argtypes = [ctypes.c_float]
        L.hg_pin_sweep.restype = ctypes.c_uint64
        L.hg_pin_sweep.argtypes = [ctypes.c_int, ctypes.c_uint64,
                                   ctypes.c_uint64, _vp, ctypes.c_uint64,
                                   ctypes.POINTER(ctypes.c_uint64)]

    def sweep(self, what: int, lo: int = 0, hi: int = 1 << 32, cap: int = 64):
        bad = np.zeros(cap, np.uint32)
        tiny = ctypes.c_uint64(0)
        n = self.lib.hg_pin_sweep(what, lo, hi, _ptr(bad), cap,
                                  ctypes.byref(tiny))
        return int(n), bad[: min(int(n), cap)], int(tiny.value)


class RefLib:
    """The reference's own host functions, compiled from its sources into
    oracle/_ref/libref_test.so by ``make -C oracle ref``.  Absent on machines
    where the reference sources were not available at build time."""

    SYMS = {
        "gemm_cpu": "_Z8gemm_cpuP14__hip_fp8_e4m3S0_P14__hip_bfloat16iii",
        "init_random": "_Z11init_randomP14__hip_fp8_e4m3mm",
        "validate_matrix": "_Z15validate_matrixP14__hip_bfloat16S0_ii",
    }

    def __init__(self, path: Optional[str] = None):
        path = path or os.path.join(HERE, "_ref", "libref_test.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = ctypes.CDLL(path)
        self.gemm_cpu_fn = getattr(self.lib, self.SYMS["gemm_cpu"])
        self.gemm_cpu_fn.argtypes = [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int]
        self.gemm_cpu_fn.restype = None
        self.init_random_fn = getattr(self.lib, self.SYMS["init_random"])
        self.init_random_fn.argtypes = [_vp, ctypes.c_size_t, ctypes.c_size_t]
        self.init_random_fn.restype = None
        self.validate_fn = getattr(self.lib, self.SYMS["validate_matrix"])
        self.validate_fn.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int]
        self.validate_fn.restype = ctypes.c_bool

    @staticmethod
    def available(path: Optional[str] = None) -> bool:
        return os.path.exists(path or os.path.join(HERE, "_ref",
                                                   "libref_test.so"))

    def gemm_cpu(self, A: np.ndarray, B: np.ndarray) -> np.ndarray:
        """test.cpp:19-30 on contiguous A (M x K), B (N x K); bf16 bits."""
        A = np.ascontiguousarray(A, dtype=np.uint8)
        B = np.ascontiguousarray(B, dtype=np.uint8)
        M, K = A.shape
        N = B.shape[0]
        C = np.empty((M, N), np.uint16)
        self.gemm_cpu_fn(_ptr(A), _ptr(B), _ptr(C), M, N, K)
        return C

    def init_random(self, n: int, seed: int) -> np.ndarray:
        out = np.empty(n, np.uint8)
        self.init_random_fn(_ptr(out), n, seed)
        return out


class RefGpu:
    """The reference's GPU kernel (fp8_4wave.hpp:334-567) behind the launcher
    of ref_kernel_launch.hip, built into oracle/_ref/libref_gpu.so by ``make
    -C oracle ref``.  Measurement only: bench.py times it beside the product
    kernel.  It has no scales and truncates to bf16."""

    SHAPES = {(4096, 4096, 4096), (8192, 8192, 8192), (8192, 28672, 8192),
              (8192, 8192, 28672)}

    def __init__(self, path: Optional[str] = None):
        path = path or os.path.join(HERE, "_ref", "libref_gpu.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = ctypes.CDLL(path)
        self.fn = self.lib.hipgemm_reference_4wave
        self.fn.argtypes = [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int,
                            ctypes.c_int, _vp]
        self.fn.restype = ctypes.c_int

    def launch(self, A_ptr: int, B_ptr: int, C_ptr: int, M: int, N: int,
               K: int, stream_ptr: int) -> None:
        err = self.fn(A_ptr, B_ptr, C_ptr, M, N, K, stream_ptr)
        if err != 0:
            raise RuntimeError(f"reference kernel launch failed: {err}")


_oracle: Optional[Oracle] = None


def get() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle
