"""CPU oracle for the grxBLAS / grxDNN hot path -- TEST INFRASTRUCTURE ONLY.

Thin ctypes wrapper over ``oracle/libgrx_oracle.so`` (built from
``grx_oracle.c`` by ``oracle/Makefile``). Only ``tests/``,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may
import this module, and only as the checker: the product (``grxcp_amd`` and
the ``libgrx*.so`` libraries) never touches it.

Each wrapped function names the reference file:line it restates; see
``grx_oracle.h``. Parity status per function:

=====================  =====================================================
function               pinned by (tests/test_oracle.py)
=====================  =====================================================
sgemm                  numpy float64 matmul, hand-computed 2x2 cases,
                       transpose identities, mutation checks
gemm_f32acc            exact-by-construction cases vs numpy float64 (exact
                       arithmetic makes the orders agree), mutation checks
igemm                  the reference's int8 known-answer tests
                       (ref src/backends/npu_c930/test_npu_c930.cc:183-238),
                       numpy int64 matmul, wrap-around vs numpy int32
dequant                numpy float32 multiply + independent RNE (torch
                       bfloat16 cast), scale == 1 special case
float_to_half et al.   numpy float16 casts over every 16-bit pattern
float_to_bf16          torch bfloat16 casts over sampled patterns
rmsnorm / layernorm    closed forms (constant rows, scale/shift invariance),
                       torch.nn.functional fp64 on CPU
attention_head         closed forms (row 0 -> V[0], Q = 0 -> prefix mean,
                       uniform V), torch scaled_dot_product_attention fp64
                       on CPU, mutation checks
softmax                closed forms (constant rows -> 1/n, two-element
                       logistic, shift invariance, rows sum to 1),
                       torch.softmax fp64 on CPU, mutation check
gelu                   published values (Phi(1), Phi(2) from the normal
                       table), the identity gelu(x) - gelu(-x) = x,
                       torch.nn.functional.gelu fp64 on CPU (both forms),
                       mutation check
=====================  =====================================================
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libgrx_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)


REF_ROOT = "/root/reference"
REF_DIR = os.path.join(_HERE, "_ref")
HOST_BLAS = os.path.join(_HERE, "libgrxblas_ref.so")
HOST_RT = os.path.join(_HERE, "libgrxrt_ref.so")


def build() -> str:
    """Compile the oracle and the CPU host backend (libgrxblas_ref.so,
    libgrxrt_ref.so) with the Makefile (gcc). Returns the oracle's path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def build_ref() -> bool:
    """Compile the reference's own grxBLAS callers (its three library gates
    and its cycle benchmark) from their sources under /root/reference into
    oracle/_ref/: once against the gfx950 libraries, once (the gates) against
    the CPU host backend. Needs the product libraries built first. Returns
    False, building nothing, where the reference is absent (the GPU box)."""
    if not os.path.isdir(REF_ROOT):
        return False
    subprocess.run(["make", "-s", "-C", _HERE, "ref", f"REF={REF_ROOT}"], check=True)
    return True


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        L.oracle_get_threads.restype = ctypes.c_int
        L.oracle_set_mutation.argtypes = [ctypes.c_int]
        L.oracle_lcg_next.argtypes = [ctypes.POINTER(ctypes.c_uint32)]
        L.oracle_lcg_next.restype = ctypes.c_uint32
        L.oracle_fill_quarters.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint32]
        L.oracle_fill_halves.argtypes = [_f32p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint32)]
        for name in ("oracle_f32_to_bf16_array", "oracle_f32_to_half_array"):
            getattr(L, name).argtypes = [_f32p, _u16p, ctypes.c_size_t]
        for name in ("oracle_bf16_to_f32_array", "oracle_half_to_f32_array"):
            getattr(L, name).argtypes = [_u16p, _f32p, ctypes.c_size_t]
        gemm_args = [ctypes.c_int] * 5 + [ctypes.c_float, _f32p, ctypes.c_int, _f32p,
                                          ctypes.c_int, ctypes.c_float, _f32p, ctypes.c_int]
        L.oracle_sgemm.argtypes = gemm_args
        L.oracle_gemm_f32acc.argtypes = gemm_args
        L.oracle_igemm.argtypes = [ctypes.c_int] * 5 + [ctypes.c_int32, _i8p, ctypes.c_int, _i8p,
                                                       ctypes.c_int, ctypes.c_int32, _i32p, ctypes.c_int]
        L.oracle_dequant.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_int, _f32p,
                                     _u16p, ctypes.c_int]
        L.oracle_rmsnorm.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                     ctypes.c_double, _f32p]
        L.oracle_layernorm.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                       _f32p, ctypes.c_double, _f32p]
        L.oracle_attention_head.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                            _f32p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int]
        L.oracle_softmax.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p]
        L.oracle_gelu.argtypes = [ctypes.c_long, ctypes.c_int, _f32p, _f32p]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(t)


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def get_threads() -> int:
    return int(lib().oracle_get_threads())


def set_mutation(which: int) -> None:
    lib().oracle_set_mutation(int(which))


# ---- generators (ref tests/libs/test_grxblas.cpp:108-113, test_grxblas_ex.cpp:33-36)

def fill_quarters(n: int, seed: int) -> np.ndarray:
    v = np.empty(n, np.float32)
    lib().oracle_fill_quarters(_p(v, _f32p), n, seed)
    return v


class HalvesStream:
    """The GemmEx gate's LCG stream: one seed continued across A, B, C."""

    def __init__(self, seed: int):
        self.seed = ctypes.c_uint32(seed)

    def take(self, n: int) -> np.ndarray:
        v = np.empty(n, np.float32)
        if n:
            lib().oracle_fill_halves(_p(v, _f32p), n, ctypes.byref(self.seed))
        return v


# ---- conversions

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_bf16_array(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_bf16_to_f32_array(_p(b, _u16p), _p(out, _f32p), b.size)
    return out


def f32_to_half(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_half_array(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def half_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_half_to_f32_array(_p(b, _u16p), _p(out, _f32p), b.size)
    return out


# ---- GEMMs (column-major flat buffers, as in grxBLAS)

def sgemm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc) -> np.ndarray:
    """ref tests/libs/test_grxblas.cpp:62-80 (fp64 accumulate). Returns new C."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    out = np.array(C, np.float32, copy=True)
    lib().oracle_sgemm(int(ta), int(tb), m, n, k, alpha, _p(A, _f32p), lda, _p(B, _f32p), ldb,
                       beta, _p(out, _f32p), ldc)
    return out


def gemm_f32acc(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc) -> np.ndarray:
    """ref tests/libs/test_grxblas_ex.cpp:45-63 (fp32 accumulate). Returns new C."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    out = np.array(C, np.float32, copy=True)
    lib().oracle_gemm_f32acc(int(ta), int(tb), m, n, k, alpha, _p(A, _f32p), lda, _p(B, _f32p),
                             ldb, beta, _p(out, _f32p), ldc)
    return out


def igemm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc) -> np.ndarray:
    """ref tests/libs/test_grxblas_ex.cpp:267-281 (int32, wraps). Returns new C."""
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    out = np.array(C, np.int32, copy=True)
    lib().oracle_igemm(int(ta), int(tb), m, n, k, int(alpha), _p(A, _i8p), lda, _p(B, _i8p), ldb,
                       int(beta), _p(out, _i32p), ldc)
    return out


def dequant(m, n, acc, ldacc, scale, ldy) -> np.ndarray:
    """bf16(f32(acc) * scale[col]) as uint16 bits, column major with ldy."""
    acc = np.ascontiguousarray(acc, np.int32)
    scale = np.ascontiguousarray(scale, np.float32)
    out = np.zeros(ldy * n, np.uint16)
    lib().oracle_dequant(m, n, _p(acc, _i32p), ldacc, _p(scale, _f32p), _p(out, _u16p), ldy)
    return out


# ---- norms and attention

def rmsnorm(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, hidden = x.shape
    g = np.ascontiguousarray(gamma, np.float32)
    y = np.empty_like(x)
    lib().oracle_rmsnorm(rows, hidden, hidden, _p(x, _f32p), _p(g, _f32p), eps, _p(y, _f32p))
    return y


def layernorm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, hidden = x.shape
    g = np.ascontiguousarray(gamma, np.float32)
    b = np.ascontiguousarray(beta, np.float32)
    y = np.empty_like(x)
    lib().oracle_layernorm(rows, hidden, hidden, _p(x, _f32p), _p(g, _f32p), _p(b, _f32p), eps,
                           _p(y, _f32p))
    return y


def softmax(x: np.ndarray) -> np.ndarray:
    """Softmax over the last axis of a 2-d float32 array."""
    x = np.ascontiguousarray(x, np.float32)
    rows, hidden = x.shape
    y = np.empty_like(x)
    lib().oracle_softmax(rows, hidden, hidden, _p(x, _f32p), _p(y, _f32p))
    return y


def gelu(x: np.ndarray, mode: int) -> np.ndarray:
    """GELU element-wise; mode 0 = erf form, 1 = tanh form."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().oracle_gelu(x.size, int(mode), _p(x, _f32p), _p(y, _f32p))
    return y


def attention_head(q, k, v, causal: bool, scale: float, row0: int = 0, row1: int | None = None):
    """One head, q/k/v [S, D] float32. Returns o [S, D] (rows outside
    [row0, row1) are zero)."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    S, D = q.shape
    if row1 is None:
        row1 = S
    o = np.zeros((S, D), np.float32)
    lib().oracle_attention_head(S, D, int(bool(causal)), float(scale), _p(q, _f32p), _p(k, _f32p),
                                _p(v, _f32p), _p(o, _f32p), int(row0), int(row1))
    return o
