"""grxcp_amd -- MI355X (gfx950) grxBLAS / grxDNN, Python side.

The product is three C-ABI shared libraries built in-tree by
``grxcp_amd/build.py`` into ``grxcp_amd/lib/``:

* ``libgrxrt.so``   -- ``include/grx/grx_runtime.h`` (device, memory, streams, events)
* ``libgrxblas.so`` -- ``include/grx/grxblas.h``
* ``libgrxdnn.so``  -- ``include/grx/grxdnn.h``

This module binds them with ctypes, exactly as a C caller links them: the
signatures below are the header declarations. It adds only plumbing for tests
and the benchmark (device buffers, status checking). There is no fallback: if
the libraries are missing, :func:`load` raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_longlong, c_size_t, c_uint, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBDIR = os.path.join(HERE, "lib")

# ---- enumerators (values from the headers) -------------------------------
GRX_R_32F, GRX_R_16F, GRX_R_8I, GRX_R_32I, GRX_R_16BF = 0, 2, 3, 10, 14
OP_N, OP_T = 0, 1
STATUS = {
    0: "SUCCESS", 1: "NOT_INITIALIZED", 2: "ALLOC_FAILED", 3: "INVALID_VALUE",
    4: "ARCH_MISMATCH", 5: "EXECUTION_FAILED", 6: "NOT_SUPPORTED", 7: "INTERNAL_ERROR",
}
SUCCESS, NOT_INITIALIZED, ALLOC_FAILED, INVALID_VALUE = 0, 1, 2, 3
GELU_ERF, GELU_TANH = 0, 1
ARCH_MISMATCH, EXECUTION_FAILED, NOT_SUPPORTED, INTERNAL_ERROR = 4, 5, 6, 7
TENSOR_FP16, TENSOR_TF32, TENSOR_FP8, TENSOR_FP4 = 0x01, 0x02, 0x04, 0x08
TENSOR_INT8, TENSOR_INT4, TENSOR_BF16 = 0x10, 0x20, 0x40
MEMCPY_DEFAULT = 4


class GrxError(RuntimeError):
    pass


class CycleSlot(ctypes.Structure):
    _fields_ = [("start", ctypes.c_uint64), ("end", ctypes.c_uint64),
                ("core", ctypes.c_uint32), ("warp", ctypes.c_uint32)]


_libs = None

# name -> (restype, argtypes) for every exported entry point
_RT = {
    "grxGetErrorName": (c_char_p, [c_int]),
    "grxGetErrorString": (c_char_p, [c_int]),
    "grxGetDeviceCount": (c_int, [POINTER(c_int)]),
    "grxSetDevice": (c_int, [c_int]),
    "grxGetDevice": (c_int, [POINTER(c_int)]),
    "grxGetDeviceProperties": (c_int, [c_void_p, c_int]),
    "grxDeviceSynchronize": (c_int, []),
    "grxMemGetInfo": (c_int, [POINTER(c_size_t), POINTER(c_size_t)]),
    "grxGetLastError": (c_int, []),
    "grxPeekAtLastError": (c_int, []),
    "grxMalloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "grxFree": (c_int, [c_void_p]),
    "grxMallocHost": (c_int, [POINTER(c_void_p), c_size_t]),
    "grxFreeHost": (c_int, [c_void_p]),
    "grxMemcpy": (c_int, [c_void_p, c_void_p, c_size_t, c_int]),
    "grxMemcpyAsync": (c_int, [c_void_p, c_void_p, c_size_t, c_int, c_void_p]),
    "grxMemset": (c_int, [c_void_p, c_int, c_size_t]),
    "grxMemsetAsync": (c_int, [c_void_p, c_int, c_size_t, c_void_p]),
    "grxStreamCreate": (c_int, [POINTER(c_void_p)]),
    "grxStreamCreateWithFlags": (c_int, [POINTER(c_void_p), c_uint]),
    "grxStreamDestroy": (c_int, [c_void_p]),
    "grxStreamSynchronize": (c_int, [c_void_p]),
    "grxStreamQuery": (c_int, [c_void_p]),
    "grxStreamWaitEvent": (c_int, [c_void_p, c_void_p, c_uint]),
    "grxEventCreate": (c_int, [POINTER(c_void_p)]),
    "grxEventCreateWithFlags": (c_int, [POINTER(c_void_p), c_uint]),
    "grxEventDestroy": (c_int, [c_void_p]),
    "grxEventRecord": (c_int, [c_void_p, c_void_p]),
    "grxEventSynchronize": (c_int, [c_void_p]),
    "grxEventQuery": (c_int, [c_void_p]),
    "grxEventElapsedTime": (c_int, [POINTER(c_float), c_void_p, c_void_p]),
}
_FP = POINTER(c_float)
_BLAS = {
    "grxblasGetStatusString": (c_char_p, [c_int]),
    "grxblasCreate": (c_int, [POINTER(c_void_p)]),
    "grxblasDestroy": (c_int, [c_void_p]),
    "grxblasSetStream": (c_int, [c_void_p, c_void_p]),
    "grxblasGetStream": (c_int, [c_void_p, POINTER(c_void_p)]),
    "grxblasGemmEx": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, _FP,
                              c_void_p, c_int, c_int, c_void_p, c_int, c_int, _FP,
                              c_void_p, c_int, c_int]),
    "grxblasGemmExNoAlloc": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, _FP,
                                     c_void_p, c_int, c_int, c_void_p, c_int, c_int, _FP,
                                     c_void_p, c_int, c_int]),
    "grxblasGemmStridedBatchedEx": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, _FP,
                                            c_void_p, c_int, c_int, c_longlong, c_void_p, c_int,
                                            c_int, c_longlong, _FP, c_void_p, c_int, c_int,
                                            c_longlong, c_int]),
    "grxblasGemmExDequant": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int,
                                     c_void_p, c_int, c_int, c_void_p, c_int, c_int,
                                     c_void_p, c_void_p, c_int, c_int]),
    "grxblasGetTensorTypes": (c_int, [c_void_p, POINTER(c_uint)]),
    "grxblasSetTensorMapSlots": (c_int, [c_void_p, c_int, c_int]),
    "grxblasGetTensorTile": (c_int, [c_void_p, POINTER(c_int), POINTER(c_int), POINTER(c_int)]),
    "grxblasSaxpy": (c_int, [c_void_p, c_int, _FP, c_void_p, c_int, c_void_p, c_int]),
    "grxblasSscal": (c_int, [c_void_p, c_int, _FP, c_void_p, c_int]),
    "grxblasSgemv": (c_int, [c_void_p, c_int, c_int, c_int, _FP, c_void_p, c_int, c_void_p,
                             c_int, _FP, c_void_p, c_int]),
    "grxblasSgemm": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, _FP, c_void_p,
                             c_int, c_void_p, c_int, _FP, c_void_p, c_int]),
    "grxblasSgemmStridedBatched": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, _FP,
                                           c_void_p, c_int, c_longlong, c_void_p, c_int,
                                           c_longlong, _FP, c_void_p, c_int, c_longlong, c_int]),
    "grxblasSetKernelPath": (c_int, [c_char_p]),
    "grxblasSetCycleProbe": (c_int, [c_void_p, c_void_p, c_int]),
    "grxblasCycleSlotsNeeded": (c_int, [c_void_p, c_int, c_int]),
    "grxblasGetLoadedKernelPath": (c_int, [c_void_p, POINTER(c_char_p)]),
}
_IP = POINTER(c_int)
_DNN = {
    "grxdnnGetStatusString": (c_char_p, [c_int]),
    "grxdnnCreate": (c_int, [POINTER(c_void_p)]),
    "grxdnnDestroy": (c_int, [c_void_p]),
    "grxdnnSetStream": (c_int, [c_void_p, c_void_p]),
    "grxdnnGetStream": (c_int, [c_void_p, POINTER(c_void_p)]),
    "grxdnnCreateTensorDescriptor": (c_int, [POINTER(c_void_p)]),
    "grxdnnDestroyTensorDescriptor": (c_int, [c_void_p]),
    "grxdnnSetTensorNdDescriptor": (c_int, [c_void_p, c_int, c_int, _IP, _IP]),
    "grxdnnGetTensorNdDescriptor": (c_int, [c_void_p, c_int, _IP, _IP, _IP, _IP]),
    "grxdnnRMSNormForward": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float,
                                     c_void_p, c_void_p]),
    "grxdnnLayerNormForward": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_float, c_void_p, c_void_p]),
    "grxdnnSoftmaxForward": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "grxdnnGeluForward": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "grxdnnCreateAttentionDescriptor": (c_int, [POINTER(c_void_p)]),
    "grxdnnDestroyAttentionDescriptor": (c_int, [c_void_p]),
    "grxdnnSetAttentionDescriptor": (c_int, [c_void_p, c_int, c_float]),
    "grxdnnGetAttentionDescriptor": (c_int, [c_void_p, _IP, _FP]),
    "grxdnnAttentionForward": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "grxdnnSetCycleProbe": (c_int, [c_void_p, c_void_p, c_int]),
    "grxdnnAttentionCycleSlotsNeeded": (c_int, [c_void_p, c_int, c_int, c_int]),
}
EXPORTS = {"libgrxrt.so": _RT, "libgrxblas.so": _BLAS, "libgrxdnn.so": _DNN}


class Libs:
    def __init__(self, rt, blas, dnn):
        self.rt, self.blas, self.dnn = rt, blas, dnn


def lib_paths() -> dict:
    return {name: os.path.join(LIBDIR, name) for name in EXPORTS}


def load() -> Libs:
    """Load the in-tree libraries (no fallback: raises if any is missing)."""
    global _libs
    if _libs is not None:
        return _libs
    handles = {}
    for name, table in EXPORTS.items():
        path = os.path.join(LIBDIR, name)
        if not os.path.exists(path):
            raise GrxError(f"{path} is missing: build it with `python -m grxcp_amd.build`")
        L = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        for fn, (res, args) in table.items():
            f = getattr(L, fn)
            f.restype = res
            f.argtypes = args
        handles[name] = L
    _libs = Libs(handles["libgrxrt.so"], handles["libgrxblas.so"], handles["libgrxdnn.so"])
    return _libs


def check(status: int, what: str = "") -> None:
    if status != SUCCESS:
        raise GrxError(f"{what}: status {status} ({STATUS.get(status, '?')})")


def check_rt(err: int, what: str = "") -> None:
    if err != 0:
        name = load().rt.grxGetErrorName(err).decode()
        raise GrxError(f"{what}: {name}")


def device_count() -> int:
    n = c_int(0)
    load().rt.grxGetDeviceCount(ctypes.byref(n))
    return n.value


# ---- device memory ---------------------------------------------------------

class DeviceBuffer:
    """A grxMalloc'd region. Freed on close()/garbage collection."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = c_void_p()
        check_rt(load().rt.grxMalloc(ctypes.byref(self.ptr), max(1, self.nbytes)), "grxMalloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes:
            assert offset + a.nbytes <= self.nbytes
            check_rt(load().rt.grxMemcpy(c_void_p(self.ptr.value + offset), a.ctypes.data_as(c_void_p),
                                         a.nbytes, MEMCPY_DEFAULT), "upload")

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        if out.nbytes:
            check_rt(load().rt.grxMemcpy(out.ctypes.data_as(c_void_p), c_void_p(self.ptr.value + offset),
                                         out.nbytes, MEMCPY_DEFAULT), "download")
        return out

    def memset(self, value: int) -> None:
        check_rt(load().rt.grxMemset(self.ptr, value, self.nbytes), "memset")

    def close(self) -> None:
        if self.ptr is not None and self.ptr.value:
            load().rt.grxFree(self.ptr)
        self.ptr = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def p(self) -> c_void_p:
        return self.ptr


def synchronize() -> None:
    check_rt(load().rt.grxDeviceSynchronize(), "grxDeviceSynchronize")


def fptr(v: float):
    return ctypes.pointer(c_float(v))


# ---- handles ----------------------------------------------------------------

class Blas:
    def __init__(self):
        self.L = load().blas
        self.h = c_void_p()
        check(self.L.grxblasCreate(ctypes.byref(self.h)), "grxblasCreate")

    def close(self):
        if self.h:
            self.L.grxblasDestroy(self.h)
            self.h = c_void_p()

    def set_stream(self, s) -> None:
        check(self.L.grxblasSetStream(self.h, s), "grxblasSetStream")

    def gemm_ex(self, ta, tb, m, n, k, alpha, A, atype, lda, B, btype, ldb, beta, C, ctype, ldc) -> int:
        return self.L.grxblasGemmEx(self.h, int(ta), int(tb), m, n, k, fptr(alpha), A, atype, lda,
                                    B, btype, ldb, fptr(beta), C, ctype, ldc)

    def gemm_ex_noalloc(self, ta, tb, m, n, k, alpha, A, atype, lda, B, btype, ldb, beta, C, ctype,
                        ldc) -> int:
        return self.L.grxblasGemmExNoAlloc(self.h, int(ta), int(tb), m, n, k, fptr(alpha), A, atype,
                                           lda, B, btype, ldb, fptr(beta), C, ctype, ldc)

    def gemm_strided_batched_ex(self, ta, tb, m, n, k, alpha, A, atype, lda, sa, B, btype, ldb, sb,
                                beta, C, ctype, ldc, sc, batch) -> int:
        return self.L.grxblasGemmStridedBatchedEx(self.h, int(ta), int(tb), m, n, k, fptr(alpha), A,
                                                  atype, lda, sa, B, btype, ldb, sb, fptr(beta), C,
                                                  ctype, ldc, sc, batch)

    def gemm_ex_dequant(self, ta, tb, m, n, k, A, atype, lda, B, btype, ldb, scale, C, ctype, ldc) -> int:
        return self.L.grxblasGemmExDequant(self.h, int(ta), int(tb), m, n, k, A, atype, lda, B, btype,
                                           ldb, scale, C, ctype, ldc)

    def sgemm(self, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc) -> int:
        return self.L.grxblasSgemm(self.h, int(ta), int(tb), m, n, k, fptr(alpha), A, lda, B, ldb,
                                   fptr(beta), C, ldc)

    def set_cycle_probe(self, slots, capacity: int) -> int:
        """Attach (or with slots=None detach) a device array of CycleSlot."""
        return self.L.grxblasSetCycleProbe(self.h, slots, capacity)

    def cycle_slots_needed(self, m: int, n: int) -> int:
        return self.L.grxblasCycleSlotsNeeded(self.h, m, n)

    def sgemm_strided_batched(self, ta, tb, m, n, k, alpha, A, lda, sa, B, ldb, sb, beta, C, ldc, sc,
                              batch) -> int:
        return self.L.grxblasSgemmStridedBatched(self.h, int(ta), int(tb), m, n, k, fptr(alpha), A, lda,
                                                 sa, B, ldb, sb, fptr(beta), C, ldc, sc, batch)


class TensorDesc:
    def __init__(self, dtype: int, dims, strides=None):
        self.L = load().dnn
        self.d = c_void_p()
        check(self.L.grxdnnCreateTensorDescriptor(ctypes.byref(self.d)), "create desc")
        dims_a = (c_int * len(dims))(*dims)
        st = None if strides is None else (c_int * len(strides))(*strides)
        check(self.L.grxdnnSetTensorNdDescriptor(self.d, dtype, len(dims), dims_a, st), "set desc")

    def close(self):
        if self.d:
            self.L.grxdnnDestroyTensorDescriptor(self.d)
            self.d = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class AttnDesc:
    def __init__(self, causal: bool, scale: float):
        self.L = load().dnn
        self.d = c_void_p()
        check(self.L.grxdnnCreateAttentionDescriptor(ctypes.byref(self.d)), "create attn desc")
        check(self.L.grxdnnSetAttentionDescriptor(self.d, int(bool(causal)), scale), "set attn desc")

    def close(self):
        if self.d:
            self.L.grxdnnDestroyAttentionDescriptor(self.d)
            self.d = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Dnn:
    def __init__(self):
        self.L = load().dnn
        self.h = c_void_p()
        check(self.L.grxdnnCreate(ctypes.byref(self.h)), "grxdnnCreate")

    def close(self):
        if self.h:
            self.L.grxdnnDestroy(self.h)
            self.h = c_void_p()

    def set_stream(self, s) -> None:
        check(self.L.grxdnnSetStream(self.h, s), "grxdnnSetStream")

    def rmsnorm(self, xd, x, wd, g, eps, yd, y) -> int:
        return self.L.grxdnnRMSNormForward(self.h, xd.d, x, wd.d, g, eps, yd.d, y)

    def layernorm(self, xd, x, wd, g, b, eps, yd, y) -> int:
        return self.L.grxdnnLayerNormForward(self.h, xd.d, x, wd.d, g, b, eps, yd.d, y)

    def attention(self, ad, qd, q, kd, k, vd, v, od, o) -> int:
        return self.L.grxdnnAttentionForward(self.h, ad.d, qd.d, q, kd.d, k, vd.d, v, od.d, o)

    def set_cycle_probe(self, slots, capacity: int) -> int:
        """Attach (or with slots=None detach) a device array of CycleSlot
        for the attention calls."""
        return self.L.grxdnnSetCycleProbe(self.h, slots, capacity)

    def attention_cycle_slots_needed(self, batch: int, heads: int, seq: int) -> int:
        return self.L.grxdnnAttentionCycleSlotsNeeded(self.h, batch, heads, seq)

    def softmax(self, xd, x, yd, y) -> int:
        return self.L.grxdnnSoftmaxForward(self.h, xd.d, x, yd.d, y)

    def gelu(self, mode: int, xd, x, yd, y) -> int:
        return self.L.grxdnnGeluForward(self.h, mode, xd.d, x, yd.d, y)


class Stream:
    def __init__(self):
        self.rt = load().rt
        self.s = c_void_p()
        check_rt(self.rt.grxStreamCreate(ctypes.byref(self.s)), "grxStreamCreate")

    def sync(self):
        check_rt(self.rt.grxStreamSynchronize(self.s), "grxStreamSynchronize")

    def close(self):
        if self.s:
            self.rt.grxStreamDestroy(self.s)
            self.s = c_void_p()


class Event:
    def __init__(self):
        self.rt = load().rt
        self.e = c_void_p()
        check_rt(self.rt.grxEventCreate(ctypes.byref(self.e)), "grxEventCreate")

    def record(self, stream) -> None:
        check_rt(self.rt.grxEventRecord(self.e, stream), "grxEventRecord")

    def elapsed_ms(self, later: "Event") -> float:
        ms = c_float(0)
        check_rt(self.rt.grxEventSynchronize(later.e), "grxEventSynchronize")
        check_rt(self.rt.grxEventElapsedTime(ctypes.byref(ms), self.e, later.e), "grxEventElapsedTime")
        return ms.value

    def close(self):
        if self.e:
            self.rt.grxEventDestroy(self.e)
            self.e = c_void_p()
