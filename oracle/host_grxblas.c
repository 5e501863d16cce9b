/* host_grxblas.c -- grxBLAS on the host CPU, behind the same grxblas.h ABI.
 *
 * TEST INFRASTRUCTURE / CPU HOST BACKEND. Built into oracle/libgrxblas_ref.so
 * (with the oracle's restatements linked in) and paired with
 * oracle/libgrxrt_ref.so. This is the "host/mock reference backend on CPU"
 * that BASELINE config 1 (fp32 SGEMM 512^3) runs on: a separate link target
 * exporting the grxblas.h symbols, chosen at link time (no run-time dispatch).
 * The product libraries never load it, and bench.py's timed region never
 * calls it.
 *
 * Arithmetic is the oracle's restatement of the reference's CPU references:
 *   Sgemm        oracle_sgemm, fp64 accumulate (ref tests/libs/test_grxblas.cpp:62-80)
 *   GemmEx f16   oracle_gemm_f32acc, fp32 accumulate in k order
 *                (ref tests/libs/test_grxblas_ex.cpp:45-63); bf16 the same
 *   GemmEx int8  oracle_igemm, int32 with wrap (ref test_grxblas_ex.cpp:267-281)
 *   Dequant      oracle_igemm + oracle_dequant
 * Argument validation follows the order and status codes of the reference's
 * library (ref src/libs/grxblas/grxblas.cpp:507-584 for GemmEx, :882-897 for
 * Sgemm, :736-865 for level 1/2), which the GPU library keeps too.
 * "Device" pointers are host pointers (libgrxrt_ref's grxMalloc is malloc);
 * every call completes before it returns.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "grx/grxblas.h"
#include "grx_oracle.h"

#define EXPORT __attribute__((visibility("default")))

struct grxblasContext {
  grxStream_t stream;
  int slot_a, slot_b;
};

static const char kPath[] = "(host CPU backend: no device kernels)";

static int integral(float v) {
  return isfinite(v) && v >= -2147483648.0f && v < 2147483648.0f && v == (float)(int32_t)v;
}

/* Elements a column-major rows x cols operand occupies with leading dim ld. */
static size_t extent(int rows, int cols, int ld) {
  if (rows <= 0 || cols <= 0) return 0;
  return (size_t)ld * (size_t)(cols - 1) + (size_t)rows;
}

EXPORT const char* grxblasGetStatusString(grxblasStatus_t s) {
  switch (s) {
    case GRXBLAS_STATUS_SUCCESS: return "success";
    case GRXBLAS_STATUS_NOT_INITIALIZED: return "library not initialized";
    case GRXBLAS_STATUS_ALLOC_FAILED: return "allocation failed";
    case GRXBLAS_STATUS_INVALID_VALUE: return "invalid argument";
    case GRXBLAS_STATUS_ARCH_MISMATCH: return "device lacks a required capability";
    case GRXBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
    case GRXBLAS_STATUS_NOT_SUPPORTED: return "not supported";
    case GRXBLAS_STATUS_INTERNAL_ERROR: return "internal error";
  }
  return "unknown status";
}

EXPORT grxblasStatus_t grxblasCreate(grxblasHandle_t* handle) {
  if (!handle) return GRXBLAS_STATUS_INVALID_VALUE;
  *handle = (grxblasHandle_t)calloc(1, sizeof(struct grxblasContext));
  return *handle ? GRXBLAS_STATUS_SUCCESS : GRXBLAS_STATUS_ALLOC_FAILED;
}
EXPORT grxblasStatus_t grxblasDestroy(grxblasHandle_t handle) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  free(handle);
  return GRXBLAS_STATUS_SUCCESS;
}
EXPORT grxblasStatus_t grxblasSetStream(grxblasHandle_t handle, grxStream_t stream) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  handle->stream = stream;
  return GRXBLAS_STATUS_SUCCESS;
}
EXPORT grxblasStatus_t grxblasGetStream(grxblasHandle_t handle, grxStream_t* stream) {
  if (!handle || !stream) return GRXBLAS_STATUS_INVALID_VALUE;
  *stream = handle->stream;
  return GRXBLAS_STATUS_SUCCESS;
}
EXPORT grxblasStatus_t grxblasSetKernelPath(const char* path) {
  (void)path;
  return GRXBLAS_STATUS_SUCCESS;
}
EXPORT grxblasStatus_t grxblasGetLoadedKernelPath(grxblasHandle_t handle, const char** path) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!path) return GRXBLAS_STATUS_INVALID_VALUE;
  *path = kPath;
  return GRXBLAS_STATUS_SUCCESS;
}
EXPORT grxblasStatus_t grxblasSetTensorMapSlots(grxblasHandle_t handle, int slotA, int slotB) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (slotA < 0 || slotB < 0 || slotA == slotB) return GRXBLAS_STATUS_INVALID_VALUE;
  handle->slot_a = slotA;
  handle->slot_b = slotB;
  return GRXBLAS_STATUS_SUCCESS;
}
EXPORT grxblasStatus_t grxblasGetTensorTypes(grxblasHandle_t handle, unsigned* typeMask) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!typeMask) return GRXBLAS_STATUS_INVALID_VALUE;
  *typeMask = GRXBLAS_TENSOR_FP16 | GRXBLAS_TENSOR_BF16 | GRXBLAS_TENSOR_INT8;
  return GRXBLAS_STATUS_SUCCESS;
}
/* The GPU library's instruction tile, so that a gate sized from this query
 * runs the same shapes on both backends. */
EXPORT grxblasStatus_t grxblasGetTensorTile(grxblasHandle_t handle, int* m, int* n, int* k) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!m || !n || !k) return GRXBLAS_STATUS_INVALID_VALUE;
  *m = 32;
  *n = 32;
  *k = 16;
  return GRXBLAS_STATUS_SUCCESS;
}
/* No waves to time on the host. */
EXPORT grxblasStatus_t grxblasSetCycleProbe(grxblasHandle_t handle, grxCycleSlot* slots,
                                            int capacity) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (slots && capacity <= 0) return GRXBLAS_STATUS_INVALID_VALUE;
  return slots ? GRXBLAS_STATUS_NOT_SUPPORTED : GRXBLAS_STATUS_SUCCESS;
}
EXPORT int grxblasCycleSlotsNeeded(grxblasHandle_t handle, int m, int n) {
  (void)handle;
  (void)m;
  (void)n;
  return 0;
}

/* ---- GEMM ------------------------------------------------------------------ */

enum In { IN_F16, IN_BF16, IN_I8 };
enum Out { OUT_F32, OUT_F16, OUT_BF16, OUT_I32, OUT_DEQ };

static void widen16(const uint16_t* src, float* dst, size_t n, int bf16) {
  if (bf16) oracle_bf16_to_f32_array(src, dst, n);
  else oracle_half_to_f32_array(src, dst, n);
}

/* One GemmEx problem of a batch. Returns 0, or -1 when out of memory. */
static int gemm_one(enum In in, enum Out out, int ta, int tb, int m, int n, int k, float alpha,
                    const void* A, int lda, const void* B, int ldb, float beta, void* C, int ldc,
                    const float* scale) {
  const int a_rows = ta ? k : m, a_cols = ta ? m : k;
  const int b_rows = tb ? n : k, b_cols = tb ? k : n;
  const size_t na = extent(a_rows, a_cols, lda), nb = extent(b_rows, b_cols, ldb);
  const size_t nc = extent(m, n, ldc);
  if (in == IN_I8) {
    int32_t* acc = (out == OUT_DEQ) ? (int32_t*)calloc(nc ? nc : 1, sizeof(int32_t))
                                    : (int32_t*)C;
    if (!acc) return -1;
    oracle_igemm(ta, tb, m, n, k, out == OUT_DEQ ? 1 : (int32_t)alpha, (const int8_t*)A, lda,
                 (const int8_t*)B, ldb, out == OUT_DEQ ? 0 : (int32_t)beta, acc, ldc);
    if (out == OUT_DEQ) {
      oracle_dequant(m, n, acc, ldc, scale, (uint16_t*)C, ldc);
      free(acc);
    }
    return 0;
  }
  const int bf = (in == IN_BF16);
  float* a = (float*)malloc((na ? na : 1) * sizeof(float));
  float* b = (float*)malloc((nb ? nb : 1) * sizeof(float));
  float* c = (out == OUT_F32) ? (float*)C : (float*)malloc((nc ? nc : 1) * sizeof(float));
  if (!a || !b || !c) {
    free(a);
    free(b);
    if (out != OUT_F32) free(c);
    return -1;
  }
  if (na) widen16((const uint16_t*)A, a, na, bf);
  if (nb) widen16((const uint16_t*)B, b, nb, bf);
  if (out != OUT_F32) widen16((const uint16_t*)C, c, nc, out == OUT_BF16);
  oracle_gemm_f32acc(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc);
  if (out != OUT_F32) {
    /* narrow the m x n window only: the padding between columns stays as it was */
    uint16_t* c16 = (uint16_t*)C;
    for (int j = 0; j < n; ++j)
      for (int i = 0; i < m; ++i) {
        const size_t ci = (size_t)i + (size_t)j * (size_t)ldc;
        c16[ci] = (out == OUT_BF16) ? oracle_float_to_bf16(c[ci]) : oracle_float_to_half(c[ci]);
      }
    free(c);
  }
  free(a);
  free(b);
  return 0;
}

static grxblasStatus_t gemm_ex_batched(grxblasHandle_t handle, grxblasOperation_t transa,
                                       grxblasOperation_t transb, int m, int n, int k,
                                       const float* alpha, const void* A, grxDataType_t Atype,
                                       int lda, long long strideA, const void* B,
                                       grxDataType_t Btype, int ldb, long long strideB,
                                       const float* beta, void* C, grxDataType_t Ctype, int ldc,
                                       long long strideC, int batch) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha || !beta) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m < 0 || n < 0 || k < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (batch < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m == 0 || n == 0 || batch == 0) return GRXBLAS_STATUS_SUCCESS;
  if (k > 0 && (!A || !B)) return GRXBLAS_STATUS_INVALID_VALUE;
  if (!C) return GRXBLAS_STATUS_INVALID_VALUE;
  const int ta = (transa == GRXBLAS_OP_T), tb = (transb == GRXBLAS_OP_T);
  if (lda < (ta ? k : m) || ldb < (tb ? n : k) || ldc < m) return GRXBLAS_STATUS_INVALID_VALUE;
  if (batch > 65535) return GRXBLAS_STATUS_NOT_SUPPORTED;

  enum In in;
  enum Out out;
  size_t ea, ec;
  if (Atype == GRX_R_16F && Btype == GRX_R_16F && Ctype == GRX_R_32F) {
    in = IN_F16; out = OUT_F32; ea = 2; ec = 4;
  } else if (Atype == GRX_R_16F && Btype == GRX_R_16F && Ctype == GRX_R_16F) {
    in = IN_F16; out = OUT_F16; ea = 2; ec = 2;
  } else if (Atype == GRX_R_16BF && Btype == GRX_R_16BF && Ctype == GRX_R_32F) {
    in = IN_BF16; out = OUT_F32; ea = 2; ec = 4;
  } else if (Atype == GRX_R_16BF && Btype == GRX_R_16BF && Ctype == GRX_R_16BF) {
    in = IN_BF16; out = OUT_BF16; ea = 2; ec = 2;
  } else if (Atype == GRX_R_8I && Btype == GRX_R_8I && Ctype == GRX_R_32I) {
    in = IN_I8; out = OUT_I32; ea = 1; ec = 4;
  } else {
    return GRXBLAS_STATUS_NOT_SUPPORTED;
  }
  if (in == IN_I8 && (!integral(*alpha) || !integral(*beta))) return GRXBLAS_STATUS_INVALID_VALUE;

  for (int z = 0; z < batch; ++z) {
    const char* a = (const char*)A + (ptrdiff_t)(strideA * z) * (ptrdiff_t)ea;
    const char* b = (const char*)B + (ptrdiff_t)(strideB * z) * (ptrdiff_t)ea;
    char* c = (char*)C + (ptrdiff_t)(strideC * z) * (ptrdiff_t)ec;
    if (gemm_one(in, out, ta, tb, m, n, k, *alpha, a, lda, b, ldb, *beta, c, ldc, NULL) != 0)
      return GRXBLAS_STATUS_ALLOC_FAILED;
  }
  return GRXBLAS_STATUS_SUCCESS;
}

EXPORT grxblasStatus_t grxblasGemmEx(grxblasHandle_t handle, grxblasOperation_t transa,
                                     grxblasOperation_t transb, int m, int n, int k,
                                     const float* alpha, const void* A, grxDataType_t Atype,
                                     int lda, const void* B, grxDataType_t Btype, int ldb,
                                     const float* beta, void* C, grxDataType_t Ctype, int ldc) {
  return gemm_ex_batched(handle, transa, transb, m, n, k, alpha, A, Atype, lda, 0, B, Btype, ldb,
                         0, beta, C, Ctype, ldc, 0, 1);
}

/* The host backend never allocates device memory, so the allocation-free
 * form is GemmEx itself (its per-call host temporaries aside). */
EXPORT grxblasStatus_t grxblasGemmExNoAlloc(grxblasHandle_t handle, grxblasOperation_t transa,
                                            grxblasOperation_t transb, int m, int n, int k,
                                            const float* alpha, const void* A, grxDataType_t Atype,
                                            int lda, const void* B, grxDataType_t Btype, int ldb,
                                            const float* beta, void* C, grxDataType_t Ctype,
                                            int ldc) {
  return gemm_ex_batched(handle, transa, transb, m, n, k, alpha, A, Atype, lda, 0, B, Btype, ldb,
                         0, beta, C, Ctype, ldc, 0, 1);
}

EXPORT grxblasStatus_t grxblasGemmStridedBatchedEx(
    grxblasHandle_t handle, grxblasOperation_t transa, grxblasOperation_t transb, int m, int n,
    int k, const float* alpha, const void* A, grxDataType_t Atype, int lda, long long strideA,
    const void* B, grxDataType_t Btype, int ldb, long long strideB, const float* beta, void* C,
    grxDataType_t Ctype, int ldc, long long strideC, int batchCount) {
  return gemm_ex_batched(handle, transa, transb, m, n, k, alpha, A, Atype, lda, strideA, B, Btype,
                         ldb, strideB, beta, C, Ctype, ldc, strideC, batchCount);
}

EXPORT grxblasStatus_t grxblasGemmExDequant(grxblasHandle_t handle, grxblasOperation_t transa,
                                            grxblasOperation_t transb, int m, int n, int k,
                                            const void* A, grxDataType_t Atype, int lda,
                                            const void* B, grxDataType_t Btype, int ldb,
                                            const float* scaleN, void* C, grxDataType_t Ctype,
                                            int ldc) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (m < 0 || n < 0 || k < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m == 0 || n == 0) return GRXBLAS_STATUS_SUCCESS;
  if (k > 0 && (!A || !B)) return GRXBLAS_STATUS_INVALID_VALUE;
  if (!C || !scaleN) return GRXBLAS_STATUS_INVALID_VALUE;
  const int ta = (transa == GRXBLAS_OP_T), tb = (transb == GRXBLAS_OP_T);
  if (lda < (ta ? k : m) || ldb < (tb ? n : k) || ldc < m) return GRXBLAS_STATUS_INVALID_VALUE;
  if (!(Atype == GRX_R_8I && Btype == GRX_R_8I && Ctype == GRX_R_16BF))
    return GRXBLAS_STATUS_NOT_SUPPORTED;
  if (gemm_one(IN_I8, OUT_DEQ, ta, tb, m, n, k, 1.0f, A, lda, B, ldb, 0.0f, C, ldc, scaleN) != 0)
    return GRXBLAS_STATUS_ALLOC_FAILED;
  return GRXBLAS_STATUS_SUCCESS;
}

static grxblasStatus_t sgemm_batched(grxblasHandle_t handle, grxblasOperation_t transa,
                                     grxblasOperation_t transb, int m, int n, int k,
                                     const float* alpha, const void* A, int lda, long long strideA,
                                     const void* B, int ldb, long long strideB, const float* beta,
                                     void* C, int ldc, long long strideC, int batch) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha || !beta) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m < 0 || n < 0 || k < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (batch < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m == 0 || n == 0 || batch == 0) return GRXBLAS_STATUS_SUCCESS;
  if (k > 0 && (!A || !B)) return GRXBLAS_STATUS_INVALID_VALUE;
  if (!C) return GRXBLAS_STATUS_INVALID_VALUE;
  const int ta = (transa == GRXBLAS_OP_T), tb = (transb == GRXBLAS_OP_T);
  if (lda < (ta ? k : m) || ldb < (tb ? n : k) || ldc < m) return GRXBLAS_STATUS_INVALID_VALUE;
  if (batch > 65535) return GRXBLAS_STATUS_NOT_SUPPORTED;
  for (int z = 0; z < batch; ++z)
    oracle_sgemm(ta, tb, m, n, k, *alpha, (const float*)A + strideA * z, lda,
                 (const float*)B + strideB * z, ldb, *beta, (float*)C + strideC * z, ldc);
  return GRXBLAS_STATUS_SUCCESS;
}

EXPORT grxblasStatus_t grxblasSgemm(grxblasHandle_t handle, grxblasOperation_t transa,
                                    grxblasOperation_t transb, int m, int n, int k,
                                    const float* alpha, const void* A, int lda, const void* B,
                                    int ldb, const float* beta, void* C, int ldc) {
  return sgemm_batched(handle, transa, transb, m, n, k, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc,
                       0, 1);
}

EXPORT grxblasStatus_t grxblasSgemmStridedBatched(
    grxblasHandle_t handle, grxblasOperation_t transa, grxblasOperation_t transb, int m, int n,
    int k, const float* alpha, const void* A, int lda, long long strideA, const void* B, int ldb,
    long long strideB, const float* beta, void* C, int ldc, long long strideC, int batchCount) {
  return sgemm_batched(handle, transa, transb, m, n, k, alpha, A, lda, strideA, B, ldb, strideB,
                       beta, C, ldc, strideC, batchCount);
}

/* ---- level 1 / 2 (BLAS increment rules: a negative increment walks the
 * vector from its far end) ------------------------------------------------- */

static ptrdiff_t start_of(int len, int inc) {
  return inc < 0 ? (ptrdiff_t)(1 - len) * inc : 0;
}

EXPORT grxblasStatus_t grxblasSaxpy(grxblasHandle_t handle, int n, const float* alpha,
                                    const float* x, int incx, float* y, int incy) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha) return GRXBLAS_STATUS_INVALID_VALUE;
  if (n < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (n == 0) return GRXBLAS_STATUS_SUCCESS;
  if (!x || !y) return GRXBLAS_STATUS_INVALID_VALUE;
  if (incx == 0 || incy == 0) return GRXBLAS_STATUS_INVALID_VALUE;
  ptrdiff_t ix = start_of(n, incx), iy = start_of(n, incy);
  for (int i = 0; i < n; ++i, ix += incx, iy += incy) y[iy] = *alpha * x[ix] + y[iy];
  return GRXBLAS_STATUS_SUCCESS;
}

EXPORT grxblasStatus_t grxblasSscal(grxblasHandle_t handle, int n, const float* alpha, float* x,
                                    int incx) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha) return GRXBLAS_STATUS_INVALID_VALUE;
  if (n < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (n == 0) return GRXBLAS_STATUS_SUCCESS;
  if (!x) return GRXBLAS_STATUS_INVALID_VALUE;
  if (incx <= 0) return GRXBLAS_STATUS_INVALID_VALUE;
  for (int i = 0; i < n; ++i) x[(ptrdiff_t)i * incx] *= *alpha;
  return GRXBLAS_STATUS_SUCCESS;
}

EXPORT grxblasStatus_t grxblasSgemv(grxblasHandle_t handle, grxblasOperation_t trans, int m,
                                    int n, const float* alpha, const void* A, int lda,
                                    const void* x, int incx, const float* beta, void* y,
                                    int incy) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha || !beta) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m < 0 || n < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m == 0 || n == 0) return GRXBLAS_STATUS_SUCCESS;
  if (!A || !x || !y) return GRXBLAS_STATUS_INVALID_VALUE;
  if (incx == 0 || incy == 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (lda < m) return GRXBLAS_STATUS_INVALID_VALUE;
  const int t = (trans == GRXBLAS_OP_T);
  const int lx = t ? m : n, ly = t ? n : m;
  const float* a = (const float*)A;
  const float* xv = (const float*)x;
  float* yv = (float*)y;
  const ptrdiff_t x0 = start_of(lx, incx);
  ptrdiff_t iy = start_of(ly, incy);
  for (int r = 0; r < ly; ++r, iy += incy) {
    double acc = 0.0;
    ptrdiff_t ix = x0;
    for (int c = 0; c < lx; ++c, ix += incx) {
      const float av = t ? a[(size_t)c + (size_t)r * (size_t)lda] : a[(size_t)r + (size_t)c * (size_t)lda];
      acc += (double)av * (double)xv[ix];
    }
    /* beta == 0 never reads y (it may hold NaN) */
    yv[iy] = (*beta == 0.0f) ? (float)(*alpha * acc)
                             : (float)(*alpha * acc + (double)*beta * yv[iy]);
  }
  return GRXBLAS_STATUS_SUCCESS;
}
