/* grxblas.h -- grxBLAS dense linear algebra, MI355X (gfx950) build.
 *
 * Drop-in replacement for the reference's public header
 * (ref: include/grx/grxblas.h). Every declaration the reference exports is
 * kept with the same name, signature, enumerator values and status semantics;
 * each one cites the reference line it replaces. The implementation behind
 * them is new: a C++ host library (libgrxblas.so) that validates arguments
 * exactly as the reference does and launches hand-written gfx950 kernels
 * (MFMA matrix cores for GemmEx, LDS-tiled FMA for Sgemm) on the handle's HIP
 * stream.
 *
 * Conventions, unchanged from the reference:
 *   - column major: element (i,j) of an m x n matrix with leading dimension
 *     ld sits at [i + j*ld];  C = alpha * op(A) * op(B) + beta * C;
 *   - leading dimensions bound op()'s STORAGE: a transposed A is stored k x m,
 *     so lda >= k;
 *   - matrix pointers are device addresses, alpha/beta are host pointers;
 *   - calls are asynchronous on the handle's stream; beta == 0 never reads C.
 *
 * Additions (absent from the reference, marked "new" below): the bfloat16
 * type (GRX_R_16BF, GRXBLAS_TENSOR_BF16), fp16/bf16 outputs for GemmEx, and
 * grxblasGemmExDequant (int8 GEMM with a per-output-channel fp32 scale and a
 * bf16 result).
 */
#ifndef GRXBLAS_H
#define GRXBLAS_H

#include "grx_cycles.h"
#include "grx_runtime.h"
#include "grx_types.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct grxblasContext* grxblasHandle_t;          /* ref grxblas.h:33 */

typedef enum {                                            /* ref grxblas.h:37-46 */
  GRXBLAS_STATUS_SUCCESS          = 0,
  GRXBLAS_STATUS_NOT_INITIALIZED  = 1,
  GRXBLAS_STATUS_ALLOC_FAILED     = 2,
  GRXBLAS_STATUS_INVALID_VALUE    = 3,
  GRXBLAS_STATUS_ARCH_MISMATCH    = 4,
  GRXBLAS_STATUS_EXECUTION_FAILED = 5,
  GRXBLAS_STATUS_NOT_SUPPORTED    = 6,
  GRXBLAS_STATUS_INTERNAL_ERROR   = 7
} grxblasStatus_t;

typedef enum {                                            /* ref grxblas.h:48-51 */
  GRXBLAS_OP_N = 0,
  GRXBLAS_OP_T = 1
} grxblasOperation_t;

/* ref grxblas.h:53 */
const char* grxblasGetStatusString(grxblasStatus_t s);

/* Handle lifecycle (ref grxblas.h:55-58). The handle is an opaque heap object
 * owned by the caller; the stream is borrowed and never destroyed here. A
 * null stream is the default stream. */
grxblasStatus_t grxblasCreate   (grxblasHandle_t* handle);
grxblasStatus_t grxblasDestroy  (grxblasHandle_t handle);
grxblasStatus_t grxblasSetStream(grxblasHandle_t handle, grxStream_t stream);
grxblasStatus_t grxblasGetStream(grxblasHandle_t handle, grxStream_t* stream);

/* Mixed-precision GEMM on the matrix cores (ref grxblas.h:97-105).
 *
 * Accepted type triples (Atype, Btype, Ctype):
 *   GRX_R_16F,  GRX_R_16F,  GRX_R_32F    fp16 in, fp32 accumulate and out
 *   GRX_R_16F,  GRX_R_16F,  GRX_R_16F    fp16 out (new)
 *   GRX_R_16BF, GRX_R_16BF, GRX_R_32F    bf16 in, fp32 accumulate and out (new)
 *   GRX_R_16BF, GRX_R_16BF, GRX_R_16BF   bf16 out, round-to-nearest-even (new)
 *   GRX_R_8I,   GRX_R_8I,   GRX_R_32I    int8 in, int32 accumulate and out
 * Anything else returns GRXBLAS_STATUS_NOT_SUPPORTED (no scalar fallback).
 * For the int8 triple alpha and beta must hold integers exactly; they are
 * applied in int32 (two's complement wrap). A non-integral value returns
 * GRXBLAS_STATUS_INVALID_VALUE rather than being rounded.
 * All four transpose combinations, ragged shapes and padded leading
 * dimensions are supported. */
grxblasStatus_t grxblasGemmEx(grxblasHandle_t handle,
                              grxblasOperation_t transa,
                              grxblasOperation_t transb,
                              int m, int n, int k,
                              const float* alpha,
                              const void* A, grxDataType_t Atype, int lda,
                              const void* B, grxDataType_t Btype, int ldb,
                              const float* beta,
                              void* C, grxDataType_t Ctype, int ldc);

/* new: strided batch of GemmEx in one launch. No counterpart in the
 * reference header: it joins grxblasGemmEx's type triples, alpha/beta rules
 * and validation (ref grxblas.h:97-105, src/libs/grxblas/grxblas.cpp:507-584)
 * with grxblasSgemmStridedBatched's batch convention (ref grxblas.h:207-212):
 * batch b computes C + b*strideC from A + b*strideA and B + b*strideB;
 * strides are signed, in elements, and a zero stride broadcasts A or B.
 * batchCount == 0 is a successful no-op, a negative one INVALID_VALUE, more
 * than 65535 NOT_SUPPORTED. With a cycle probe attached, the capacity must
 * cover batchCount times the slots of one GemmEx of the same shape. */
grxblasStatus_t grxblasGemmStridedBatchedEx(grxblasHandle_t handle,
                                            grxblasOperation_t transa,
                                            grxblasOperation_t transb,
                                            int m, int n, int k,
                                            const float* alpha,
                                            const void* A, grxDataType_t Atype, int lda,
                                            long long strideA,
                                            const void* B, grxDataType_t Btype, int ldb,
                                            long long strideB,
                                            const float* beta,
                                            void* C, grxDataType_t Ctype, int ldc,
                                            long long strideC, int batchCount);

/* new: grxblasGemmEx that allocates nothing. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, type triples, validation, status codes and results as
 * grxblasGemmEx; where grxblasGemmEx would place transposed operand copies
 * or split-K partials in a workspace the handle allocates, this call uses a
 * static __device__ array of 64 MiB per device. The array is loaded onto a
 * device by the first call of this function there (which also creates one
 * event per device; make that first call outside graph capture), and the
 * device then holds it until the process ends; processes that never call
 * this function do not hold it. A problem that needs more scratch than that
 * returns GRXBLAS_STATUS_NOT_SUPPORTED (with a one-line message) and
 * launches nothing. Every call on one device shares that device's array:
 * a call on another stream than the previous scratch user's waits, on the
 * GPU, for that user's launch (hipStreamWaitEvent), so calls from several
 * streams, handles or threads take turns. Under HIP graph capture that wait
 * is left out: a captured call is ordered only by its graph and stream. */
grxblasStatus_t grxblasGemmExNoAlloc(grxblasHandle_t handle,
                                     grxblasOperation_t transa,
                                     grxblasOperation_t transb,
                                     int m, int n, int k,
                                     const float* alpha,
                                     const void* A, grxDataType_t Atype, int lda,
                                     const void* B, grxDataType_t Btype, int ldb,
                                     const float* beta,
                                     void* C, grxDataType_t Ctype, int ldc);

/* new: int8 GEMM with per-output-channel dequantisation.
 *
 *   acc[i,j] = sum_l op(A)[i,l] * op(B)[l,j]                 (exact, int32)
 *   C[i,j]   = bf16_rne( f32_rne( f32_rne((float)acc[i,j]) * scaleN[j] ) )
 *
 * A, B are GRX_R_8I; C is GRX_R_16BF, column major with ldc >= m; scaleN is a
 * DEVICE array of n fp32 scales, one per output column (output channel).
 * Validation order and status codes follow grxblasGemmEx; a null scaleN is
 * INVALID_VALUE; any other type triple is NOT_SUPPORTED. k == 0 writes
 * bf16(0 * scale). No counterpart in the reference (its int8 path ends at int32
 * C, ref src/libs/grxblas/grxblas.cpp:580-584). */
grxblasStatus_t grxblasGemmExDequant(grxblasHandle_t handle,
                                     grxblasOperation_t transa,
                                     grxblasOperation_t transb,
                                     int m, int n, int k,
                                     const void* A, grxDataType_t Atype, int lda,
                                     const void* B, grxDataType_t Btype, int ldb,
                                     const float* scaleN,
                                     void* C, grxDataType_t Ctype, int ldc);

/* ref grxblas.h:118-125; GRXBLAS_TENSOR_BF16 is new. */
typedef enum {
  GRXBLAS_TENSOR_FP16 = 0x01,
  GRXBLAS_TENSOR_TF32 = 0x02,
  GRXBLAS_TENSOR_FP8  = 0x04,
  GRXBLAS_TENSOR_FP4  = 0x08,
  GRXBLAS_TENSOR_INT8 = 0x10,
  GRXBLAS_TENSOR_INT4 = 0x20,
  GRXBLAS_TENSOR_BF16 = 0x40
} grxblasTensorType_t;

/* The input types GemmEx accepts on this device, as GRXBLAS_TENSOR_* bits
 * (ref grxblas.h:130-131). On gfx950: FP16 | BF16 | INT8. A device other than
 * gfx950 returns ARCH_MISMATCH: the library carries gfx950 code only. */
grxblasStatus_t grxblasGetTensorTypes(grxblasHandle_t handle,
                                      unsigned* typeMask);

/* ref grxblas.h:134-135. gfx950 has no descriptor slots: the call validates
 * its arguments (non-negative, distinct) and records them, nothing more. */
grxblasStatus_t grxblasSetTensorMapSlots(grxblasHandle_t handle,
                                         int slotA, int slotB);

/* The matrix-core tile one wavefront computes per instruction on GemmEx's
 * general path, which small problems that are unaligned or in layouts other
 * than (T,N) take (ref grxblas.h:142-143): 32 x 32 x 16 for fp16/bf16
 * (v_mfma_f32_32x32x16_*; int8 32 x 32 x 32). Aligned (T,N) problems, and
 * larger ones behind operand copies, run 16 x 16 x 32
 * instructions (int8 16 x 16 x 64): eight by eight per wavefront on 256 x
 * 256 tiles, four by four on 128 x 128 tiles. */
grxblasStatus_t grxblasGetTensorTile(grxblasHandle_t handle,
                                     int* m, int* n, int* k);

/* Level 1 and 2 (ref grxblas.h:164-183). Memory bound, fp32, BLAS increment
 * rules (negative walks backwards, zero refused, sscal needs incx > 0). */
grxblasStatus_t grxblasSaxpy(grxblasHandle_t handle, int n, const float* alpha,
                             const float* x, int incx, float* y, int incy);
grxblasStatus_t grxblasSscal(grxblasHandle_t handle, int n, const float* alpha,
                             float* x, int incx);
grxblasStatus_t grxblasSgemv(grxblasHandle_t handle, grxblasOperation_t trans,
                             int m, int n, const float* alpha,
                             const void* A, int lda,
                             const void* x, int incx,
                             const float* beta,
                             void* y, int incy);

/* Single-precision GEMM (ref grxblas.h:187-195). */
grxblasStatus_t grxblasSgemm(grxblasHandle_t handle,
                             grxblasOperation_t transa,
                             grxblasOperation_t transb,
                             int m, int n, int k,
                             const float* alpha,
                             const void* A, int lda,
                             const void* B, int ldb,
                             const float* beta,
                             void* C, int ldc);

/* Strided batch of Sgemm in one launch (ref grxblas.h:207-212). Strides are
 * signed, in elements; a zero stride broadcasts A or B. */
grxblasStatus_t grxblasSgemmStridedBatched(
    grxblasHandle_t handle, grxblasOperation_t transa,
    grxblasOperation_t transb, int m, int n, int k, const float* alpha,
    const void* A, int lda, long long strideA,
    const void* B, int ldb, long long strideB,
    const float* beta, void* C, int ldc, long long strideC, int batchCount);

/* Where the kernels come from (ref grxblas.h:227). On this build the gfx950
 * code objects are linked into libgrxblas.so itself. A configured directory
 * (this call, else $GRXBLAS_KERNEL_PATH) must be the directory that holds the
 * loaded libgrxblas.so; otherwise the first kernel call fails with
 * NOT_INITIALIZED and a one-line hint, mirroring the reference's "no fallback
 * past a configured source". NULL or "" clears the setting. */
grxblasStatus_t grxblasSetKernelPath(const char* path);

/* Per-wave cycle records (ref grxblas.h:240-242). With a slot array attached,
 * the next Sgemm/GemmEx calls record one grxCycleSlot per wave. capacity must
 * cover grxblasCycleSlotsNeeded for the call. NULL turns recording off. */
grxblasStatus_t grxblasSetCycleProbe(grxblasHandle_t handle,
                                     grxCycleSlot* slots, int capacity);
int             grxblasCycleSlotsNeeded(grxblasHandle_t handle, int m, int n);

/* The file the kernels were loaded from (libgrxblas.so), or NULL before the
 * first kernel call (ref grxblas.h:247-248). */
grxblasStatus_t grxblasGetLoadedKernelPath(grxblasHandle_t handle,
                                           const char** path);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* GRXBLAS_H */
