/* grxdnn.h -- grxDNN forward primitives, MI355X (gfx950) build.
 *
 * The reference plans grxDNN but ships no code for it: a CMake slot
 * (ref: src/libs/CMakeLists.txt:12), an architecture entry naming grxdnn.h
 * (ref: docs/designs/grxcp_architecture.md:594, 640) and roadmap phase 6
 * (ref: docs/designs/grxcp_roadmap.md:864-877: "softmax, layernorm, ...,
 * attention; grxBLAS + custom kernels"). This header is therefore designed
 * new, in grxBLAS's style (ref: include/grx/grxblas.h): an opaque handle with
 * a borrowed stream, status codes with grxBLAS's values, device pointers for
 * tensors, host values for scalars, asynchronous calls, validation before any
 * device work and NOT_SUPPORTED instead of a silent fallback.
 *
 * Tensors are described cuDNN-style by an N-d descriptor (type, dims,
 * strides in elements). The innermost dimension must have stride 1.
 */
#ifndef GRXDNN_H
#define GRXDNN_H

#include "grx_cycles.h"
#include "grx_runtime.h"
#include "grx_types.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct grxdnnContext*          grxdnnHandle_t;
typedef struct grxdnnTensorStruct*     grxdnnTensorDescriptor_t;
typedef struct grxdnnAttentionStruct*  grxdnnAttentionDescriptor_t;

/* Same values as grxblasStatus_t (ref include/grx/grxblas.h:37-46). */
typedef enum {
  GRXDNN_STATUS_SUCCESS          = 0,
  GRXDNN_STATUS_NOT_INITIALIZED  = 1,
  GRXDNN_STATUS_ALLOC_FAILED     = 2,
  GRXDNN_STATUS_INVALID_VALUE    = 3,
  GRXDNN_STATUS_ARCH_MISMATCH    = 4,
  GRXDNN_STATUS_EXECUTION_FAILED = 5,
  GRXDNN_STATUS_NOT_SUPPORTED    = 6,
  GRXDNN_STATUS_INTERNAL_ERROR   = 7
} grxdnnStatus_t;

#define GRXDNN_DIM_MAX 8

const char* grxdnnGetStatusString(grxdnnStatus_t s);

grxdnnStatus_t grxdnnCreate   (grxdnnHandle_t* handle);
grxdnnStatus_t grxdnnDestroy  (grxdnnHandle_t handle);
grxdnnStatus_t grxdnnSetStream(grxdnnHandle_t handle, grxStream_t stream);
grxdnnStatus_t grxdnnGetStream(grxdnnHandle_t handle, grxStream_t* stream);

/* ---- tensor descriptors ------------------------------------------------- */
grxdnnStatus_t grxdnnCreateTensorDescriptor (grxdnnTensorDescriptor_t* desc);
grxdnnStatus_t grxdnnDestroyTensorDescriptor(grxdnnTensorDescriptor_t desc);
/* 1 <= nbDims <= GRXDNN_DIM_MAX; dims >= 0; strides >= 0 in elements.
 * strides may be NULL for a packed (row-major, last dimension contiguous)
 * layout. */
grxdnnStatus_t grxdnnSetTensorNdDescriptor(grxdnnTensorDescriptor_t desc,
                                           grxDataType_t dataType, int nbDims,
                                           const int dims[],
                                           const int strides[]);
grxdnnStatus_t grxdnnGetTensorNdDescriptor(grxdnnTensorDescriptor_t desc,
                                           int nbDimsRequested,
                                           grxDataType_t* dataType,
                                           int* nbDims, int dims[],
                                           int strides[]);

/* ---- normalisation ------------------------------------------------------
 * x, y: [..., hidden]; every dimension but the last is a row index, the last
 * is normalised. The row dimensions must flatten to one row stride (packed
 * rows, or rows padded by a constant pitch). gamma/beta: 1-d [hidden],
 * contiguous, same type as x. Supported types: GRX_R_16BF, GRX_R_16F,
 * GRX_R_32F, with y of the same type and shape as x. Reductions are fp32.
 *
 *   RMSNorm:   y = x * rsqrt(mean(x^2) + eps) * gamma
 *   LayerNorm: y = (x - mean(x)) * rsqrt(var(x) + eps) * gamma + beta
 *              (biased variance)
 * eps must be finite and >= 0. hidden must be >= 1 and <= 65536. */
grxdnnStatus_t grxdnnRMSNormForward(grxdnnHandle_t handle,
                                    grxdnnTensorDescriptor_t xDesc,
                                    const void* x,
                                    grxdnnTensorDescriptor_t wDesc,
                                    const void* gamma, float eps,
                                    grxdnnTensorDescriptor_t yDesc, void* y);

grxdnnStatus_t grxdnnLayerNormForward(grxdnnHandle_t handle,
                                      grxdnnTensorDescriptor_t xDesc,
                                      const void* x,
                                      grxdnnTensorDescriptor_t wDesc,
                                      const void* gamma, const void* beta,
                                      float eps,
                                      grxdnnTensorDescriptor_t yDesc, void* y);

/* ---- softmax (forward) ---------------------------------------------------
 * Over the last dimension of x, every other dimension a row index:
 *   y[..., i] = exp(x[..., i] - m) / sum_j exp(x[..., j] - m),  m = max_j x[..., j]
 * Same layout rules and types as the normalisations above (rows flatten to
 * one row stride, innermost stride 1; GRX_R_16BF, GRX_R_16F or GRX_R_32F; y
 * of x's type and shape); fp32 arithmetic, y rounded once. A row whose every
 * element is -inf gives NaN, as the formula does. hidden: 1 .. 2^24.
 * (New: planned by ref docs/designs/grxcp_roadmap.md:864-877.) */
grxdnnStatus_t grxdnnSoftmaxForward(grxdnnHandle_t handle,
                                    grxdnnTensorDescriptor_t xDesc, const void* x,
                                    grxdnnTensorDescriptor_t yDesc, void* y);

/* ---- GELU (forward, element-wise) -----------------------------------------
 *   GRXDNN_GELU_ERF:  y = x/2 * (1 + erf(x / sqrt(2)))
 *   GRXDNN_GELU_TANH: y = x/2 * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3)))
 * x and y: descriptors of the same shape and type (GRX_R_16BF, GRX_R_16F,
 * GRX_R_32F) under the row layout rules above; fp32 arithmetic, y rounded
 * once; y may be x (in place). hidden: 1 .. 2^24.
 * (New: planned by ref docs/designs/grxcp_roadmap.md:864-877.) */
typedef enum {
  GRXDNN_GELU_ERF  = 0,
  GRXDNN_GELU_TANH = 1
} grxdnnGeluMode_t;

grxdnnStatus_t grxdnnGeluForward(grxdnnHandle_t handle, grxdnnGeluMode_t mode,
                                 grxdnnTensorDescriptor_t xDesc, const void* x,
                                 grxdnnTensorDescriptor_t yDesc, void* y);

/* ---- fused scaled-dot-product attention (forward) ----------------------
 *
 *   O[b,h,i,:] = sum_j softmax_j( scale * <Q[b,h,i,:], K[b,h,j,:]> + mask ) V[b,h,j,:]
 *
 * with mask = -inf for j > i when causal (the query and key sequences have
 * the same length and are aligned at position 0). Q, K, V, O are 4-d
 * [B, H, S, D] descriptors of one type (GRX_R_16BF or GRX_R_16F), innermost
 * stride 1, with equal B, H, S and D. Supported head dimensions: 64, 128.
 * The other strides are multiples of 8 elements and the pointers 16-byte
 * aligned, and each tensor's sequence stride times 2 * (S + 256) bytes stays
 * below 2^31 (else NOT_SUPPORTED); O's elements must not share addresses (else
 * INVALID_VALUE), while Q, K and V may (a broadcast). O must share no
 * element with K or V, and none with Q unless it is Q itself (same pointer,
 * same strides: in place); else INVALID_VALUE. Where O and the other view
 * have the same strides the test is exact, element by element (O in its own
 * slot of a packed [B, S, n, H, D] buffer is accepted); otherwise it is on
 * the address ranges the descriptors span.
 * Softmax and both products accumulate in fp32; O is rounded once (RNE). */
grxdnnStatus_t grxdnnCreateAttentionDescriptor (grxdnnAttentionDescriptor_t* d);
grxdnnStatus_t grxdnnDestroyAttentionDescriptor(grxdnnAttentionDescriptor_t d);
/* causal: 0 or 1. softmaxScale: finite and > 0 (1/sqrt(D) is the usual). */
grxdnnStatus_t grxdnnSetAttentionDescriptor(grxdnnAttentionDescriptor_t d,
                                            int causal, float softmaxScale);
grxdnnStatus_t grxdnnGetAttentionDescriptor(grxdnnAttentionDescriptor_t d,
                                            int* causal, float* softmaxScale);

grxdnnStatus_t grxdnnAttentionForward(grxdnnHandle_t handle,
                                      grxdnnAttentionDescriptor_t attnDesc,
                                      grxdnnTensorDescriptor_t qDesc, const void* q,
                                      grxdnnTensorDescriptor_t kDesc, const void* k,
                                      grxdnnTensorDescriptor_t vDesc, const void* v,
                                      grxdnnTensorDescriptor_t oDesc, void* o);

/* Per-wave cycle records of grxdnnAttentionForward, in grxBLAS's probe
 * format and manner (grx_cycles.h; ref include/grx/grxblas.h:240-242, which
 * grxDNN, new, extends to attention). With a slot array attached, the next
 * attention calls write one grxCycleSlot per wave that has work (slot =
 * workgroup * waves per workgroup + wave; s_memtime at entry and exit, core
 * = XCD << 16 | CU id); capacity must cover
 * grxdnnAttentionCycleSlotsNeeded for the call's B, H and S, else the call
 * returns INVALID_VALUE before any device work. NULL turns recording off. */
grxdnnStatus_t grxdnnSetCycleProbe(grxdnnHandle_t handle, grxCycleSlot* slots,
                                   int capacity);
int            grxdnnAttentionCycleSlotsNeeded(grxdnnHandle_t handle, int batch,
                                               int heads, int seqLen);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* GRXDNN_H */
