/* grx_types.h -- core types of the grx host API, MI355X (gfx950) build.
 *
 * The subset of the reference's core types that the grxBLAS / grxDNN hot path
 * and its callers touch. Enumerator VALUES are kept identical to the
 * reference (ref: include/grx/grx_types.h:22-45, 120-134) so that code which
 * switches on them, logs them or stores them keeps working unchanged.
 *
 * One addition: GRX_R_16BF = 14 (the same value CUDA uses for CUDA_R_16BF).
 * The reference leaves bfloat16 out because its tensor unit has no bf16 mode;
 * gfx950's matrix cores do, so here it is a first-class GemmEx type.
 */
#ifndef GRX_TYPES_H
#define GRX_TYPES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime errors (ref: include/grx/grx_types.h:22-45) ---------------- */
typedef enum {
  grxSuccess                     = 0,
  grxErrorInvalidValue           = 1,
  grxErrorMemoryAllocation       = 2,
  grxErrorInitializationError    = 3,
  grxErrorInvalidDevice          = 4,
  grxErrorInvalidDevicePointer   = 5,
  grxErrorInvalidMemcpyDirection = 6,
  grxErrorInvalidResourceHandle  = 7,
  grxErrorNotReady               = 8,
  grxErrorNotSupported           = 9,
  grxErrorInvalidKernelImage     = 10,
  grxErrorInvalidDeviceFunction  = 11,
  grxErrorLaunchFailure          = 12,
  grxErrorLaunchOutOfResources   = 13,
  grxErrorDeviceLost             = 14,
  grxErrorTimeout                = 15,
  grxErrorFileNotFound           = 16,
  grxErrorInvalidSymbol          = 17,
  grxErrorUnknown                = 999
} grxError_t;

/* ---- opaque handles (ref: include/grx/grx_types.h:70-79) ----------------
 * On this build a grxStream_t IS a hipStream_t and a grxEvent_t IS a
 * hipEvent_t, cast through an incomplete struct type so that C callers never
 * need HIP headers. A null grxStream_t is the device's default stream. */
typedef struct grxStream* grxStream_t;
typedef struct grxEvent*  grxEvent_t;

#define grxStreamDefault      0x00u
#define grxStreamNonBlocking  0x01u
#define grxEventDefault       0x00u
#define grxEventBlockingSync  0x01u
#define grxEventDisableTiming 0x02u

/* ---- copies (ref: include/grx/grx_types.h:85-94) ------------------------- */
typedef enum {
  grxMemcpyHostToHost     = 0,
  grxMemcpyHostToDevice   = 1,
  grxMemcpyDeviceToHost   = 2,
  grxMemcpyDeviceToDevice = 3,
  grxMemcpyDefault        = 4  /* direction inferred from the pointers */
} grxMemcpyKind;

/* ---- element types (ref: include/grx/grx_types.h:120-134) --------------- */
typedef enum {
  GRX_R_32F  = 0,   /* IEEE binary32 */
  GRX_R_16F  = 2,   /* IEEE binary16 */
  GRX_R_8I   = 3,   /* signed 8-bit integer */
  GRX_R_32I  = 10,  /* signed 32-bit integer */
  GRX_R_16BF = 14   /* bfloat16 (new on this build; CUDA_R_16BF's value) */
} grxDataType_t;

/* ---- device model (ref: include/grx/grx_types.h:140-216) ----------------
 * The property struct keeps the reference's field list and order so callers
 * that print or test fields compile unchanged. Values describe the HIP device:
 * warpSize is the wavefront width (64), multiProcessorCount the CU count,
 * clusterCount the XCD count. */
typedef enum { GRX_DEVICE_TYPE_GPU = 0, GRX_DEVICE_TYPE_NPU = 1 } grxDeviceType_t;

typedef enum {
  GRX_BACKEND_SIMX    = 0,
  GRX_BACKEND_RTLSIM  = 1,
  GRX_BACKEND_XRT     = 2,
  GRX_BACKEND_OPAE    = 3,
  GRX_BACKEND_GEM5    = 4,
  GRX_BACKEND_SILICON = 5
} grxBackend_t;

#define GRX_CAP_KERNEL_LAUNCH       (1u << 0)
#define GRX_CAP_STREAMS             (1u << 1)
#define GRX_CAP_EVENTS              (1u << 2)
#define GRX_CAP_MEMCPY              (1u << 3)
#define GRX_CAP_GEMM                (1u << 4)
#define GRX_CAP_UNIFIED_ADDRESSING  (1u << 5)
#define GRX_CAP_TENSOR_CORE         (1u << 6)
#define GRX_CAP_ASYNC_COPY          (1u << 7)
#define GRX_CAP_RAY_TRACING         (1u << 8)
#define GRX_CAP_COOPERATIVE_LAUNCH  (1u << 9)
#define GRX_CAP_GLOBAL_ATOMICS      (1u << 10)

typedef struct {
  char            name[128];
  grxDeviceType_t deviceType;
  grxBackend_t    backend;
  unsigned int    capabilities;
  int             computeCapabilityMajor;
  int             computeCapabilityMinor;

  int    warpSize;
  int    maxWarpsPerMultiProcessor;
  int    multiProcessorCount;
  int    clusterCount;
  int    socketSize;
  int    issueWidth;
  int    maxThreadsPerBlock;
  int    maxThreadsDim[3];
  int    maxGridSize[3];
  int    numBarriers;

  size_t totalGlobalMem;
  size_t sharedMemPerMultiprocessor;
  size_t sharedMemPerBlock;
  int    memBankCount;
  size_t memBankSize;
  int    cacheLineSize;
  int    clockRateMHz;
  size_t peakMemoryBandwidthMBs;
  int    unifiedAddressing;
  int    managedMemory;
  size_t pinnedMemTotal;
  size_t pinnedMemFree;

  int    warpShuffleIsEmulated;
  int    eventTimingIsDeviceSide;
  int    constantMemoryIsGlobal;
} grxDeviceProp_t;

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* GRX_TYPES_H */
