/* grx_runtime.h -- the runtime subset the grxBLAS / grxDNN hot path needs.
 *
 * The reference's L1 runtime (ref: include/grx/grx_runtime.h:25-234) drives
 * the GRX-G100 through vortex2.h: module loading, fat binaries, DXA tensor
 * maps, occupancy. None of that exists on MI355X. What callers of the math
 * libraries actually use -- device selection, allocation, copies, streams,
 * events, synchronisation -- is kept here with the reference's names and
 * semantics, implemented as thin calls into HIP (libgrxrt.so).
 *
 * grxStream_t / grxEvent_t are hipStream_t / hipEvent_t; the runtime never
 * wraps them, so a caller that already owns a HIP stream may pass it cast.
 */
#ifndef GRX_RUNTIME_H
#define GRX_RUNTIME_H

#include "grx_types.h"

#ifdef __cplusplus
extern "C" {
#endif

const char* grxGetErrorName  (grxError_t e);   /* ref grx_types.h:47 */
const char* grxGetErrorString(grxError_t e);   /* ref grx_types.h:48 */

/* device management (ref: grx_runtime.h:25-31) */
grxError_t grxGetDeviceCount     (int* count);
grxError_t grxSetDevice          (int device);
grxError_t grxGetDevice          (int* device);
grxError_t grxGetDeviceProperties(grxDeviceProp_t* prop, int device);
grxError_t grxDeviceSynchronize  (void);
grxError_t grxMemGetInfo         (size_t* freeBytes, size_t* totalBytes);

/* errors (ref: grx_runtime.h:44-45) */
grxError_t grxGetLastError   (void);
grxError_t grxPeekAtLastError(void);

/* memory (ref: grx_runtime.h:51-76) */
grxError_t grxMalloc     (void** ptr, size_t size);
grxError_t grxFree       (void* ptr);
grxError_t grxMallocHost (void** ptr, size_t size);
grxError_t grxFreeHost   (void* ptr);
grxError_t grxMemcpy     (void* dst, const void* src, size_t count,
                          grxMemcpyKind kind);
grxError_t grxMemcpyAsync(void* dst, const void* src, size_t count,
                          grxMemcpyKind kind, grxStream_t stream);
grxError_t grxMemset     (void* dst, int value, size_t count);
grxError_t grxMemsetAsync(void* dst, int value, size_t count,
                          grxStream_t stream);

/* streams (ref: grx_runtime.h:88-97). Every stream is created at the
 * default priority. */
grxError_t grxStreamCreate         (grxStream_t* stream);
grxError_t grxStreamCreateWithFlags(grxStream_t* stream, unsigned int flags);
grxError_t grxStreamDestroy        (grxStream_t stream);
grxError_t grxStreamSynchronize    (grxStream_t stream);
grxError_t grxStreamQuery          (grxStream_t stream);
grxError_t grxStreamWaitEvent      (grxStream_t stream, grxEvent_t event,
                                    unsigned int flags);

/* events (ref: grx_runtime.h:108-114). Timing is device-side (HIP events). */
grxError_t grxEventCreate         (grxEvent_t* event);
grxError_t grxEventCreateWithFlags(grxEvent_t* event, unsigned int flags);
grxError_t grxEventDestroy        (grxEvent_t event);
grxError_t grxEventRecord         (grxEvent_t event, grxStream_t stream);
grxError_t grxEventSynchronize    (grxEvent_t event);
grxError_t grxEventQuery          (grxEvent_t event);
grxError_t grxEventElapsedTime    (float* ms, grxEvent_t start, grxEvent_t end);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* GRX_RUNTIME_H */
