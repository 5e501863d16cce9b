/* host_grxrt.c -- the grx runtime subset of grx_runtime.h on the host CPU.
 *
 * TEST INFRASTRUCTURE / CPU HOST BACKEND. Built into oracle/libgrxrt_ref.so,
 * the runtime half of the CPU host backend that BASELINE config 1 ("runs on
 * the repo's host/mock reference backend on CPU") names. The reference's own
 * mock driver records launches and computes nothing (ref
 * tests/mock/vortex_mock.cpp:27-29); this one is a real CPU device: one
 * device, "device" memory is host memory, copies are memcpy, streams and
 * events are bookkeeping objects and every call completes before it returns
 * (so synchronisation is a no-op). The product libraries (libgrxrt.so,
 * libgrxblas.so, libgrxdnn.so) never load it.
 *
 * Names, signatures and error codes follow include/grx/grx_runtime.h (ref
 * include/grx/grx_runtime.h:25-114).
 */
#define _POSIX_C_SOURCE 200809L
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include "grx/grx_runtime.h"

#define EXPORT __attribute__((visibility("default")))

static _Thread_local grxError_t t_last = grxSuccess;

static grxError_t rec(grxError_t e) {
  if (e != grxSuccess) t_last = e;
  return e;
}

struct grxStream { int magic; };
struct grxEvent { int magic; double t_ms; int recorded; unsigned flags; };
enum { kStreamMagic = 0x57524d53, kEventMagic = 0x544e5645 };

static double now_ms(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec * 1e3 + (double)ts.tv_nsec * 1e-6;
}

EXPORT const char* grxGetErrorName(grxError_t e) {
  switch (e) {
    case grxSuccess: return "grxSuccess";
    case grxErrorInvalidValue: return "grxErrorInvalidValue";
    case grxErrorMemoryAllocation: return "grxErrorMemoryAllocation";
    case grxErrorInitializationError: return "grxErrorInitializationError";
    case grxErrorInvalidDevice: return "grxErrorInvalidDevice";
    case grxErrorInvalidDevicePointer: return "grxErrorInvalidDevicePointer";
    case grxErrorInvalidMemcpyDirection: return "grxErrorInvalidMemcpyDirection";
    case grxErrorInvalidResourceHandle: return "grxErrorInvalidResourceHandle";
    case grxErrorNotReady: return "grxErrorNotReady";
    case grxErrorNotSupported: return "grxErrorNotSupported";
    default: return "grxErrorUnknown";
  }
}

EXPORT const char* grxGetErrorString(grxError_t e) {
  switch (e) {
    case grxSuccess: return "no error";
    case grxErrorInvalidValue: return "invalid argument";
    case grxErrorMemoryAllocation: return "out of host memory";
    case grxErrorInvalidDevice: return "invalid device ordinal (the host backend has one device)";
    case grxErrorInvalidMemcpyDirection: return "invalid copy direction";
    case grxErrorInvalidResourceHandle: return "invalid stream or event";
    case grxErrorNotReady: return "not ready";
    case grxErrorNotSupported: return "not supported by the host backend";
    default: return "unknown error";
  }
}

EXPORT grxError_t grxGetDeviceCount(int* count) {
  if (!count) return rec(grxErrorInvalidValue);
  *count = 1;
  return grxSuccess;
}
EXPORT grxError_t grxSetDevice(int device) {
  return rec(device == 0 ? grxSuccess : grxErrorInvalidDevice);
}
EXPORT grxError_t grxGetDevice(int* device) {
  if (!device) return rec(grxErrorInvalidValue);
  *device = 0;
  return grxSuccess;
}
EXPORT grxError_t grxGetDeviceProperties(grxDeviceProp_t* p, int device) {
  if (!p) return rec(grxErrorInvalidValue);
  if (device != 0) return rec(grxErrorInvalidDevice);
  memset(p, 0, sizeof *p);
  strncpy(p->name, "host CPU (grxBLAS reference backend)", sizeof p->name - 1);
  p->deviceType = GRX_DEVICE_TYPE_GPU;
  p->backend = GRX_BACKEND_SIMX;
  p->capabilities = GRX_CAP_STREAMS | GRX_CAP_EVENTS | GRX_CAP_MEMCPY | GRX_CAP_GEMM |
                    GRX_CAP_UNIFIED_ADDRESSING;
  p->warpSize = 1;
  p->maxWarpsPerMultiProcessor = 1;
  const long cpus = sysconf(_SC_NPROCESSORS_ONLN);
  p->multiProcessorCount = cpus > 0 ? (int)cpus : 1;
  p->clusterCount = 1;
  p->socketSize = 1;
  p->issueWidth = 1;
  p->maxThreadsPerBlock = 1;
  p->maxThreadsDim[0] = p->maxThreadsDim[1] = p->maxThreadsDim[2] = 1;
  p->maxGridSize[0] = p->maxGridSize[1] = p->maxGridSize[2] = 1;
  const long pages = sysconf(_SC_PHYS_PAGES), psz = sysconf(_SC_PAGE_SIZE);
  p->totalGlobalMem = (pages > 0 && psz > 0) ? (size_t)pages * (size_t)psz : 0;
  p->cacheLineSize = 64;
  p->unifiedAddressing = 1;
  p->eventTimingIsDeviceSide = 0;
  return grxSuccess;
}
EXPORT grxError_t grxDeviceSynchronize(void) { return grxSuccess; }
EXPORT grxError_t grxMemGetInfo(size_t* freeBytes, size_t* totalBytes) {
  if (!freeBytes || !totalBytes) return rec(grxErrorInvalidValue);
  const long av = sysconf(_SC_AVPHYS_PAGES), pages = sysconf(_SC_PHYS_PAGES),
             psz = sysconf(_SC_PAGE_SIZE);
  *freeBytes = (av > 0 && psz > 0) ? (size_t)av * (size_t)psz : 0;
  *totalBytes = (pages > 0 && psz > 0) ? (size_t)pages * (size_t)psz : 0;
  return grxSuccess;
}

EXPORT grxError_t grxGetLastError(void) {
  const grxError_t e = t_last;
  t_last = grxSuccess;
  return e;
}
EXPORT grxError_t grxPeekAtLastError(void) { return t_last; }

EXPORT grxError_t grxMalloc(void** ptr, size_t size) {
  if (!ptr) return rec(grxErrorInvalidValue);
  *ptr = NULL;
  if (size == 0) return grxSuccess;
  /* 256-byte alignment, as device allocations have */
  if (posix_memalign(ptr, 256, size) != 0) {
    *ptr = NULL;
    return rec(grxErrorMemoryAllocation);
  }
  return grxSuccess;
}
EXPORT grxError_t grxFree(void* ptr) {
  free(ptr);
  return grxSuccess;
}
EXPORT grxError_t grxMallocHost(void** ptr, size_t size) { return grxMalloc(ptr, size); }
EXPORT grxError_t grxFreeHost(void* ptr) { return grxFree(ptr); }

EXPORT grxError_t grxMemcpy(void* dst, const void* src, size_t count, grxMemcpyKind kind) {
  if ((int)kind < (int)grxMemcpyHostToHost || (int)kind > (int)grxMemcpyDefault)
    return rec(grxErrorInvalidMemcpyDirection);
  if (count == 0) return grxSuccess;
  if (!dst || !src) return rec(grxErrorInvalidValue);
  memmove(dst, src, count);
  return grxSuccess;
}
static int stream_ok(grxStream_t s) { return !s || s->magic == kStreamMagic; }
EXPORT grxError_t grxMemcpyAsync(void* dst, const void* src, size_t count, grxMemcpyKind kind,
                                 grxStream_t stream) {
  if (!stream_ok(stream)) return rec(grxErrorInvalidResourceHandle);
  return grxMemcpy(dst, src, count, kind);
}
EXPORT grxError_t grxMemset(void* dst, int value, size_t count) {
  if (count == 0) return grxSuccess;
  if (!dst) return rec(grxErrorInvalidValue);
  memset(dst, value, count);
  return grxSuccess;
}
EXPORT grxError_t grxMemsetAsync(void* dst, int value, size_t count, grxStream_t stream) {
  if (!stream_ok(stream)) return rec(grxErrorInvalidResourceHandle);
  return grxMemset(dst, value, count);
}

EXPORT grxError_t grxStreamCreate(grxStream_t* stream) {
  return grxStreamCreateWithFlags(stream, grxStreamDefault);
}
EXPORT grxError_t grxStreamCreateWithFlags(grxStream_t* stream, unsigned int flags) {
  if (!stream || (flags & ~grxStreamNonBlocking)) return rec(grxErrorInvalidValue);
  struct grxStream* s = (struct grxStream*)malloc(sizeof *s);
  if (!s) return rec(grxErrorMemoryAllocation);
  s->magic = kStreamMagic;
  *stream = s;
  return grxSuccess;
}
EXPORT grxError_t grxStreamDestroy(grxStream_t stream) {
  if (!stream || stream->magic != kStreamMagic) return rec(grxErrorInvalidResourceHandle);
  stream->magic = 0;
  free(stream);
  return grxSuccess;
}
EXPORT grxError_t grxStreamSynchronize(grxStream_t stream) {
  return stream_ok(stream) ? grxSuccess : rec(grxErrorInvalidResourceHandle);
}
EXPORT grxError_t grxStreamQuery(grxStream_t stream) {
  return stream_ok(stream) ? grxSuccess : rec(grxErrorInvalidResourceHandle);
}
static int event_ok(grxEvent_t e) { return e && e->magic == kEventMagic; }
EXPORT grxError_t grxStreamWaitEvent(grxStream_t stream, grxEvent_t event, unsigned int flags) {
  if (!stream_ok(stream) || !event_ok(event)) return rec(grxErrorInvalidResourceHandle);
  return flags == 0 ? grxSuccess : rec(grxErrorInvalidValue);
}

EXPORT grxError_t grxEventCreate(grxEvent_t* event) {
  return grxEventCreateWithFlags(event, grxEventDefault);
}
EXPORT grxError_t grxEventCreateWithFlags(grxEvent_t* event, unsigned int flags) {
  if (!event || (flags & ~(grxEventBlockingSync | grxEventDisableTiming)))
    return rec(grxErrorInvalidValue);
  struct grxEvent* e = (struct grxEvent*)calloc(1, sizeof *e);
  if (!e) return rec(grxErrorMemoryAllocation);
  e->magic = kEventMagic;
  e->flags = flags;
  *event = e;
  return grxSuccess;
}
EXPORT grxError_t grxEventDestroy(grxEvent_t event) {
  if (!event_ok(event)) return rec(grxErrorInvalidResourceHandle);
  event->magic = 0;
  free(event);
  return grxSuccess;
}
EXPORT grxError_t grxEventRecord(grxEvent_t event, grxStream_t stream) {
  if (!event_ok(event) || !stream_ok(stream)) return rec(grxErrorInvalidResourceHandle);
  event->t_ms = now_ms();
  event->recorded = 1;
  return grxSuccess;
}
EXPORT grxError_t grxEventSynchronize(grxEvent_t event) {
  return event_ok(event) ? grxSuccess : rec(grxErrorInvalidResourceHandle);
}
EXPORT grxError_t grxEventQuery(grxEvent_t event) {
  return event_ok(event) ? grxSuccess : rec(grxErrorInvalidResourceHandle);
}
EXPORT grxError_t grxEventElapsedTime(float* ms, grxEvent_t start, grxEvent_t end) {
  if (!ms) return rec(grxErrorInvalidValue);
  if (!event_ok(start) || !event_ok(end)) return rec(grxErrorInvalidResourceHandle);
  if (!start->recorded || !end->recorded) return rec(grxErrorNotReady);
  if ((start->flags | end->flags) & grxEventDisableTiming) return rec(grxErrorInvalidResourceHandle);
  *ms = (float)(end->t_ms - start->t_ms);
  return grxSuccess;
}
