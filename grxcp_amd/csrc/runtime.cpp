// libgrxrt.so -- the grx runtime subset, as direct calls into HIP.
//
// Replaces the reference's L1 runtime for the calls the math-library hot path
// and its callers use (ref: src/runtime/{context,memory,stream,event,error}.cpp,
// declared at ref include/grx/grx_runtime.h:25-114). There is no module
// loader, fat binary, tensor-map or occupancy machinery here: the gfx950
// kernels are linked into libgrxblas.so / libgrxdnn.so and launched with
// hipLaunchKernelGGL by those libraries.

#include <grx/grx_runtime.h>

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>

#include "hip_status.h"

namespace {

thread_local grxError_t t_last_error = grxSuccess;

grxError_t record(hipError_t e) {
  const grxError_t g = grx_from_hip(e);
  if (g != grxSuccess) t_last_error = g;
  return g;
}

hipMemcpyKind to_hip(grxMemcpyKind k, bool* ok) {
  *ok = true;
  switch (k) {
    case grxMemcpyHostToHost:     return hipMemcpyHostToHost;
    case grxMemcpyHostToDevice:   return hipMemcpyHostToDevice;
    case grxMemcpyDeviceToHost:   return hipMemcpyDeviceToHost;
    case grxMemcpyDeviceToDevice: return hipMemcpyDeviceToDevice;
    case grxMemcpyDefault:        return hipMemcpyDefault;
  }
  *ok = false;
  return hipMemcpyDefault;
}

hipStream_t hs(grxStream_t s) { return reinterpret_cast<hipStream_t>(s); }
hipEvent_t he(grxEvent_t e) { return reinterpret_cast<hipEvent_t>(e); }

}  // namespace

// The C API is the only thing these libraries export (built with
// -fvisibility=hidden).
#pragma GCC visibility push(default)
extern "C" {

const char* grxGetErrorName(grxError_t e) {
  switch (e) {
#define GRX_NAME(x) case x: return #x;
    GRX_NAME(grxSuccess)
    GRX_NAME(grxErrorInvalidValue)
    GRX_NAME(grxErrorMemoryAllocation)
    GRX_NAME(grxErrorInitializationError)
    GRX_NAME(grxErrorInvalidDevice)
    GRX_NAME(grxErrorInvalidDevicePointer)
    GRX_NAME(grxErrorInvalidMemcpyDirection)
    GRX_NAME(grxErrorInvalidResourceHandle)
    GRX_NAME(grxErrorNotReady)
    GRX_NAME(grxErrorNotSupported)
    GRX_NAME(grxErrorInvalidKernelImage)
    GRX_NAME(grxErrorInvalidDeviceFunction)
    GRX_NAME(grxErrorLaunchFailure)
    GRX_NAME(grxErrorLaunchOutOfResources)
    GRX_NAME(grxErrorDeviceLost)
    GRX_NAME(grxErrorTimeout)
    GRX_NAME(grxErrorFileNotFound)
    GRX_NAME(grxErrorInvalidSymbol)
    GRX_NAME(grxErrorUnknown)
#undef GRX_NAME
  }
  return "grxErrorUnknown";
}

const char* grxGetErrorString(grxError_t e) {
  switch (e) {
    case grxSuccess:                     return "no error";
    case grxErrorInvalidValue:           return "invalid argument";
    case grxErrorMemoryAllocation:       return "out of memory";
    case grxErrorInitializationError:    return "initialization error";
    case grxErrorInvalidDevice:          return "invalid or absent device";
    case grxErrorInvalidDevicePointer:   return "invalid device pointer";
    case grxErrorInvalidMemcpyDirection: return "invalid copy direction";
    case grxErrorInvalidResourceHandle:  return "invalid resource handle";
    case grxErrorNotReady:               return "not ready";
    case grxErrorNotSupported:           return "not supported";
    case grxErrorInvalidKernelImage:     return "no kernel image for this device";
    case grxErrorInvalidDeviceFunction:  return "invalid device function";
    case grxErrorLaunchFailure:          return "kernel launch failure";
    case grxErrorLaunchOutOfResources:   return "launch out of resources";
    case grxErrorDeviceLost:             return "device lost";
    case grxErrorTimeout:                return "timeout";
    case grxErrorFileNotFound:           return "file not found";
    case grxErrorInvalidSymbol:          return "invalid symbol";
    case grxErrorUnknown:                return "unknown error";
  }
  return "unknown error";
}

grxError_t grxGetDeviceCount(int* count) {
  if (!count) return grxErrorInvalidValue;
  *count = 0;
  const hipError_t e = hipGetDeviceCount(count);
  if (e == hipErrorNoDevice) { *count = 0; return grxSuccess; }
  return record(e);
}

grxError_t grxSetDevice(int device) { return record(hipSetDevice(device)); }

grxError_t grxGetDevice(int* device) {
  if (!device) return grxErrorInvalidValue;
  return record(hipGetDevice(device));
}

grxError_t grxGetDeviceProperties(grxDeviceProp_t* prop, int device) {
  if (!prop) return grxErrorInvalidValue;
  hipDeviceProp_t p;
  const hipError_t e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return record(e);
  std::memset(prop, 0, sizeof(*prop));
  std::snprintf(prop->name, sizeof(prop->name), "%.96s (%.24s)", p.name, p.gcnArchName);
  prop->deviceType = GRX_DEVICE_TYPE_GPU;
  prop->backend = GRX_BACKEND_SILICON;
  prop->capabilities = GRX_CAP_KERNEL_LAUNCH | GRX_CAP_STREAMS | GRX_CAP_EVENTS |
                       GRX_CAP_MEMCPY | GRX_CAP_GEMM | GRX_CAP_UNIFIED_ADDRESSING |
                       GRX_CAP_COOPERATIVE_LAUNCH | GRX_CAP_GLOBAL_ATOMICS;
  // Matrix cores and an LDS-staging path exist on CDNA3/CDNA4 (gfx94x/gfx95x).
  if (std::strncmp(p.gcnArchName, "gfx95", 5) == 0 ||
      std::strncmp(p.gcnArchName, "gfx94", 5) == 0)
    prop->capabilities |= GRX_CAP_TENSOR_CORE | GRX_CAP_ASYNC_COPY;
  prop->computeCapabilityMajor = p.major;
  prop->computeCapabilityMinor = p.minor;
  prop->warpSize = p.warpSize;
  prop->maxWarpsPerMultiProcessor =
      p.warpSize > 0 ? p.maxThreadsPerMultiProcessor / p.warpSize : 0;
  prop->multiProcessorCount = p.multiProcessorCount;
  int xcc = 1;
  if (hipDeviceGetAttribute(&xcc, hipDeviceAttributeNumberOfXccs, device) != hipSuccess ||
      xcc < 1)
    xcc = 1;
  prop->clusterCount = xcc;
  prop->socketSize = 1;
  prop->issueWidth = 1;
  prop->maxThreadsPerBlock = p.maxThreadsPerBlock;
  for (int i = 0; i < 3; ++i) {
    prop->maxThreadsDim[i] = p.maxThreadsDim[i];
    prop->maxGridSize[i] = p.maxGridSize[i];
  }
  prop->numBarriers = 16;
  prop->totalGlobalMem = p.totalGlobalMem;
  prop->sharedMemPerMultiprocessor = p.maxSharedMemoryPerMultiProcessor;
  prop->sharedMemPerBlock = p.sharedMemPerBlock;
  prop->memBankCount = 64;
  prop->memBankSize = 4;
  prop->cacheLineSize = 128;
  prop->clockRateMHz = p.clockRate / 1000;
  // bus width (bits) x memory clock (kHz) x 2 (DDR) / 8 -> bytes/ms -> MB/s
  prop->peakMemoryBandwidthMBs =
      (size_t)((double)p.memoryBusWidth / 8.0 * (double)p.memoryClockRate * 2.0 / 1000.0);
  prop->unifiedAddressing = 1;
  prop->managedMemory = p.managedMemory;
  prop->warpShuffleIsEmulated = 0;
  prop->eventTimingIsDeviceSide = 1;
  prop->constantMemoryIsGlobal = 0;
  return grxSuccess;
}

grxError_t grxDeviceSynchronize(void) { return record(hipDeviceSynchronize()); }

grxError_t grxMemGetInfo(size_t* freeBytes, size_t* totalBytes) {
  if (!freeBytes || !totalBytes) return grxErrorInvalidValue;
  return record(hipMemGetInfo(freeBytes, totalBytes));
}

grxError_t grxGetLastError(void) {
  const grxError_t e = t_last_error;
  t_last_error = grxSuccess;
  return e;
}

grxError_t grxPeekAtLastError(void) { return t_last_error; }

grxError_t grxMalloc(void** ptr, size_t size) {
  if (!ptr) return grxErrorInvalidValue;
  *ptr = nullptr;
  if (size == 0) return grxSuccess;
  return record(hipMalloc(ptr, size));
}

grxError_t grxFree(void* ptr) {
  if (!ptr) return grxSuccess;
  return record(hipFree(ptr));
}

grxError_t grxMallocHost(void** ptr, size_t size) {
  if (!ptr) return grxErrorInvalidValue;
  *ptr = nullptr;
  if (size == 0) return grxSuccess;
  return record(hipHostMalloc(ptr, size, hipHostMallocDefault));
}

grxError_t grxFreeHost(void* ptr) {
  if (!ptr) return grxSuccess;
  return record(hipHostFree(ptr));
}

grxError_t grxMemcpy(void* dst, const void* src, size_t count, grxMemcpyKind kind) {
  if (count == 0) return grxSuccess;
  if (!dst || !src) return grxErrorInvalidValue;
  bool ok = false;
  const hipMemcpyKind k = to_hip(kind, &ok);
  if (!ok) return grxErrorInvalidMemcpyDirection;
  return record(hipMemcpy(dst, src, count, k));
}

grxError_t grxMemcpyAsync(void* dst, const void* src, size_t count,
                          grxMemcpyKind kind, grxStream_t stream) {
  if (count == 0) return grxSuccess;
  if (!dst || !src) return grxErrorInvalidValue;
  bool ok = false;
  const hipMemcpyKind k = to_hip(kind, &ok);
  if (!ok) return grxErrorInvalidMemcpyDirection;
  return record(hipMemcpyAsync(dst, src, count, k, hs(stream)));
}

grxError_t grxMemset(void* dst, int value, size_t count) {
  if (count == 0) return grxSuccess;
  if (!dst) return grxErrorInvalidValue;
  return record(hipMemset(dst, value, count));
}

grxError_t grxMemsetAsync(void* dst, int value, size_t count, grxStream_t stream) {
  if (count == 0) return grxSuccess;
  if (!dst) return grxErrorInvalidValue;
  return record(hipMemsetAsync(dst, value, count, hs(stream)));
}

grxError_t grxStreamCreate(grxStream_t* stream) {
  return grxStreamCreateWithFlags(stream, grxStreamDefault);
}

grxError_t grxStreamCreateWithFlags(grxStream_t* stream, unsigned int flags) {
  if (!stream) return grxErrorInvalidValue;
  if (flags & ~grxStreamNonBlocking) return grxErrorInvalidValue;
  hipStream_t s = nullptr;
  const hipError_t e = hipStreamCreateWithFlags(
      &s, (flags & grxStreamNonBlocking) ? hipStreamNonBlocking : hipStreamDefault);
  if (e != hipSuccess) return record(e);
  *stream = reinterpret_cast<grxStream_t>(s);
  return grxSuccess;
}

grxError_t grxStreamDestroy(grxStream_t stream) {
  if (!stream) return grxErrorInvalidResourceHandle;
  return record(hipStreamDestroy(hs(stream)));
}

grxError_t grxStreamSynchronize(grxStream_t stream) {
  return record(hipStreamSynchronize(hs(stream)));
}

grxError_t grxStreamQuery(grxStream_t stream) {
  const hipError_t e = hipStreamQuery(hs(stream));
  if (e == hipErrorNotReady) return grxErrorNotReady;
  return record(e);
}

grxError_t grxStreamWaitEvent(grxStream_t stream, grxEvent_t event, unsigned int flags) {
  if (!event) return grxErrorInvalidResourceHandle;
  return record(hipStreamWaitEvent(hs(stream), he(event), flags));
}

grxError_t grxEventCreate(grxEvent_t* event) {
  return grxEventCreateWithFlags(event, grxEventDefault);
}

grxError_t grxEventCreateWithFlags(grxEvent_t* event, unsigned int flags) {
  if (!event) return grxErrorInvalidValue;
  if (flags & ~(grxEventBlockingSync | grxEventDisableTiming)) return grxErrorInvalidValue;
  unsigned hf = hipEventDefault;
  if (flags & grxEventBlockingSync) hf |= hipEventBlockingSync;
  if (flags & grxEventDisableTiming) hf |= hipEventDisableTiming;
  hipEvent_t ev = nullptr;
  const hipError_t e = hipEventCreateWithFlags(&ev, hf);
  if (e != hipSuccess) return record(e);
  *event = reinterpret_cast<grxEvent_t>(ev);
  return grxSuccess;
}

grxError_t grxEventDestroy(grxEvent_t event) {
  if (!event) return grxErrorInvalidResourceHandle;
  return record(hipEventDestroy(he(event)));
}

grxError_t grxEventRecord(grxEvent_t event, grxStream_t stream) {
  if (!event) return grxErrorInvalidResourceHandle;
  return record(hipEventRecord(he(event), hs(stream)));
}

grxError_t grxEventSynchronize(grxEvent_t event) {
  if (!event) return grxErrorInvalidResourceHandle;
  return record(hipEventSynchronize(he(event)));
}

grxError_t grxEventQuery(grxEvent_t event) {
  if (!event) return grxErrorInvalidResourceHandle;
  const hipError_t e = hipEventQuery(he(event));
  if (e == hipErrorNotReady) return grxErrorNotReady;
  return record(e);
}

grxError_t grxEventElapsedTime(float* ms, grxEvent_t start, grxEvent_t end) {
  if (!ms) return grxErrorInvalidValue;
  if (!start || !end) return grxErrorInvalidResourceHandle;
  return record(hipEventElapsedTime(ms, he(start), he(end)));
}

}  // extern "C"
#pragma GCC visibility pop
