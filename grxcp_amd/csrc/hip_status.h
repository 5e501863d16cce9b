// Internal: the single HIP -> grx error table, shared by the three libraries
// (inline, so each library carries it without exporting it).
#ifndef GRXCP_HIP_STATUS_H
#define GRXCP_HIP_STATUS_H

#include <grx/grx_types.h>
#include <hip/hip_runtime_api.h>

// One table from HIP's error space to grx's (the role of the reference's
// error map, ref src/runtime/error.cpp:9-24).
inline grxError_t grx_from_hip(hipError_t e) {
  switch (e) {
    case hipSuccess:                    return grxSuccess;
    case hipErrorInvalidValue:          return grxErrorInvalidValue;
    case hipErrorOutOfMemory:           return grxErrorMemoryAllocation;
    case hipErrorNotInitialized:        return grxErrorInitializationError;
    case hipErrorNoDevice:
    case hipErrorInvalidDevice:         return grxErrorInvalidDevice;
    case hipErrorInvalidDevicePointer:  return grxErrorInvalidDevicePointer;
    case hipErrorInvalidMemcpyDirection:return grxErrorInvalidMemcpyDirection;
    case hipErrorInvalidHandle:         return grxErrorInvalidResourceHandle;
    case hipErrorNotReady:              return grxErrorNotReady;
    case hipErrorNotSupported:          return grxErrorNotSupported;
    case hipErrorInvalidImage:
    case hipErrorNoBinaryForGpu:        return grxErrorInvalidKernelImage;
    case hipErrorInvalidDeviceFunction: return grxErrorInvalidDeviceFunction;
    case hipErrorLaunchFailure:         return grxErrorLaunchFailure;
    case hipErrorLaunchOutOfResources:  return grxErrorLaunchOutOfResources;
    case hipErrorLaunchTimeOut:         return grxErrorTimeout;
    case hipErrorFileNotFound:          return grxErrorFileNotFound;
    case hipErrorInvalidSymbol:         return grxErrorInvalidSymbol;
    default:                            return grxErrorUnknown;
  }
}

#endif
