// Internal: the single HIP -> grx error table, shared by the three libraries.
#ifndef GRXCP_HIP_STATUS_H
#define GRXCP_HIP_STATUS_H

#include <grx/grx_types.h>
#include <hip/hip_runtime_api.h>

grxError_t grx_from_hip(hipError_t e);

#endif
