/* grx.h -- umbrella header for host code (ref: include/grx/grx.h:1-9).
 *
 * Every reference caller of the math libraries starts with
 * `#include <grx/grx.h>` (ref tests/libs/test_grxblas.cpp:20,
 * test_grxblas_ex.cpp:16, test_grxblas_l12.cpp:14,
 * tests/bench/gemm_cycles.cpp:29), so it is shipped under the same name.
 * The reference's umbrella also pulls in grx_tensormap.h (GRX-G100 DXA tensor
 * maps); MI355X has no DXA engine and this build ships no tensor-map API, so
 * the umbrella covers the types and the runtime subset that exist here.
 * Plain C99 and C++.
 */
#ifndef GRX_H
#define GRX_H

#include "grx_types.h"
#include "grx_runtime.h"

#endif /* GRX_H */
