// libgrxblas.so -- grxBLAS host library for gfx950.
//
// Keeps the reference's API contract (ref: src/libs/grxblas/grxblas.cpp):
// the same validation order and status codes, calls asynchronous on the
// handle's stream, no silent fallback for an unsupported type pairing. What
// changes is everything under it: there is no .vxbin module to load, no
// shape-query kernel and no DXA descriptor to program -- the gfx950 kernels
// are compiled into this library and launched directly on the HIP stream.

#include <grx/grxblas.h>

#include <hip/hip_runtime_api.h>

#include <dlfcn.h>
#include <limits.h>
#include <stdlib.h>

#include <array>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "hip_status.h"
#include "launch.h"

// Device scratch for transposed operand copies (GemmEx layouts other than
// T,N) and split-K partial sums: one per (device, stream), grown on demand and
// kept until grxblasDestroy. Stream order alone keeps two GEMMs from using
// one workspace at once, so no event is recorded per call (an event record
// costs ~2.5 us of GPU time, 10 % of a small split-K GEMM). A handle that
// meets more than kStreamSlots streams on one device frees the least recently
// used workspace (hipFree waits for the device) and gives it to the new one.
struct GemmWorkspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  hipStream_t stream = nullptr;
  uint64_t tick = 0;                // last use, for eviction
  bool bound = false;               // stream is meaningful (0 is the null stream)
};
constexpr int kStreamSlots = 4;

struct grxblasContext {
  hipStream_t stream = nullptr;
  std::mutex mutex;
  std::array<std::array<GemmWorkspace, kStreamSlots>, 64> ws{};
  uint64_t ws_tick = 0;
  std::string kernel_path;           // set by the first successful kernel lookup
  std::array<signed char, 64> device_ok{};  // per device: 0 unknown, 1 ok, -1 refused
  grxblasStatus_t device_status[64];
  grxCycleSlot* probe = nullptr;
  int probe_capacity = 0;
  int slot_a = 0, slot_b = 1;
};

namespace {

std::mutex g_path_mutex;
std::string g_kernel_path;

// This library's own file: the kernels live in it.
std::string self_path() {
  Dl_info info{};
  if (dladdr((void*)&grxblasCreate, &info) == 0 || !info.dli_fname) return {};
  char buf[PATH_MAX];
  if (!realpath(info.dli_fname, buf)) return info.dli_fname;
  return buf;
}

// Configured source first, with no fallback past it (the reference's rule,
// ref src/libs/grxblas/grxblas.cpp:33-58): a configured directory that is not
// the one holding this library's kernels is an error, not a hint.
grxblasStatus_t ensure_kernels_locked(grxblasContext& ctx) {
  if (!ctx.kernel_path.empty()) return GRXBLAS_STATUS_SUCCESS;
  std::string configured;
  {
    std::lock_guard<std::mutex> lock(g_path_mutex);
    configured = g_kernel_path;
  }
  if (configured.empty()) {
    const char* env = std::getenv("GRXBLAS_KERNEL_PATH");
    if (env) configured = env;
  }
  const std::string self = self_path();
  if (!configured.empty()) {
    const std::string want = configured + "/libgrxblas.so";
    char buf[PATH_MAX];
    const bool same = realpath(want.c_str(), buf) && self == buf;
    if (!same) {
      std::fprintf(stderr,
                   "grxblas: the gfx950 kernels are in %s, not in the configured "
                   "directory %s.\n"
                   "         Point GRXBLAS_KERNEL_PATH / grxblasSetKernelPath at the "
                   "directory holding libgrxblas.so, or unset it.\n",
                   self.c_str(), configured.c_str());
      return GRXBLAS_STATUS_NOT_INITIALIZED;
    }
  }
  ctx.kernel_path = self;
  return GRXBLAS_STATUS_SUCCESS;
}

// The device must be a gfx950: the library carries gfx950 code objects only.
grxblasStatus_t ensure_device_locked(grxblasContext& ctx) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    static bool said = false;
    if (!said) {
      said = true;
      std::fprintf(stderr, "grxblas: no HIP device is available.\n");
    }
    return GRXBLAS_STATUS_ARCH_MISMATCH;
  }
  if (dev >= (int)ctx.device_ok.size()) return GRXBLAS_STATUS_NOT_SUPPORTED;
  if (ctx.device_ok[dev] == 1) return GRXBLAS_STATUS_SUCCESS;
  if (ctx.device_ok[dev] == -1) return ctx.device_status[dev];
  hipDeviceProp_t p;
  grxblasStatus_t st = GRXBLAS_STATUS_SUCCESS;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) {
    st = GRXBLAS_STATUS_INTERNAL_ERROR;
  } else if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0 || p.warpSize != 64) {
    std::fprintf(stderr,
                 "grxblas: this build carries gfx950 kernels (wave64); device %d is %s "
                 "(warp %d).\n",
                 dev, p.gcnArchName, p.warpSize);
    st = GRXBLAS_STATUS_ARCH_MISMATCH;
  }
  ctx.device_ok[dev] = (st == GRXBLAS_STATUS_SUCCESS) ? 1 : -1;
  ctx.device_status[dev] = st;
  return st;
}

grxblasStatus_t ensure_ready(grxblasContext& ctx) {
  std::lock_guard<std::mutex> lock(ctx.mutex);
  grxblasStatus_t s = ensure_kernels_locked(ctx);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;
  return ensure_device_locked(ctx);
}

// HIP errors to grxBLAS status (the role of ref grxblas.cpp:173-182).
grxblasStatus_t from_hip(hipError_t e) {
  switch (grx_from_hip(e)) {
    case grxSuccess:                   return GRXBLAS_STATUS_SUCCESS;
    case grxErrorMemoryAllocation:     return GRXBLAS_STATUS_ALLOC_FAILED;
    case grxErrorInvalidValue:         return GRXBLAS_STATUS_INVALID_VALUE;
    case grxErrorInvalidDevicePointer: return GRXBLAS_STATUS_INVALID_VALUE;
    case grxErrorNotSupported:         return GRXBLAS_STATUS_NOT_SUPPORTED;
    case grxErrorInvalidKernelImage:   return GRXBLAS_STATUS_ARCH_MISMATCH;
    default:                           return GRXBLAS_STATUS_EXECUTION_FAILED;
  }
}

bool integral(float v) {
  return std::isfinite(v) && v >= -2147483648.0f && v < 2147483648.0f &&
         v == (float)(int32_t)v;
}

constexpr unsigned kTypeMask = GRXBLAS_TENSOR_FP16 | GRXBLAS_TENSOR_BF16 | GRXBLAS_TENSOR_INT8;

void say_types_once() {
  static bool said = false;
  if (said) return;
  said = true;
  std::fprintf(stderr,
               "grxblas: grxblasGemmEx accepts (16F,16F,32F), (16F,16F,16F), (16BF,16BF,32F), "
               "(16BF,16BF,16BF)\n         and (8I,8I,32I); int8 to bf16 with a per-column "
               "scale is grxblasGemmExDequant.\n");
}

// Probe slots for a launch: checked against the attached capacity.
grxblasStatus_t probe_for(grxblasContext& ctx, int64_t needed, grxCycleSlot** out) {
  std::lock_guard<std::mutex> lock(ctx.mutex);
  *out = nullptr;
  if (!ctx.probe) return GRXBLAS_STATUS_SUCCESS;
  if ((int64_t)ctx.probe_capacity < needed) return GRXBLAS_STATUS_INVALID_VALUE;
  *out = ctx.probe;
  return GRXBLAS_STATUS_SUCCESS;
}

// Give d the workspace of (current device, stream) if the launch wants one
// (else the launch takes a path that needs none). Called with ctx.mutex held.
hipError_t attach_workspace_locked(grxblasContext& ctx, grxk::MmaIn in, grxk::MmaOut out,
                                   grxk::GemmDesc& d, hipStream_t stream) {
  const size_t need = grxk::gemm_workspace_bytes(in, out, d);
  if (need == 0) return hipSuccess;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= (int)ctx.ws.size()) return hipSuccess;
  auto& slots = ctx.ws[dev];
  GemmWorkspace* w = nullptr;
  for (GemmWorkspace& c : slots)
    if (c.bound && c.stream == stream) w = &c;
  if (!w) {
    for (GemmWorkspace& c : slots)
      if (!w || !c.bound || (w->bound && c.tick < w->tick)) w = &c;
    if (w->ptr) {
      // hipFree waits for the device, so no GEMM on the old stream still uses it.
      (void)hipFree(w->ptr);
      w->ptr = nullptr;
      w->bytes = 0;
    }
    w->stream = stream;
    w->bound = true;
  }
  w->tick = ++ctx.ws_tick;
  if (w->bytes < need) {
    if (w->ptr) {
      (void)hipFree(w->ptr);
      w->ptr = nullptr;
      w->bytes = 0;
    }
    if (hipMalloc(&w->ptr, need) != hipSuccess) {
      (void)hipGetLastError();
      w->ptr = nullptr;
      return hipSuccess;  // no workspace: a path that needs none
    }
    w->bytes = need;
  }
  d.ws = w->ptr;
  d.ws_bytes = w->bytes;
  return hipSuccess;
}

// One GemmEx-family launch with the workspace attached as needed. The lock
// spans attach and launch, so another thread on this handle cannot free or
// regrow the workspace between the two.
grxblasStatus_t launch_gemm(grxblasContext& ctx, grxk::MmaIn in, grxk::MmaOut out,
                            grxk::GemmDesc& d) {
  std::lock_guard<std::mutex> lock(ctx.mutex);
  hipError_t e = attach_workspace_locked(ctx, in, out, d, ctx.stream);
  if (e == hipSuccess) e = grxk::launch_mma_gemm(in, out, d, ctx.stream);
  return from_hip(e);
}

// The allocation-free form: the same plan with the library's static
// per-device scratch (grxk::NoAllocScratch) in place of the handle's
// workspace. Calls no hipMalloc/hipFree; a plan that needs more scratch
// than the array holds is refused before anything is launched. A plan that
// uses the scratch holds the device's scratch lock from before its launch
// until the launch is recorded, so calls on other streams wait for it.
grxblasStatus_t launch_gemm_noalloc(grxblasContext& ctx, grxk::MmaIn in, grxk::MmaOut out,
                                    grxk::GemmDesc& d) {
  size_t need = grxk::gemm_workspace_bytes(in, out, d);
  if (need > grxk::kNoAllocScratchBytes) {
    // Padded copies of both operands (K not a multiple of 16 bytes) or a
    // staged C that do not fit the scratch: the plan without them (the
    // general path).
    d.pad_copies = false;
    need = grxk::gemm_workspace_bytes(in, out, d);
  }
  if (need > grxk::kNoAllocScratchBytes) {
    std::fprintf(stderr,
                 "grxblas: grxblasGemmExNoAlloc: this problem needs %zu bytes of scratch "
                 "(operand copies / split-K partials), more than the %zu bytes the library "
                 "holds per device; call grxblasGemmEx instead.\n",
                 need, grxk::kNoAllocScratchBytes);
    return GRXBLAS_STATUS_NOT_SUPPORTED;
  }
  if (need == 0) return from_hip(grxk::launch_mma_gemm(in, out, d, ctx.stream));
  grxk::NoAllocScratch scratch(ctx.stream);
  if (!scratch.ptr()) return GRXBLAS_STATUS_INTERNAL_ERROR;
  d.ws = scratch.ptr();
  d.ws_bytes = grxk::kNoAllocScratchBytes;
  const hipError_t e = grxk::launch_mma_gemm(in, out, d, ctx.stream);
  const hipError_t r = scratch.release(e == hipSuccess);
  return from_hip(e != hipSuccess ? e : r);
}

// GemmEx and its strided batch. Validation order of ref
// src/libs/grxblas/grxblas.cpp:507-524, the batch count checked where
// SgemmStridedBatched checks it. no_alloc: grxblasGemmExNoAlloc.
grxblasStatus_t gemm_ex_batched(grxblasHandle_t handle, grxblasOperation_t transa,
                                grxblasOperation_t transb, int m, int n, int k,
                                const float* alpha, const void* A, grxDataType_t Atype, int lda,
                                long long strideA, const void* B, grxDataType_t Btype, int ldb,
                                long long strideB, const float* beta, void* C,
                                grxDataType_t Ctype, int ldc, long long strideC, int batch,
                                bool no_alloc = false) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha || !beta) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m < 0 || n < 0 || k < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (batch < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m == 0 || n == 0 || batch == 0) return GRXBLAS_STATUS_SUCCESS;
  if (k > 0 && (!A || !B)) return GRXBLAS_STATUS_INVALID_VALUE;
  if (!C) return GRXBLAS_STATUS_INVALID_VALUE;
  const bool ta = (transa == GRXBLAS_OP_T);
  const bool tb = (transb == GRXBLAS_OP_T);
  if (lda < (ta ? k : m) || ldb < (tb ? n : k) || ldc < m) return GRXBLAS_STATUS_INVALID_VALUE;
  if (batch > 65535) return GRXBLAS_STATUS_NOT_SUPPORTED;

  const grxblasStatus_t s = ensure_ready(*handle);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;

  // Type pairing after the device is known (ref grxblas.cpp:552-575).
  grxk::MmaIn in;
  grxk::MmaOut out;
  if (Atype == GRX_R_16F && Btype == GRX_R_16F && Ctype == GRX_R_32F) {
    in = grxk::MmaIn::F16; out = grxk::MmaOut::F32;
  } else if (Atype == GRX_R_16F && Btype == GRX_R_16F && Ctype == GRX_R_16F) {
    in = grxk::MmaIn::F16; out = grxk::MmaOut::F16;
  } else if (Atype == GRX_R_16BF && Btype == GRX_R_16BF && Ctype == GRX_R_32F) {
    in = grxk::MmaIn::BF16; out = grxk::MmaOut::F32;
  } else if (Atype == GRX_R_16BF && Btype == GRX_R_16BF && Ctype == GRX_R_16BF) {
    in = grxk::MmaIn::BF16; out = grxk::MmaOut::BF16;
  } else if (Atype == GRX_R_8I && Btype == GRX_R_8I && Ctype == GRX_R_32I) {
    in = grxk::MmaIn::I8; out = grxk::MmaOut::I32;
  } else {
    say_types_once();
    return GRXBLAS_STATUS_NOT_SUPPORTED;
  }
  // Integral alpha/beta for the int8 pairing (ref grxblas.cpp:577-584).
  if (in == grxk::MmaIn::I8 && (!integral(*alpha) || !integral(*beta)))
    return GRXBLAS_STATUS_INVALID_VALUE;

  grxCycleSlot* probe = nullptr;
  const grxblasStatus_t ps =
      probe_for(*handle, grxk::gemm_probe_slots(m, n) * (int64_t)batch, &probe);
  if (ps != GRXBLAS_STATUS_SUCCESS) return ps;

  grxk::GemmDesc d{};
  d.m = m; d.n = n; d.k = k;
  d.ta = ta; d.tb = tb;
  d.a = A; d.lda = lda;
  d.b = B; d.ldb = ldb;
  d.c = C; d.ldc = ldc;
  d.alpha = *alpha; d.beta = *beta;
  if (in == grxk::MmaIn::I8) { d.ialpha = (int32_t)*alpha; d.ibeta = (int32_t)*beta; }
  d.probe = probe;
  d.batch = batch;
  d.stride_a = strideA; d.stride_b = strideB; d.stride_c = strideC;
  if (no_alloc) return launch_gemm_noalloc(*handle, in, out, d);
  return launch_gemm(*handle, in, out, d);
}

}  // namespace

// The C API is the only thing these libraries export (built with
// -fvisibility=hidden).
#pragma GCC visibility push(default)
extern "C" {

const char* grxblasGetStatusString(grxblasStatus_t s) {
  switch (s) {
    case GRXBLAS_STATUS_SUCCESS:          return "success";
    case GRXBLAS_STATUS_NOT_INITIALIZED:  return "library not initialized (kernels not found?)";
    case GRXBLAS_STATUS_ALLOC_FAILED:     return "allocation failed";
    case GRXBLAS_STATUS_INVALID_VALUE:    return "invalid argument";
    case GRXBLAS_STATUS_ARCH_MISMATCH:    return "device lacks a required capability";
    case GRXBLAS_STATUS_EXECUTION_FAILED: return "kernel execution failed";
    case GRXBLAS_STATUS_NOT_SUPPORTED:    return "not supported";
    case GRXBLAS_STATUS_INTERNAL_ERROR:   return "internal error";
  }
  return "unknown status";
}

grxblasStatus_t grxblasCreate(grxblasHandle_t* handle) {
  if (!handle) return GRXBLAS_STATUS_INVALID_VALUE;
  *handle = new (std::nothrow) grxblasContext();
  return *handle ? GRXBLAS_STATUS_SUCCESS : GRXBLAS_STATUS_ALLOC_FAILED;
}

grxblasStatus_t grxblasDestroy(grxblasHandle_t handle) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  int cur = 0;
  const bool have_cur = hipGetDevice(&cur) == hipSuccess;
  for (int dev = 0; dev < (int)handle->ws.size(); ++dev) {
    for (GemmWorkspace& w : handle->ws[dev]) {
      if (!w.ptr) continue;
      if (hipSetDevice(dev) != hipSuccess) break;
      (void)hipFree(w.ptr);  // waits for the GEMMs that read it
    }
  }
  if (have_cur) (void)hipSetDevice(cur);
  delete handle;
  return GRXBLAS_STATUS_SUCCESS;
}

grxblasStatus_t grxblasSetStream(grxblasHandle_t handle, grxStream_t stream) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  handle->stream = reinterpret_cast<hipStream_t>(stream);
  return GRXBLAS_STATUS_SUCCESS;
}

grxblasStatus_t grxblasGetStream(grxblasHandle_t handle, grxStream_t* stream) {
  if (!handle || !stream) return GRXBLAS_STATUS_INVALID_VALUE;
  *stream = reinterpret_cast<grxStream_t>(handle->stream);
  return GRXBLAS_STATUS_SUCCESS;
}

grxblasStatus_t grxblasSetKernelPath(const char* path) {
  std::lock_guard<std::mutex> lock(g_path_mutex);
  g_kernel_path = path ? path : "";
  return GRXBLAS_STATUS_SUCCESS;
}

grxblasStatus_t grxblasSetTensorMapSlots(grxblasHandle_t handle, int slotA, int slotB) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (slotA < 0 || slotB < 0 || slotA == slotB) return GRXBLAS_STATUS_INVALID_VALUE;
  std::lock_guard<std::mutex> lock(handle->mutex);
  handle->slot_a = slotA;
  handle->slot_b = slotB;
  return GRXBLAS_STATUS_SUCCESS;
}

grxblasStatus_t grxblasGetTensorTypes(grxblasHandle_t handle, unsigned* typeMask) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!typeMask) return GRXBLAS_STATUS_INVALID_VALUE;
  const grxblasStatus_t s = ensure_ready(*handle);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;
  *typeMask = kTypeMask;
  return GRXBLAS_STATUS_SUCCESS;
}

grxblasStatus_t grxblasGetTensorTile(grxblasHandle_t handle, int* m, int* n, int* k) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!m || !n || !k) return GRXBLAS_STATUS_INVALID_VALUE;
  const grxblasStatus_t s = ensure_ready(*handle);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;
  *m = 32;
  *n = 32;
  *k = 16;
  return GRXBLAS_STATUS_SUCCESS;
}

grxblasStatus_t grxblasGemmEx(grxblasHandle_t handle, grxblasOperation_t transa,
                              grxblasOperation_t transb, int m, int n, int k,
                              const float* alpha, const void* A, grxDataType_t Atype, int lda,
                              const void* B, grxDataType_t Btype, int ldb, const float* beta,
                              void* C, grxDataType_t Ctype, int ldc) {
  return gemm_ex_batched(handle, transa, transb, m, n, k, alpha, A, Atype, lda, 0, B, Btype,
                         ldb, 0, beta, C, Ctype, ldc, 0, 1);
}

grxblasStatus_t grxblasGemmExNoAlloc(grxblasHandle_t handle, grxblasOperation_t transa,
                                     grxblasOperation_t transb, int m, int n, int k,
                                     const float* alpha, const void* A, grxDataType_t Atype,
                                     int lda, const void* B, grxDataType_t Btype, int ldb,
                                     const float* beta, void* C, grxDataType_t Ctype, int ldc) {
  return gemm_ex_batched(handle, transa, transb, m, n, k, alpha, A, Atype, lda, 0, B, Btype,
                         ldb, 0, beta, C, Ctype, ldc, 0, 1, true);
}

grxblasStatus_t grxblasGemmStridedBatchedEx(grxblasHandle_t handle, grxblasOperation_t transa,
                                            grxblasOperation_t transb, int m, int n, int k,
                                            const float* alpha, const void* A,
                                            grxDataType_t Atype, int lda, long long strideA,
                                            const void* B, grxDataType_t Btype, int ldb,
                                            long long strideB, const float* beta, void* C,
                                            grxDataType_t Ctype, int ldc, long long strideC,
                                            int batchCount) {
  return gemm_ex_batched(handle, transa, transb, m, n, k, alpha, A, Atype, lda, strideA, B,
                         Btype, ldb, strideB, beta, C, Ctype, ldc, strideC, batchCount);
}

grxblasStatus_t grxblasGemmExDequant(grxblasHandle_t handle, grxblasOperation_t transa,
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
  const bool ta = (transa == GRXBLAS_OP_T);
  const bool tb = (transb == GRXBLAS_OP_T);
  if (lda < (ta ? k : m) || ldb < (tb ? n : k) || ldc < m) return GRXBLAS_STATUS_INVALID_VALUE;

  const grxblasStatus_t s = ensure_ready(*handle);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;
  if (!(Atype == GRX_R_8I && Btype == GRX_R_8I && Ctype == GRX_R_16BF)) {
    static bool said = false;
    if (!said) {
      said = true;
      std::fprintf(stderr, "grxblas: grxblasGemmExDequant takes (8I, 8I, 16BF) only.\n");
    }
    return GRXBLAS_STATUS_NOT_SUPPORTED;
  }
  grxCycleSlot* probe = nullptr;
  const grxblasStatus_t ps = probe_for(*handle, grxk::gemm_probe_slots(m, n), &probe);
  if (ps != GRXBLAS_STATUS_SUCCESS) return ps;

  grxk::GemmDesc d{};
  d.m = m; d.n = n; d.k = k;
  d.ta = ta; d.tb = tb;
  d.a = A; d.lda = lda;
  d.b = B; d.ldb = ldb;
  d.c = C; d.ldc = ldc;
  d.scale = scaleN;
  d.probe = probe;
  return launch_gemm(*handle, grxk::MmaIn::I8, grxk::MmaOut::DEQ_BF16, d);
}

grxblasStatus_t grxblasSetCycleProbe(grxblasHandle_t handle, grxCycleSlot* slots, int capacity) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (slots && capacity <= 0) return GRXBLAS_STATUS_INVALID_VALUE;
  std::lock_guard<std::mutex> lock(handle->mutex);
  handle->probe = slots;
  handle->probe_capacity = slots ? capacity : 0;
  return GRXBLAS_STATUS_SUCCESS;
}

int grxblasCycleSlotsNeeded(grxblasHandle_t handle, int m, int n) {
  (void)handle;
  const int64_t s = grxk::gemm_probe_slots(m, n);
  return s > INT_MAX ? INT_MAX : (int)s;
}

grxblasStatus_t grxblasGetLoadedKernelPath(grxblasHandle_t handle, const char** path) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!path) return GRXBLAS_STATUS_INVALID_VALUE;
  std::lock_guard<std::mutex> lock(handle->mutex);
  *path = handle->kernel_path.empty() ? nullptr : handle->kernel_path.c_str();
  return GRXBLAS_STATUS_SUCCESS;
}

// ---- level 1 / 2 (ref grxblas.cpp:736-865) ---------------------------------

grxblasStatus_t grxblasSaxpy(grxblasHandle_t handle, int n, const float* alpha, const float* x,
                             int incx, float* y, int incy) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha) return GRXBLAS_STATUS_INVALID_VALUE;
  if (n < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (n == 0) return GRXBLAS_STATUS_SUCCESS;
  if (!x || !y) return GRXBLAS_STATUS_INVALID_VALUE;
  if (incx == 0 || incy == 0) return GRXBLAS_STATUS_INVALID_VALUE;
  const grxblasStatus_t s = ensure_ready(*handle);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;
  grxCycleSlot* probe = nullptr;
  const grxblasStatus_t ps = probe_for(*handle, 4 * grxk::l1_blocks(n), &probe);
  if (ps != GRXBLAS_STATUS_SUCCESS) return ps;
  return from_hip(grxk::launch_saxpy(n, *alpha, x, incx, y, incy, probe, handle->stream));
}

grxblasStatus_t grxblasSscal(grxblasHandle_t handle, int n, const float* alpha, float* x,
                             int incx) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha) return GRXBLAS_STATUS_INVALID_VALUE;
  if (n < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (n == 0) return GRXBLAS_STATUS_SUCCESS;
  if (!x) return GRXBLAS_STATUS_INVALID_VALUE;
  if (incx <= 0) return GRXBLAS_STATUS_INVALID_VALUE;
  const grxblasStatus_t s = ensure_ready(*handle);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;
  grxCycleSlot* probe = nullptr;
  const grxblasStatus_t ps = probe_for(*handle, 4 * grxk::l1_blocks(n), &probe);
  if (ps != GRXBLAS_STATUS_SUCCESS) return ps;
  return from_hip(grxk::launch_sscal(n, *alpha, x, incx, probe, handle->stream));
}

grxblasStatus_t grxblasSgemv(grxblasHandle_t handle, grxblasOperation_t trans, int m, int n,
                             const float* alpha, const void* A, int lda, const void* x,
                             int incx, const float* beta, void* y, int incy) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha || !beta) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m < 0 || n < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m == 0 || n == 0) return GRXBLAS_STATUS_SUCCESS;
  if (!A || !x || !y) return GRXBLAS_STATUS_INVALID_VALUE;
  if (incx == 0 || incy == 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (lda < m) return GRXBLAS_STATUS_INVALID_VALUE;
  const grxblasStatus_t s = ensure_ready(*handle);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;
  grxCycleSlot* probe = nullptr;
  const grxblasStatus_t ps =
      probe_for(*handle, 4 * grxk::sgemv_blocks(trans == GRXBLAS_OP_T, m, n), &probe);
  if (ps != GRXBLAS_STATUS_SUCCESS) return ps;
  return from_hip(grxk::launch_sgemv(trans == GRXBLAS_OP_T, m, n, *alpha, (const float*)A, lda,
                                     (const float*)x, incx, *beta, (float*)y, incy, probe,
                                     handle->stream));
}

// ---- Sgemm / SgemmStridedBatched: one body (ref grxblas.cpp:867-963) --------

static grxblasStatus_t sgemm_batched(grxblasHandle_t handle, grxblasOperation_t transa,
                                     grxblasOperation_t transb, int m, int n, int k,
                                     const float* alpha, const void* A, int lda,
                                     long long strideA, const void* B, int ldb,
                                     long long strideB, const float* beta, void* C, int ldc,
                                     long long strideC, int batch) {
  if (!handle) return GRXBLAS_STATUS_NOT_INITIALIZED;
  if (!alpha || !beta) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m < 0 || n < 0 || k < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (batch < 0) return GRXBLAS_STATUS_INVALID_VALUE;
  if (m == 0 || n == 0 || batch == 0) return GRXBLAS_STATUS_SUCCESS;
  if (k > 0 && (!A || !B)) return GRXBLAS_STATUS_INVALID_VALUE;
  if (!C) return GRXBLAS_STATUS_INVALID_VALUE;
  const int min_lda = (transa == GRXBLAS_OP_N) ? m : k;
  const int min_ldb = (transb == GRXBLAS_OP_N) ? k : n;
  if (lda < min_lda || ldb < min_ldb || ldc < m) return GRXBLAS_STATUS_INVALID_VALUE;
  if (batch > 65535) return GRXBLAS_STATUS_NOT_SUPPORTED;

  const grxblasStatus_t s = ensure_ready(*handle);
  if (s != GRXBLAS_STATUS_SUCCESS) return s;

  grxCycleSlot* probe = nullptr;
  const grxblasStatus_t ps =
      probe_for(*handle, grxk::gemm_probe_slots(m, n) * (int64_t)batch, &probe);
  if (ps != GRXBLAS_STATUS_SUCCESS) return ps;

  grxk::SgemmDesc d{};
  d.m = m; d.n = n; d.k = k; d.batch = batch;
  d.ta = (transa == GRXBLAS_OP_T);
  d.tb = (transb == GRXBLAS_OP_T);
  d.a = (const float*)A; d.lda = lda; d.stride_a = strideA;
  d.b = (const float*)B; d.ldb = ldb; d.stride_b = strideB;
  d.c = (float*)C; d.ldc = ldc; d.stride_c = strideC;
  d.alpha = *alpha; d.beta = *beta;
  d.probe = probe;
  if (!probe) {
    // Problems that fill the GPU with 256x256 tiles run the GemmEx TN kernel
    // on fp32 (behind K-contiguous copies for other layouts) when its
    // workspace is there; the rest, and calls with a cycle probe, sgemm_mfma.
    grxk::GemmDesc g{};
    g.m = m; g.n = n; g.k = k; g.batch = batch;
    g.ta = d.ta; g.tb = d.tb;
    g.a = A; g.lda = lda; g.stride_a = strideA;
    g.b = B; g.ldb = ldb; g.stride_b = strideB;
    g.c = C; g.ldc = ldc; g.stride_c = strideC;
    g.alpha = *alpha; g.beta = *beta;
    if (grxk::fp32_mma_wanted(g)) {
      std::lock_guard<std::mutex> lock(handle->mutex);
      hipError_t e = attach_workspace_locked(*handle, grxk::MmaIn::F32, grxk::MmaOut::F32, g,
                                             handle->stream);
      if (e == hipSuccess &&
          grxk::gemm_workspace_bytes(grxk::MmaIn::F32, grxk::MmaOut::F32, g) <= g.ws_bytes)
        return from_hip(grxk::launch_mma_gemm(grxk::MmaIn::F32, grxk::MmaOut::F32, g,
                                              handle->stream));
    }
  }
  return from_hip(grxk::launch_sgemm(d, handle->stream));
}

grxblasStatus_t grxblasSgemm(grxblasHandle_t handle, grxblasOperation_t transa,
                             grxblasOperation_t transb, int m, int n, int k, const float* alpha,
                             const void* A, int lda, const void* B, int ldb, const float* beta,
                             void* C, int ldc) {
  return sgemm_batched(handle, transa, transb, m, n, k, alpha, A, lda, 0, B, ldb, 0, beta, C,
                       ldc, 0, 1);
}

grxblasStatus_t grxblasSgemmStridedBatched(grxblasHandle_t handle, grxblasOperation_t transa,
                                           grxblasOperation_t transb, int m, int n, int k,
                                           const float* alpha, const void* A, int lda,
                                           long long strideA, const void* B, int ldb,
                                           long long strideB, const float* beta, void* C,
                                           int ldc, long long strideC, int batchCount) {
  return sgemm_batched(handle, transa, transb, m, n, k, alpha, A, lda, strideA, B, ldb, strideB,
                       beta, C, ldc, strideC, batchCount);
}

}  // extern "C"
#pragma GCC visibility pop
