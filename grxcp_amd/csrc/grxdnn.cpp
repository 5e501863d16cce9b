// libgrxdnn.so -- grxDNN host library for gfx950.
//
// The reference plans grxDNN (ref: src/libs/CMakeLists.txt:12,
// docs/designs/grxcp_architecture.md:594,640, docs/designs/grxcp_roadmap.md:
// 864-877) but ships no code, so this library follows grxBLAS's host
// conventions (ref: src/libs/grxblas/grxblas.cpp): an opaque handle with a
// borrowed stream, every argument validated before any device work, the same
// status values, NOT_SUPPORTED instead of a silent fallback, asynchronous
// launches on the handle's stream.

#include <grx/grxdnn.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>

#include "hip_status.h"
#include "launch.h"

struct grxdnnContext {
  hipStream_t stream = nullptr;
  grxCycleSlot* probe = nullptr;
  int probe_capacity = 0;
  std::mutex mutex;
  std::array<signed char, 64> device_ok{};
  grxdnnStatus_t device_status[64];
};

struct grxdnnTensorStruct {
  bool set = false;
  grxDataType_t type = GRX_R_32F;
  int nb = 0;
  int dims[GRXDNN_DIM_MAX] = {0};
  int strides[GRXDNN_DIM_MAX] = {0};
};

struct grxdnnAttentionStruct {
  bool set = false;
  int causal = 0;
  float scale = 1.0f;
};

namespace {

grxdnnStatus_t ensure_device(grxdnnContext& ctx) {
  std::lock_guard<std::mutex> lock(ctx.mutex);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    static bool said = false;
    if (!said) {
      said = true;
      std::fprintf(stderr, "grxdnn: no HIP device is available.\n");
    }
    return GRXDNN_STATUS_ARCH_MISMATCH;
  }
  if (dev >= (int)ctx.device_ok.size()) return GRXDNN_STATUS_NOT_SUPPORTED;
  if (ctx.device_ok[dev] == 1) return GRXDNN_STATUS_SUCCESS;
  if (ctx.device_ok[dev] == -1) return ctx.device_status[dev];
  hipDeviceProp_t p;
  grxdnnStatus_t st = GRXDNN_STATUS_SUCCESS;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) {
    st = GRXDNN_STATUS_INTERNAL_ERROR;
  } else if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0 || p.warpSize != 64) {
    std::fprintf(stderr, "grxdnn: this build carries gfx950 kernels; device %d is %s.\n", dev,
                 p.gcnArchName);
    st = GRXDNN_STATUS_ARCH_MISMATCH;
  }
  ctx.device_ok[dev] = (st == GRXDNN_STATUS_SUCCESS) ? 1 : -1;
  ctx.device_status[dev] = st;
  return st;
}

grxdnnStatus_t from_hip(hipError_t e) {
  switch (grx_from_hip(e)) {
    case grxSuccess:                   return GRXDNN_STATUS_SUCCESS;
    case grxErrorMemoryAllocation:     return GRXDNN_STATUS_ALLOC_FAILED;
    case grxErrorInvalidValue:         return GRXDNN_STATUS_INVALID_VALUE;
    case grxErrorInvalidDevicePointer: return GRXDNN_STATUS_INVALID_VALUE;
    case grxErrorNotSupported:         return GRXDNN_STATUS_NOT_SUPPORTED;
    case grxErrorInvalidKernelImage:   return GRXDNN_STATUS_ARCH_MISMATCH;
    default:                           return GRXDNN_STATUS_EXECUTION_FAILED;
  }
}

bool known_type(grxDataType_t t) {
  return t == GRX_R_32F || t == GRX_R_16F || t == GRX_R_8I || t == GRX_R_32I || t == GRX_R_16BF;
}

bool same_shape(const grxdnnTensorStruct& a, const grxdnnTensorStruct& b) {
  if (a.nb != b.nb) return false;
  for (int i = 0; i < a.nb; ++i)
    if (a.dims[i] != b.dims[i]) return false;
  return true;
}

// Rows of a [..., hidden] tensor: all leading dimensions must collapse into
// one row index with a single pitch. Returns false if they do not.
bool row_layout(const grxdnnTensorStruct& t, int64_t* rows, int64_t* pitch) {
  const int nb = t.nb;
  const int hidden = t.dims[nb - 1];
  if (nb == 1) { *rows = 1; *pitch = hidden; return true; }
  int64_t r = 1;
  for (int i = 0; i < nb - 1; ++i) r *= t.dims[i];
  *rows = r;
  *pitch = t.strides[nb - 2];
  if (*pitch < hidden) return r <= 1;
  for (int i = 0; i < nb - 2; ++i)
    if (t.dims[i + 1] > 1 && (int64_t)t.strides[i] != (int64_t)t.strides[i + 1] * t.dims[i + 1])
      return false;
  return true;
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

// No two elements of an output share an address: taken in increasing stride
// order (dimensions of extent 1 aside), each stride covers the extent of the
// dimensions below it. An input may overlap itself (a broadcast); an output
// that did would be written by several threads.
bool no_overlap(const grxdnnTensorStruct& t) {
  int idx[GRXDNN_DIM_MAX];
  int n = 0;
  for (int i = 0; i < t.nb; ++i)
    if (t.dims[i] > 1) idx[n++] = i;
  for (int a = 1; a < n; ++a)
    for (int b = a; b > 0 && t.strides[idx[b]] < t.strides[idx[b - 1]]; --b) {
      const int x = idx[b];
      idx[b] = idx[b - 1];
      idx[b - 1] = x;
    }
  int64_t extent = 1;
  for (int j = 0; j < n; ++j) {
    const int i = idx[j];
    if ((int64_t)t.strides[i] < extent) return false;
    extent = (int64_t)t.strides[i] * t.dims[i];
  }
  return true;
}

// Byte interval [lo, hi) covered by a tensor at p (strides are non-negative).
struct Span { uintptr_t lo, hi; };
Span span_of(const grxdnnTensorStruct& t, const void* p, size_t elem) {
  int64_t last = 0;
  for (int i = 0; i < t.nb; ++i)
    if (t.dims[i] > 0) last += (int64_t)t.strides[i] * (t.dims[i] - 1);
  const uintptr_t lo = (uintptr_t)p;
  return {lo, lo + (uintptr_t)((last + 1) * (int64_t)elem)};
}
bool intersect(Span a, Span b) { return a.lo < b.hi && b.lo < a.hi; }

bool same_strides(const grxdnnTensorStruct& a, const grxdnnTensorStruct& b) {
  for (int i = 0; i < a.nb; ++i)
    if (a.strides[i] != b.strides[i]) return false;
  return true;
}

// Whether delta = sum_i strides[i] * d_i has a solution with |d_i| <
// extents[i], for dimensions taken in decreasing stride order from `from`;
// reach[i] is the largest |sum| the dimensions after i can make. Returns
// true ("may share an element") when the search would take too many steps.
bool offset_reachable(const int64_t* strides, const int64_t* extents, const int64_t* reach,
                      int n, int from, int64_t delta, int* budget) {
  if (from == n) return delta == 0;
  const int64_t s = strides[from], r = reach[from], e = extents[from] - 1;
  // d with |delta - s*d| <= r: d in [ceil((delta-r)/s), floor((delta+r)/s)]
  auto floor_div = [](int64_t a, int64_t b) { return a >= 0 ? a / b : -((-a + b - 1) / b); };
  int64_t lo = -floor_div(-(delta - r), s), hi = floor_div(delta + r, s);
  if (lo < -e) lo = -e;
  if (hi > e) hi = e;
  for (int64_t d = lo; d <= hi; ++d) {
    if (--*budget < 0) return true;
    if (offset_reachable(strides, extents, reach, n, from + 1, delta - s * d, budget)) return true;
  }
  return false;
}

// Two views of one shape and the same strides (bases a and b, elements of
// `elem` bytes) share an element's address. An exact test of the element
// offsets, so that e.g. O written over the Q slot of a packed [B,S,3,H,D]
// QKV buffer is told apart from O overlapping K or V. Views whose bases do
// not differ by whole elements are taken to overlap when their spans do.
bool views_share_element(const grxdnnTensorStruct& t, const void* a, const void* b, size_t elem) {
  const int64_t diff = (int64_t)((intptr_t)b - (intptr_t)a);
  if (diff % (int64_t)elem != 0) return intersect(span_of(t, a, elem), span_of(t, b, elem));
  int64_t strides[GRXDNN_DIM_MAX], extents[GRXDNN_DIM_MAX], reach[GRXDNN_DIM_MAX];
  int n = 0;
  for (int i = 0; i < t.nb; ++i) {
    if (t.dims[i] <= 0) return false;                      // an empty view
    if (t.dims[i] == 1 || t.strides[i] == 0) continue;     // contributes no offset
    strides[n] = t.strides[i];
    extents[n] = t.dims[i];
    ++n;
  }
  for (int x = 1; x < n; ++x)                              // decreasing stride
    for (int y = x; y > 0 && strides[y] > strides[y - 1]; --y) {
      std::swap(strides[y], strides[y - 1]);
      std::swap(extents[y], extents[y - 1]);
    }
  int64_t acc = 0;
  for (int i = n - 1; i >= 0; --i) {
    reach[i] = acc;
    acc += strides[i] * (extents[i] - 1);
  }
  int budget = 4096;
  return offset_reachable(strides, extents, reach, n, 0, diff / (int64_t)elem, &budget);
}

// O may share no element with x: the exact test where the two views have the
// same strides, the span test otherwise.
bool may_alias(const grxdnnTensorStruct& od, const void* o, const grxdnnTensorStruct& xd,
               const void* x) {
  if (same_strides(od, xd)) return views_share_element(od, o, x, 2);
  return intersect(span_of(od, o, 2), span_of(xd, x, 2));
}

grxdnnStatus_t norm_common(grxdnnHandle_t handle, grxdnnTensorDescriptor_t xDesc, const void* x,
                           grxdnnTensorDescriptor_t wDesc, const void* gamma, const void* beta,
                           bool layer, float eps, grxdnnTensorDescriptor_t yDesc, void* y) {
  if (!handle) return GRXDNN_STATUS_NOT_INITIALIZED;
  if (!xDesc || !wDesc || !yDesc) return GRXDNN_STATUS_INVALID_VALUE;
  if (!xDesc->set || !wDesc->set || !yDesc->set) return GRXDNN_STATUS_INVALID_VALUE;
  if (!same_shape(*xDesc, *yDesc)) return GRXDNN_STATUS_INVALID_VALUE;
  const int hidden = xDesc->dims[xDesc->nb - 1];
  if (wDesc->nb != 1 || wDesc->dims[0] != hidden) return GRXDNN_STATUS_INVALID_VALUE;
  if (!std::isfinite(eps) || eps < 0.0f) return GRXDNN_STATUS_INVALID_VALUE;
  if (xDesc->type != yDesc->type || xDesc->type != wDesc->type) return GRXDNN_STATUS_NOT_SUPPORTED;
  grxk::NormType nt;
  switch (xDesc->type) {
    case GRX_R_16BF: nt = grxk::NormType::BF16; break;
    case GRX_R_16F:  nt = grxk::NormType::F16; break;
    case GRX_R_32F:  nt = grxk::NormType::F32; break;
    default: return GRXDNN_STATUS_NOT_SUPPORTED;
  }
  int64_t rows = 0, xp = 0, yp = 0, yrows = 0;
  for (int i = 0; i < xDesc->nb - 1; ++i)
    if (xDesc->dims[i] == 0) return GRXDNN_STATUS_SUCCESS;  // no rows: nothing to do
  if (hidden <= 0) return GRXDNN_STATUS_INVALID_VALUE;
  if (hidden > 65536) return GRXDNN_STATUS_NOT_SUPPORTED;
  if (xDesc->strides[xDesc->nb - 1] != 1 || yDesc->strides[yDesc->nb - 1] != 1 ||
      wDesc->strides[0] != 1)
    return GRXDNN_STATUS_NOT_SUPPORTED;
  if (!row_layout(*xDesc, &rows, &xp) || !row_layout(*yDesc, &yrows, &yp))
    return GRXDNN_STATUS_NOT_SUPPORTED;
  if (!x || !gamma || !y || (layer && !beta)) return GRXDNN_STATUS_INVALID_VALUE;

  const grxdnnStatus_t s = ensure_device(*handle);
  if (s != GRXDNN_STATUS_SUCCESS) return s;

  grxk::NormDesc d{};
  d.rows = rows;
  d.hidden = hidden;
  d.x_row_stride = xp;
  d.y_row_stride = yp;
  d.x = x; d.gamma = gamma; d.beta = beta; d.y = y;
  d.eps = eps;
  const hipError_t e = layer ? grxk::launch_layernorm(nt, d, handle->stream)
                             : grxk::launch_rmsnorm(nt, d, handle->stream);
  return from_hip(e);
}

// Softmax / GELU: x and y of one type and shape, rows flattening to one
// stride each, innermost stride 1.
grxdnnStatus_t row_common(grxdnnHandle_t handle, grxdnnTensorDescriptor_t xDesc, const void* x,
                          grxdnnTensorDescriptor_t yDesc, void* y, grxk::NormType* nt,
                          grxk::RowDesc* d, bool* empty) {
  *empty = false;
  if (!handle) return GRXDNN_STATUS_NOT_INITIALIZED;
  if (!xDesc || !yDesc || !xDesc->set || !yDesc->set) return GRXDNN_STATUS_INVALID_VALUE;
  if (!same_shape(*xDesc, *yDesc)) return GRXDNN_STATUS_INVALID_VALUE;
  if (xDesc->type != yDesc->type) return GRXDNN_STATUS_NOT_SUPPORTED;
  switch (xDesc->type) {
    case GRX_R_16BF: *nt = grxk::NormType::BF16; break;
    case GRX_R_16F:  *nt = grxk::NormType::F16; break;
    case GRX_R_32F:  *nt = grxk::NormType::F32; break;
    default: return GRXDNN_STATUS_NOT_SUPPORTED;
  }
  for (int i = 0; i < xDesc->nb - 1; ++i)
    if (xDesc->dims[i] == 0) {  // no rows: nothing to do
      *empty = true;
      return GRXDNN_STATUS_SUCCESS;
    }
  const int hidden = xDesc->dims[xDesc->nb - 1];
  if (hidden <= 0) return GRXDNN_STATUS_INVALID_VALUE;
  if (hidden > (1 << 24)) return GRXDNN_STATUS_NOT_SUPPORTED;
  if (xDesc->strides[xDesc->nb - 1] != 1 || yDesc->strides[yDesc->nb - 1] != 1)
    return GRXDNN_STATUS_NOT_SUPPORTED;
  int64_t rows = 0, yrows = 0, xp = 0, yp = 0;
  if (!row_layout(*xDesc, &rows, &xp) || !row_layout(*yDesc, &yrows, &yp))
    return GRXDNN_STATUS_NOT_SUPPORTED;
  if (!x || !y) return GRXDNN_STATUS_INVALID_VALUE;
  const grxdnnStatus_t s = ensure_device(*handle);
  if (s != GRXDNN_STATUS_SUCCESS) return s;
  d->rows = rows;
  d->hidden = hidden;
  d->x_row_stride = xp;
  d->y_row_stride = yp;
  d->x = x;
  d->y = y;
  return GRXDNN_STATUS_SUCCESS;
}

}  // namespace

// The C API is the only thing these libraries export (built with
// -fvisibility=hidden).
#pragma GCC visibility push(default)
extern "C" {

const char* grxdnnGetStatusString(grxdnnStatus_t s) {
  switch (s) {
    case GRXDNN_STATUS_SUCCESS:          return "success";
    case GRXDNN_STATUS_NOT_INITIALIZED:  return "library not initialized";
    case GRXDNN_STATUS_ALLOC_FAILED:     return "allocation failed";
    case GRXDNN_STATUS_INVALID_VALUE:    return "invalid argument";
    case GRXDNN_STATUS_ARCH_MISMATCH:    return "device lacks a required capability";
    case GRXDNN_STATUS_EXECUTION_FAILED: return "kernel execution failed";
    case GRXDNN_STATUS_NOT_SUPPORTED:    return "not supported";
    case GRXDNN_STATUS_INTERNAL_ERROR:   return "internal error";
  }
  return "unknown status";
}

grxdnnStatus_t grxdnnCreate(grxdnnHandle_t* handle) {
  if (!handle) return GRXDNN_STATUS_INVALID_VALUE;
  *handle = new (std::nothrow) grxdnnContext();
  return *handle ? GRXDNN_STATUS_SUCCESS : GRXDNN_STATUS_ALLOC_FAILED;
}

grxdnnStatus_t grxdnnDestroy(grxdnnHandle_t handle) {
  if (!handle) return GRXDNN_STATUS_NOT_INITIALIZED;
  delete handle;
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnSetStream(grxdnnHandle_t handle, grxStream_t stream) {
  if (!handle) return GRXDNN_STATUS_NOT_INITIALIZED;
  handle->stream = reinterpret_cast<hipStream_t>(stream);
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnGetStream(grxdnnHandle_t handle, grxStream_t* stream) {
  if (!handle || !stream) return GRXDNN_STATUS_INVALID_VALUE;
  *stream = reinterpret_cast<grxStream_t>(handle->stream);
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnCreateTensorDescriptor(grxdnnTensorDescriptor_t* desc) {
  if (!desc) return GRXDNN_STATUS_INVALID_VALUE;
  *desc = new (std::nothrow) grxdnnTensorStruct();
  return *desc ? GRXDNN_STATUS_SUCCESS : GRXDNN_STATUS_ALLOC_FAILED;
}

grxdnnStatus_t grxdnnDestroyTensorDescriptor(grxdnnTensorDescriptor_t desc) {
  if (!desc) return GRXDNN_STATUS_INVALID_VALUE;
  delete desc;
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnSetTensorNdDescriptor(grxdnnTensorDescriptor_t desc, grxDataType_t dataType,
                                           int nbDims, const int dims[], const int strides[]) {
  if (!desc || !dims) return GRXDNN_STATUS_INVALID_VALUE;
  if (nbDims < 1 || nbDims > GRXDNN_DIM_MAX) return GRXDNN_STATUS_INVALID_VALUE;
  if (!known_type(dataType)) return GRXDNN_STATUS_INVALID_VALUE;
  for (int i = 0; i < nbDims; ++i) {
    if (dims[i] < 0) return GRXDNN_STATUS_INVALID_VALUE;
    if (strides && strides[i] < 0) return GRXDNN_STATUS_INVALID_VALUE;
  }
  grxdnnTensorStruct t;
  t.set = true;
  t.type = dataType;
  t.nb = nbDims;
  int64_t packed = 1;
  for (int i = nbDims - 1; i >= 0; --i) {
    t.dims[i] = dims[i];
    if (strides) {
      t.strides[i] = strides[i];
    } else {
      if (packed > 0x7fffffff) return GRXDNN_STATUS_INVALID_VALUE;
      t.strides[i] = (int)packed;
    }
    packed *= (dims[i] > 0 ? dims[i] : 1);
  }
  *desc = t;
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnGetTensorNdDescriptor(grxdnnTensorDescriptor_t desc, int nbDimsRequested,
                                           grxDataType_t* dataType, int* nbDims, int dims[],
                                           int strides[]) {
  if (!desc || !desc->set) return GRXDNN_STATUS_INVALID_VALUE;
  if (nbDimsRequested < 0) return GRXDNN_STATUS_INVALID_VALUE;
  if (dataType) *dataType = desc->type;
  if (nbDims) *nbDims = desc->nb;
  const int n = nbDimsRequested < desc->nb ? nbDimsRequested : desc->nb;
  for (int i = 0; i < n; ++i) {
    if (dims) dims[i] = desc->dims[i];
    if (strides) strides[i] = desc->strides[i];
  }
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnRMSNormForward(grxdnnHandle_t handle, grxdnnTensorDescriptor_t xDesc,
                                    const void* x, grxdnnTensorDescriptor_t wDesc,
                                    const void* gamma, float eps, grxdnnTensorDescriptor_t yDesc,
                                    void* y) {
  return norm_common(handle, xDesc, x, wDesc, gamma, nullptr, false, eps, yDesc, y);
}

grxdnnStatus_t grxdnnLayerNormForward(grxdnnHandle_t handle, grxdnnTensorDescriptor_t xDesc,
                                      const void* x, grxdnnTensorDescriptor_t wDesc,
                                      const void* gamma, const void* beta, float eps,
                                      grxdnnTensorDescriptor_t yDesc, void* y) {
  return norm_common(handle, xDesc, x, wDesc, gamma, beta, true, eps, yDesc, y);
}

grxdnnStatus_t grxdnnSoftmaxForward(grxdnnHandle_t handle, grxdnnTensorDescriptor_t xDesc,
                                    const void* x, grxdnnTensorDescriptor_t yDesc, void* y) {
  grxk::NormType nt{};
  grxk::RowDesc d{};
  bool empty = false;
  const grxdnnStatus_t s = row_common(handle, xDesc, x, yDesc, y, &nt, &d, &empty);
  if (s != GRXDNN_STATUS_SUCCESS || empty) return s;
  return from_hip(grxk::launch_softmax(nt, d, handle->stream));
}

grxdnnStatus_t grxdnnGeluForward(grxdnnHandle_t handle, grxdnnGeluMode_t mode,
                                 grxdnnTensorDescriptor_t xDesc, const void* x,
                                 grxdnnTensorDescriptor_t yDesc, void* y) {
  if (!handle) return GRXDNN_STATUS_NOT_INITIALIZED;
  if (mode != GRXDNN_GELU_ERF && mode != GRXDNN_GELU_TANH) return GRXDNN_STATUS_INVALID_VALUE;
  grxk::NormType nt{};
  grxk::RowDesc d{};
  bool empty = false;
  const grxdnnStatus_t s = row_common(handle, xDesc, x, yDesc, y, &nt, &d, &empty);
  if (s != GRXDNN_STATUS_SUCCESS || empty) return s;
  return from_hip(grxk::launch_gelu(nt, mode == GRXDNN_GELU_TANH, d, handle->stream));
}

grxdnnStatus_t grxdnnCreateAttentionDescriptor(grxdnnAttentionDescriptor_t* d) {
  if (!d) return GRXDNN_STATUS_INVALID_VALUE;
  *d = new (std::nothrow) grxdnnAttentionStruct();
  return *d ? GRXDNN_STATUS_SUCCESS : GRXDNN_STATUS_ALLOC_FAILED;
}

grxdnnStatus_t grxdnnDestroyAttentionDescriptor(grxdnnAttentionDescriptor_t d) {
  if (!d) return GRXDNN_STATUS_INVALID_VALUE;
  delete d;
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnSetAttentionDescriptor(grxdnnAttentionDescriptor_t d, int causal,
                                            float softmaxScale) {
  if (!d) return GRXDNN_STATUS_INVALID_VALUE;
  if (causal != 0 && causal != 1) return GRXDNN_STATUS_INVALID_VALUE;
  if (!std::isfinite(softmaxScale) || softmaxScale <= 0.0f) return GRXDNN_STATUS_INVALID_VALUE;
  d->set = true;
  d->causal = causal;
  d->scale = softmaxScale;
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnGetAttentionDescriptor(grxdnnAttentionDescriptor_t d, int* causal,
                                            float* softmaxScale) {
  if (!d || !d->set) return GRXDNN_STATUS_INVALID_VALUE;
  if (causal) *causal = d->causal;
  if (softmaxScale) *softmaxScale = d->scale;
  return GRXDNN_STATUS_SUCCESS;
}

grxdnnStatus_t grxdnnAttentionForward(grxdnnHandle_t handle, grxdnnAttentionDescriptor_t attnDesc,
                                      grxdnnTensorDescriptor_t qDesc, const void* q,
                                      grxdnnTensorDescriptor_t kDesc, const void* k,
                                      grxdnnTensorDescriptor_t vDesc, const void* v,
                                      grxdnnTensorDescriptor_t oDesc, void* o) {
  if (!handle) return GRXDNN_STATUS_NOT_INITIALIZED;
  if (!attnDesc || !qDesc || !kDesc || !vDesc || !oDesc) return GRXDNN_STATUS_INVALID_VALUE;
  if (!attnDesc->set || !qDesc->set || !kDesc->set || !vDesc->set || !oDesc->set)
    return GRXDNN_STATUS_INVALID_VALUE;
  if (qDesc->nb != 4 || !same_shape(*qDesc, *kDesc) || !same_shape(*qDesc, *vDesc) ||
      !same_shape(*qDesc, *oDesc))
    return GRXDNN_STATUS_INVALID_VALUE;
  const grxDataType_t t = qDesc->type;
  if (kDesc->type != t || vDesc->type != t || oDesc->type != t) return GRXDNN_STATUS_NOT_SUPPORTED;
  if (t != GRX_R_16BF && t != GRX_R_16F) return GRXDNN_STATUS_NOT_SUPPORTED;
  const int B = qDesc->dims[0], H = qDesc->dims[1], S = qDesc->dims[2], D = qDesc->dims[3];
  if (D != 64 && D != 128) return GRXDNN_STATUS_NOT_SUPPORTED;
  if ((int64_t)B * H * S == 0) return GRXDNN_STATUS_SUCCESS;
  const grxdnnTensorStruct* all[4] = {qDesc, kDesc, vDesc, oDesc};
  for (const grxdnnTensorStruct* d : all) {
    // 16-byte vector access along the head dimension needs a contiguous head
    // dimension and 16-byte aligned rows.
    if (d->strides[3] != 1) return GRXDNN_STATUS_NOT_SUPPORTED;
    for (int i = 0; i < 3; ++i)
      if (d->strides[i] % 8 != 0) return GRXDNN_STATUS_NOT_SUPPORTED;
  }
  if (!no_overlap(*oDesc)) return GRXDNN_STATUS_INVALID_VALUE;
  if (!q || !k || !v || !o) return GRXDNN_STATUS_INVALID_VALUE;
  // A workgroup writes its O rows while workgroups of other query tiles of
  // the same head still read K and V, so O may not share an element with
  // them. O == Q with the same layout is safe (a workgroup reads only its own
  // Q rows, before it writes them); any other overlap with Q is refused too.
  // Views with O's strides are compared element by element (O over the Q
  // slot of a packed QKV buffer is accepted), others by their byte spans.
  if (may_alias(*oDesc, o, *kDesc, k) || may_alias(*oDesc, o, *vDesc, v))
    return GRXDNN_STATUS_INVALID_VALUE;
  if (may_alias(*oDesc, o, *qDesc, q) && !(o == q && same_strides(*oDesc, *qDesc)))
    return GRXDNN_STATUS_INVALID_VALUE;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return GRXDNN_STATUS_NOT_SUPPORTED;

  const grxdnnStatus_t s = ensure_device(*handle);
  if (s != GRXDNN_STATUS_SUCCESS) return s;

  grxk::AttnDesc d{};
  d.B = B; d.H = H; d.S = S; d.D = D;
  d.causal = attnDesc->causal != 0;
  d.scale = attnDesc->scale;
  d.q = q; d.q_sb = qDesc->strides[0]; d.q_sh = qDesc->strides[1]; d.q_ss = qDesc->strides[2];
  d.k = k; d.k_sb = kDesc->strides[0]; d.k_sh = kDesc->strides[1]; d.k_ss = kDesc->strides[2];
  d.v = v; d.v_sb = vDesc->strides[0]; d.v_sh = vDesc->strides[1]; d.v_ss = vDesc->strides[2];
  d.o = o; d.o_sb = oDesc->strides[0]; d.o_sh = oDesc->strides[1]; d.o_ss = oDesc->strides[2];
  {
    std::lock_guard<std::mutex> lock(handle->mutex);
    if (handle->probe) {
      if (handle->probe_capacity < grxk::attention_probe_slots(B, H, S))
        return GRXDNN_STATUS_INVALID_VALUE;
      d.probe = handle->probe;
    }
  }
  return from_hip(grxk::launch_attention(
      t == GRX_R_16BF ? grxk::AttnType::BF16 : grxk::AttnType::F16, d, handle->stream));
}

grxdnnStatus_t grxdnnSetCycleProbe(grxdnnHandle_t handle, grxCycleSlot* slots, int capacity) {
  if (!handle) return GRXDNN_STATUS_NOT_INITIALIZED;
  if (slots && capacity <= 0) return GRXDNN_STATUS_INVALID_VALUE;
  std::lock_guard<std::mutex> lock(handle->mutex);
  handle->probe = slots;
  handle->probe_capacity = slots ? capacity : 0;
  return GRXDNN_STATUS_SUCCESS;
}

int grxdnnAttentionCycleSlotsNeeded(grxdnnHandle_t handle, int batch, int heads, int seqLen) {
  (void)handle;
  if (batch <= 0 || heads <= 0 || seqLen <= 0) return 0;
  const int64_t s = grxk::attention_probe_slots(batch, heads, seqLen);
  return s > INT_MAX ? INT_MAX : (int)s;
}

}  // extern "C"
#pragma GCC visibility pop
