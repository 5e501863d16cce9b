// grxDNN softmax (over the last dimension) and GELU forward on gfx950.
//
// New: the reference plans both for grxDNN (ref
// docs/designs/grxcp_roadmap.md:864-877, grxcp_architecture.md:594) and ships
// neither. Both are HBM-bound streams: x is read once and y written once.
//
// Softmax, rows of up to 256 16-byte chunks: one row per wavefront, held
// packed in registers; the row max and the sum of exp(x - max) are in-register
// wave reductions (no LDS, no barrier). Up to 4096 chunks: one row per workgroup,
// two or four chunks per thread in registers, one LDS combine per statistic.
// y = exp(x - max) / sum in fp32, rounded once (16-bit outputs use the
// hardware exp2, fp32 the library expf). Longer or unaligned rows: one row
// per workgroup, three element-wise passes (max, sum, write) re-reading x.
// GELU: one 16-byte chunk per thread, over the tensor as one array when its
// rows are contiguous, else row by row (element-wise for unaligned layouts);
// erf or tanh form in fp32, rounded once.

#include "../launch.h"
#include "device_common.h"
#include "row_io.h"

namespace grxk {
namespace {

// exp(d) for d <= 0. 16-bit outputs take the hardware exp2 of d*log2(e)
// (relative error well under their half ulp); fp32 keeps the library expf.
template <NormType T> __device__ __forceinline__ float exp_le0(float d) {
  if constexpr (T == NormType::F32) return expf(d);
  else return __builtin_amdgcn_exp2f(d * 1.4426950408889634f);
}

struct RParams {
  const uint8_t* x;
  uint8_t* y;
  int64_t x_rs, y_rs;  // row strides, elements
  int64_t rows;
  int hidden;
};

template <NormType T, int NC>
__global__ __launch_bounds__(256) void softmax_wave(RParams p) {
  using IO = Io<T>;
  constexpr int V = IO::kVec;
  const int lane = threadIdx.x & 63;
  const int nchunks = p.hidden / V;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < p.rows; row += nwaves) {
    const uint8_t* xrow = p.x + row * p.x_rs * (int64_t)(16 / V);
    uint8_t* yrow = p.y + row * p.y_rs * (int64_t)(16 / V);
    u32x4 raw[NC];
#pragma unroll
    for (int q = 0; q < NC; ++q) {
      const int c = lane + 64 * q;
      raw[q] = c < nchunks ? __builtin_nontemporal_load((const u32x4*)xrow + c) : u32x4{0, 0, 0, 0};
    }
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < NC; ++q) {
      if (lane + 64 * q >= nchunks) continue;
      float v[V];
      IO::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < V; ++e) mx = fmaxf(mx, v[e]);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < NC; ++q) {
      if (lane + 64 * q >= nchunks) continue;
      float v[V];
      IO::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < V; ++e) sum += exp_le0<T>(v[e] - mx);
    }
    // Keep only the packed row live between passes.
#pragma unroll
    for (int q = 0; q < NC; ++q) asm volatile("" : "+v"(raw[q]));
    const float inv = 1.0f / wave_sum(sum);
#pragma unroll
    for (int q = 0; q < NC; ++q) {
      const int c = lane + 64 * q;
      if (c >= nchunks) continue;
      float v[V], o[V];
      IO::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < V; ++e) o[e] = exp_le0<T>(v[e] - mx) * inv;
      __builtin_nontemporal_store(IO::pack(o), (u32x4*)yrow + c);
    }
  }
}

// One row per NT-thread workgroup, NQ 16-byte chunks per thread (chunk
// tid + NT*q), held in registers: the streaming layout that measured fastest
// for rows of 2K-32K 16-bit elements (chunks/2 threads of two chunks each).
// The row max and the sum are each a wave butterfly plus one LDS combine of
// the waves' partials in a fixed order, identical in every thread.
template <NormType T, int NT, int NQ>
__global__ __launch_bounds__(NT) void softmax_block(RParams p) {
  using IO = Io<T>;
  constexpr int V = IO::kVec;
  constexpr int NW = NT / 64;
  __shared__ float red[2][NW];
  const int tid = threadIdx.x;
  const int nchunks = p.hidden / V;
  for (int64_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
    const uint8_t* xrow = p.x + row * p.x_rs * (int64_t)(16 / V);
    uint8_t* yrow = p.y + row * p.y_rs * (int64_t)(16 / V);
    u32x4 raw[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = tid + NT * q;
      raw[q] = c < nchunks ? __builtin_nontemporal_load((const u32x4*)xrow + c) : u32x4{0, 0, 0, 0};
    }
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (tid + NT * q >= nchunks) continue;
      float v[V];
      IO::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < V; ++e) mx = fmaxf(mx, v[e]);
    }
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[0][tid >> 6] = mx;
    __syncthreads();
    mx = red[0][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, red[0][w]);
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (tid + NT * q >= nchunks) continue;
      float v[V];
      IO::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < V; ++e) sum += exp_le0<T>(v[e] - mx);
    }
    sum = wave_sum(sum);
    if ((tid & 63) == 0) red[1][tid >> 6] = sum;
    __syncthreads();
    sum = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) sum += red[1][w];
    const float inv = 1.0f / sum;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = tid + NT * q;
      if (c >= nchunks) continue;
      float v[V], o[V];
      IO::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < V; ++e) o[e] = exp_le0<T>(v[e] - mx) * inv;
      __builtin_nontemporal_store(IO::pack(o), (u32x4*)yrow + c);
    }
    // Only a grid of fewer workgroups than rows (over 2^30 rows) loops: the
    // next row's partials must not land before every wave has read these.
    if (row + gridDim.x < p.rows) __syncthreads();
  }
}

// Identical in every thread of the 256-thread workgroup.
__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  v = is_max ? wave_max(v) : wave_sum(v);
  __syncthreads();  // red[] may still be read from a previous reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return is_max ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]))
                : (red[0] + red[1]) + (red[2] + red[3]);
}

template <NormType T>
__global__ __launch_bounds__(256) void softmax_rows(RParams p) {
  using IO = Io<T>;
  __shared__ float red[4];
  const int tid = threadIdx.x;
  for (int64_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
    const int64_t xo = row * p.x_rs, yo = row * p.y_rs;
    float mx = -INFINITY;
    for (int c = tid; c < p.hidden; c += 256) mx = fmaxf(mx, IO::ld(p.x, xo + c));
    mx = block_reduce(mx, red, true);
    float sum = 0.0f;
    for (int c = tid; c < p.hidden; c += 256) sum += exp_le0<T>(IO::ld(p.x, xo + c) - mx);
    const float inv = 1.0f / block_reduce(sum, red, false);
    for (int c = tid; c < p.hidden; c += 256) IO::st(p.y, yo + c, exp_le0<T>(IO::ld(p.x, xo + c) - mx) * inv);
  }
}

// Standard normal CDF, Phi(x) = erfc(-x / sqrt 2) / 2, through the Chebyshev
// fit of erfc in Press et al., Numerical Recipes in C (2nd ed., section 6.2,
// erfcc): erfc(z) = t exp(-z^2 + Q(t)), t = 1 / (1 + z/2), z >= 0, fractional
// error below 1.2e-7 for every z (1.05e-7 measured in float64 against scipy).
// The sign of x picks erfc(|z|)/2 or 1 - erfc(|z|)/2, so a small result is
// never the difference of two numbers near 1 (1 + erff(x / sqrt 2) is 0 in
// fp32 from x = -5.4 on), and no branch splits a wave. One reciprocal, one
// exp2 and 17 other VALU instructions (16384 x 8192 bf16: 5980 GB/s, against
// 5032 with the library erff and 3061 with the library erfcf, whose
// interval branches make it compute-bound).
__device__ __forceinline__ float normal_cdf(float x) {
  const float z = fabsf(x) * 0.7071067811865476f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float q = 0.17087277f;
  q = fmaf(t, q, -0.82215223f);
  q = fmaf(t, q, 1.48851587f);
  q = fmaf(t, q, -1.13520398f);
  q = fmaf(t, q, 0.27886807f);
  q = fmaf(t, q, -0.18628806f);
  q = fmaf(t, q, 0.09678418f);
  q = fmaf(t, q, 0.37409196f);
  q = fmaf(t, q, 1.00002368f);
  q = fmaf(t, q, -1.26551223f);
  const float a = fmaf(-z, z, q);                          // ln(erfc(z) / t)
  // erfc(z) / 2 = t * 2^(a log2(e) - 1)
  const float h = t * __builtin_amdgcn_exp2f(fmaf(a, 1.4426950408889634f, -1.0f));
  return x < 0.0f ? h : 1.0f - h;
}

// The tanh form uses x/2 (1 + tanh z) = x * sigmoid(2z) = x / (1 + exp(-2z)):
// one hardware exp2 and one reciprocal instead of a library tanh. The erf
// form is x * Phi(x) with Phi as above. Neither forms 1 + erf or 1 + tanh,
// which cancel in the negative tail, so small results keep their relative
// precision.
template <bool TANH> __device__ __forceinline__ float gelu(float x) {
  if (TANH) {
    const float z = 0.7978845608028654f * (x + 0.044715f * x * x * x);  // sqrt(2/pi)(x + 0.044715 x^3)
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * z));  // 2 log2(e)
  }
  return x * normal_cdf(x);
}

template <NormType T, bool TANH>
__global__ __launch_bounds__(256) void gelu_vec(RParams p) {
  using IO = Io<T>;
  constexpr int V = IO::kVec;
  const int nchunks = p.hidden / V;
  const int64_t total = p.rows * nchunks;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    const int64_t row = i / nchunks;
    const int c = (int)(i - row * nchunks);
    const u32x4 w = __builtin_nontemporal_load(
        (const u32x4*)(p.x + row * p.x_rs * (int64_t)(16 / V)) + c);
    float v[V];
    IO::unpack(w, v);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = gelu<TANH>(v[e]);
    __builtin_nontemporal_store(IO::pack(v), (u32x4*)(p.y + row * p.y_rs * (int64_t)(16 / V)) + c);
  }
}

// Contiguous rows (pitch == hidden): the tensor is one array of chunks, one
// chunk per thread, no row arithmetic.
template <NormType T, bool TANH>
__global__ __launch_bounds__(256) void gelu_flat(RParams p) {
  using IO = Io<T>;
  constexpr int V = IO::kVec;
  const int64_t total = p.rows * (int64_t)(p.hidden / V);
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    const u32x4 w = __builtin_nontemporal_load((const u32x4*)p.x + i);
    float v[V];
    IO::unpack(w, v);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = gelu<TANH>(v[e]);
    __builtin_nontemporal_store(IO::pack(v), (u32x4*)p.y + i);
  }
}

template <NormType T, bool TANH>
__global__ __launch_bounds__(256) void gelu_scalar(RParams p) {
  using IO = Io<T>;
  const int64_t total = p.rows * p.hidden;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    const int64_t row = i / p.hidden;
    const int c = (int)(i - row * p.hidden);
    IO::st(p.y, row * p.y_rs + c, gelu<TANH>(IO::ld(p.x, row * p.x_rs + c)));
  }
}

RParams make_params(const RowDesc& d) {
  RParams p{};
  p.x = (const uint8_t*)d.x;
  p.y = (uint8_t*)d.y;
  p.x_rs = d.x_row_stride;
  p.y_rs = d.y_row_stride;
  p.rows = d.rows;
  p.hidden = d.hidden;
  return p;
}

template <NormType T>
bool vec_layout(const RowDesc& d) {
  constexpr int V = Io<T>::kVec;
  return d.hidden % V == 0 && d.x_row_stride % V == 0 && d.y_row_stride % V == 0 &&
         (uintptr_t)d.x % 16 == 0 && (uintptr_t)d.y % 16 == 0;
}

template <NormType T>
hipError_t run_softmax(const RowDesc& d, hipStream_t s) {
  const RParams p = make_params(d);
  const int nchunks = d.hidden / Io<T>::kVec;
  const unsigned wgrid = (unsigned)std::min<int64_t>((d.rows + 3) / 4, 1 << 30);
  const bool vec = vec_layout<T>(d);
  const unsigned bgrid = (unsigned)std::min<int64_t>(d.rows, 1 << 30);
  if (vec && nchunks <= 64) hipLaunchKernelGGL((softmax_wave<T, 1>), dim3(wgrid), dim3(256), 0, s, p);
  else if (vec && nchunks <= 128) hipLaunchKernelGGL((softmax_wave<T, 2>), dim3(wgrid), dim3(256), 0, s, p);
  else if (vec && nchunks <= 256) hipLaunchKernelGGL((softmax_wave<T, 4>), dim3(wgrid), dim3(256), 0, s, p);
  else if (vec && nchunks <= 512) hipLaunchKernelGGL((softmax_block<T, 256, 2>), dim3(bgrid), dim3(256), 0, s, p);
  else if (vec && nchunks <= 1024) hipLaunchKernelGGL((softmax_block<T, 512, 2>), dim3(bgrid), dim3(512), 0, s, p);
  else if (vec && nchunks <= 2048) hipLaunchKernelGGL((softmax_block<T, 1024, 2>), dim3(bgrid), dim3(1024), 0, s, p);
  else if (vec && nchunks <= 4096) hipLaunchKernelGGL((softmax_block<T, 1024, 4>), dim3(bgrid), dim3(1024), 0, s, p);
  else hipLaunchKernelGGL((softmax_rows<T>), dim3(bgrid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <NormType T, bool TANH>
hipError_t run_gelu(const RowDesc& d, hipStream_t s) {
  const RParams p = make_params(d);
  const bool vec = vec_layout<T>(d);
  const int64_t items = vec ? d.rows * (d.hidden / Io<T>::kVec) : d.rows * d.hidden;
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((items + 255) / 256, 1 << 20));
  const bool flat = d.rows == 1 || (d.x_row_stride == d.hidden && d.y_row_stride == d.hidden);
  if (vec && flat) hipLaunchKernelGGL((gelu_flat<T, TANH>), dim3(grid), dim3(256), 0, s, p);
  else if (vec) hipLaunchKernelGGL((gelu_vec<T, TANH>), dim3(grid), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((gelu_scalar<T, TANH>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_softmax(NormType t, const RowDesc& d, hipStream_t s) {
  switch (t) {
    case NormType::BF16: return run_softmax<NormType::BF16>(d, s);
    case NormType::F16:  return run_softmax<NormType::F16>(d, s);
    case NormType::F32:  return run_softmax<NormType::F32>(d, s);
  }
  return hipErrorNotSupported;
}

hipError_t launch_gelu(NormType t, bool tanh_form, const RowDesc& d, hipStream_t s) {
  switch (t) {
    case NormType::BF16: return tanh_form ? run_gelu<NormType::BF16, true>(d, s) : run_gelu<NormType::BF16, false>(d, s);
    case NormType::F16:  return tanh_form ? run_gelu<NormType::F16, true>(d, s) : run_gelu<NormType::F16, false>(d, s);
    case NormType::F32:  return tanh_form ? run_gelu<NormType::F32, true>(d, s) : run_gelu<NormType::F32, false>(d, s);
  }
  return hipErrorNotSupported;
}

}  // namespace grxk
