// grxDNN RMSNorm / LayerNorm forward on gfx950.
//
// New (the reference plans grxDNN normalisation but ships none:
// ref docs/designs/grxcp_roadmap.md:864-877). HBM-bound: every byte of x is
// read once and every byte of y written once, so the design goal is streaming
// bandwidth, not arithmetic.
//
//  * rows of up to 256 16-byte chunks (2048 bf16): one row per 64-lane
//    wavefront, held packed in registers between the statistics pass and the
//    output pass; both statistics are in-register wave reductions, so there
//    is no LDS and no barrier and every wave streams independently;
//  * longer rows (up to 4096 chunks): one row per workgroup of chunks/2
//    threads (256, 512 or 1024), two chunks per thread held in registers,
//    one LDS combine per statistic; x is still read from HBM exactly once;
//  * longer still: x re-read per pass (from L2);
//  * 16-byte non-temporal loads of x and stores of y, gamma/beta via the
//    normal cached path (every row reuses them);
//  * statistics in fp32: wavefront butterfly (DPP and row swaps) then an LDS
//    combine of the waves' partials, summed in a fixed order so every thread
//    sees the same value.
//    LayerNorm's variance is the two-pass (x - mean)^2 form over the cached
//    registers, which costs no extra memory traffic.
// Rows whose length, pitch or base alignment rule out 16-byte chunks take a
// scalar path with the same arithmetic.

#include "../launch.h"
#include "device_common.h"
#include "row_io.h"

namespace grxk {
namespace {

struct NParams {
  const uint8_t* x;
  const uint8_t* gamma;
  const uint8_t* beta;
  uint8_t* y;
  int64_t x_rs, y_rs;  // row strides, elements
  int64_t rows;
  int rows_per_wg;     // norm_block: adjacent rows per workgroup
  int hidden;
  float eps;
};

// Sum over the 256-thread workgroup, identical in every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();  // red[] may still be read from a previous reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// One row per NT-thread workgroup, NQ 16-byte chunks per thread (chunk
// tid + NT*q), for rows longer than a wavefront handles well. Measured on
// 268 MB of bf16 rows: two chunks per thread with NT = chunks/2 streams at
// 6.2-6.3 TB/s, against 5.6-5.8 TB/s for one row per wavefront at these
// lengths. Each statistic is one wave butterfly plus one barrier; the waves'
// partials are summed in a fixed order, so every thread sees the same value.
// On large inputs a workgroup takes two adjacent rows, with gamma and beta
// loaded once into registers (blocks of rows_per_wg rows, strided by the
// grid). Measured at 16384 x 8192 bf16, five interleaved repeats: one row per
// workgroup re-reads gamma (and beta) per row, and their per-workgroup read
// from L2 costs 3 % (a copy without gamma: 6460 against 6270 GB/s); two rows
// a grid stride apart took LayerNorm from 5960 to 6050 GB/s but RMSNorm
// down 0.8 %; two adjacent rows: RMSNorm 6250 -> 6310, LayerNorm 6050 ->
// 6120; four or eight rows per workgroup, sharing gamma through LDS between
// the halves of a 1024-thread workgroup, or prefetching the next row's x
// measured slower. The partials alternate between two LDS slots by row, so
// a wave still reading one row's partials cannot see the next row's writes,
// and the loop needs no barrier of its own.
template <NormType T, bool LAYER, int NT, int NQ>
__global__ __launch_bounds__(NT) void norm_block(NParams p) {
  using IO = Io<T>;
  constexpr int V = IO::kVec;
  constexpr int NW = NT / 64;
  __shared__ float red[2][2][NW];   // [row parity][statistic][wave]
  const int tid = threadIdx.x;
  const int nchunks = p.hidden / V;
  const float inv_h = 1.0f / (float)p.hidden;
  int parity = 0;
  auto combine = [&](float v, int slot) {
    v = wave_sum(v);
    if ((tid & 63) == 0) red[parity][slot][tid >> 6] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += red[parity][slot][w];
    return t;
  };
  u32x4 graw[NQ], braw[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c = tid + NT * q;
    graw[q] = c < nchunks ? ((const u32x4*)p.gamma)[c] : u32x4{0, 0, 0, 0};
    braw[q] = (LAYER && c < nchunks) ? ((const u32x4*)p.beta)[c] : u32x4{0, 0, 0, 0};
  }

  const int64_t rb = p.rows_per_wg;
  for (int64_t base = (int64_t)blockIdx.x * rb; base < p.rows; base += (int64_t)gridDim.x * rb)
  for (int64_t row = base, rend = min(p.rows, base + rb); row < rend; ++row, parity ^= 1) {
    const uint8_t* xrow = p.x + row * p.x_rs * (int64_t)(16 / V);
    uint8_t* yrow = p.y + row * p.y_rs * (int64_t)(16 / V);
    u32x4 raw[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = tid + NT * q;
      raw[q] = c < nchunks ? __builtin_nontemporal_load((const u32x4*)xrow + c) : u32x4{0, 0, 0, 0};
    }
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      float v[V];
      IO::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < V; ++e) s += LAYER ? v[e] : v[e] * v[e];
    }
    s = combine(s, 0);
    float mean = 0.0f, inv;
    if (LAYER) {
      mean = s * inv_h;
      float d2 = 0.0f;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        if (tid + NT * q >= nchunks) continue;
        float v[V];
        IO::unpack(raw[q], v);
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float d = v[e] - mean;
          d2 += d * d;
        }
      }
      d2 = combine(d2, 1);
      inv = 1.0f / sqrtf(d2 * inv_h + p.eps);
    } else {
      inv = 1.0f / sqrtf(s * inv_h + p.eps);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = tid + NT * q;
      if (c >= nchunks) continue;
      float v[V], g[V], o[V];
      IO::unpack(raw[q], v);
      IO::unpack(graw[q], g);
      if (LAYER) {
        float b[V];
        IO::unpack(braw[q], b);
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = (v[e] - mean) * inv * g[e] + b[e];
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = v[e] * inv * g[e];
      }
      __builtin_nontemporal_store(IO::pack(o), (u32x4*)yrow + c);
    }
  }
}

// One row per 64-lane wavefront, for rows of up to NC x 64 16-byte chunks:
// the row lives in the wave's registers, both statistics are wave
// reductions (lane moves only: no LDS, no barrier), so every wave streams
// independently and a CU keeps ~20 rows of loads in flight.
template <NormType T, bool LAYER, int NC>
__global__ __launch_bounds__(256) void norm_wave(NParams p) {
  using IO = Io<T>;
  constexpr int V = IO::kVec;
  const int lane = threadIdx.x & 63;
  const int nchunks = p.hidden / V;
  const float inv_h = 1.0f / (float)p.hidden;
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
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < NC; ++q) {
      float v[V];
      IO::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < V; ++e) s += LAYER ? v[e] : v[e] * v[e];
    }
    // Keep only the packed row live between passes (unpacking again is a
    // couple of ALU ops; holding 8*NC floats would halve the waves per CU).
#pragma unroll
    for (int q = 0; q < NC; ++q) asm volatile("" : "+v"(raw[q]));
    s = wave_sum(s);
    float mean = 0.0f, inv;
    if (LAYER) {
      mean = s * inv_h;
      float d2 = 0.0f;
#pragma unroll
      for (int q = 0; q < NC; ++q) {
        if (lane + 64 * q >= nchunks) continue;
        float v[V];
        IO::unpack(raw[q], v);
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float d = v[e] - mean;
          d2 += d * d;
        }
      }
      d2 = wave_sum(d2);
#pragma unroll
      for (int q = 0; q < NC; ++q) asm volatile("" : "+v"(raw[q]));
      inv = 1.0f / sqrtf(d2 * inv_h + p.eps);
    } else {
      inv = 1.0f / sqrtf(s * inv_h + p.eps);
    }
#pragma unroll
    for (int q = 0; q < NC; ++q) {
      const int c = lane + 64 * q;
      if (c >= nchunks) continue;
      float v[V], g[V], o[V];
      IO::unpack(raw[q], v);
      IO::unpack(((const u32x4*)p.gamma)[c], g);
      if (LAYER) {
        float b[V];
        IO::unpack(((const u32x4*)p.beta)[c], b);
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = (v[e] - mean) * inv * g[e] + b[e];
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = v[e] * inv * g[e];
      }
      __builtin_nontemporal_store(IO::pack(o), (u32x4*)yrow + c);
    }
  }
}

// Any length / alignment: element-wise, x re-read for each pass.
template <NormType T, bool LAYER>
__global__ __launch_bounds__(256) void norm_scalar(NParams p) {
  using IO = Io<T>;
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const float inv_h = 1.0f / (float)p.hidden;
  for (int64_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
    const int64_t xo = row * p.x_rs, yo = row * p.y_rs;
    float s = 0.0f;
    for (int c = tid; c < p.hidden; c += 256) {
      const float x = IO::ld(p.x, xo + c);
      s += LAYER ? x : x * x;
    }
    s = block_sum(s, red);
    float mean = 0.0f, inv;
    if (LAYER) {
      mean = s * inv_h;
      float d2 = 0.0f;
      for (int c = tid; c < p.hidden; c += 256) {
        const float d = IO::ld(p.x, xo + c) - mean;
        d2 += d * d;
      }
      d2 = block_sum(d2, red);
      inv = 1.0f / sqrtf(d2 * inv_h + p.eps);
    } else {
      inv = 1.0f / sqrtf(s * inv_h + p.eps);
    }
    for (int c = tid; c < p.hidden; c += 256) {
      const float x = IO::ld(p.x, xo + c);
      const float g = IO::ld(p.gamma, c);
      const float o = LAYER ? (x - mean) * inv * g + IO::ld(p.beta, c) : x * inv * g;
      IO::st(p.y, yo + c, o);
    }
  }
}

template <NormType T, bool LAYER>
hipError_t run(const NormDesc& d, hipStream_t s) {
  NParams p{};
  p.x = (const uint8_t*)d.x;
  p.gamma = (const uint8_t*)d.gamma;
  p.beta = (const uint8_t*)d.beta;
  p.y = (uint8_t*)d.y;
  p.x_rs = d.x_row_stride;
  p.y_rs = d.y_row_stride;
  p.rows = d.rows;
  p.hidden = d.hidden;
  p.eps = d.eps;
  constexpr int V = Io<T>::kVec;
  const unsigned grid = (unsigned)std::min<int64_t>(d.rows, 1 << 30);
  auto al = [](const void* q) { return ((uintptr_t)q % 16) == 0; };
  const bool vec = d.hidden % V == 0 && d.x_row_stride % V == 0 && d.y_row_stride % V == 0 &&
                   al(d.x) && al(d.y) && al(d.gamma) && (!LAYER || al(d.beta));
  const int nchunks = d.hidden / V;
  const unsigned wgrid = (unsigned)std::min<int64_t>((d.rows + 3) / 4, 1 << 30);
  // norm_block: two adjacent rows per workgroup where that still leaves at
  // least four workgroups per CU
  p.rows_per_wg = d.rows >= 2048 ? 2 : 1;
  const unsigned bgrid =
      (unsigned)std::min<int64_t>((d.rows + p.rows_per_wg - 1) / p.rows_per_wg, 1 << 30);
  if (vec && nchunks <= 64) {
    hipLaunchKernelGGL((norm_wave<T, LAYER, 1>), dim3(wgrid), dim3(256), 0, s, p);
  } else if (vec && nchunks <= 128) {
    hipLaunchKernelGGL((norm_wave<T, LAYER, 2>), dim3(wgrid), dim3(256), 0, s, p);
  } else if (vec && nchunks <= 256) {
    hipLaunchKernelGGL((norm_wave<T, LAYER, 4>), dim3(wgrid), dim3(256), 0, s, p);
  } else if (vec && nchunks <= 512) {
    hipLaunchKernelGGL((norm_block<T, LAYER, 256, 2>), dim3(bgrid), dim3(256), 0, s, p);
  } else if (vec && nchunks <= 1024) {
    hipLaunchKernelGGL((norm_block<T, LAYER, 512, 2>), dim3(bgrid), dim3(512), 0, s, p);
  } else if (vec && nchunks <= 2048) {
    hipLaunchKernelGGL((norm_block<T, LAYER, 1024, 2>), dim3(bgrid), dim3(1024), 0, s, p);
  } else if (vec && nchunks <= 4096) {
    hipLaunchKernelGGL((norm_block<T, LAYER, 1024, 4>), dim3(bgrid), dim3(1024), 0, s, p);
  } else {
    hipLaunchKernelGGL((norm_scalar<T, LAYER>), dim3(grid), dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rmsnorm(NormType t, const NormDesc& d, hipStream_t s) {
  switch (t) {
    case NormType::BF16: return run<NormType::BF16, false>(d, s);
    case NormType::F16:  return run<NormType::F16, false>(d, s);
    case NormType::F32:  return run<NormType::F32, false>(d, s);
  }
  return hipErrorNotSupported;
}

hipError_t launch_layernorm(NormType t, const NormDesc& d, hipStream_t s) {
  switch (t) {
    case NormType::BF16: return run<NormType::BF16, true>(d, s);
    case NormType::F16:  return run<NormType::F16, true>(d, s);
    case NormType::F32:  return run<NormType::F32, true>(d, s);
  }
  return hipErrorNotSupported;
}

}  // namespace grxk
