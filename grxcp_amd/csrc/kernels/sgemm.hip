// grxBLAS fp32 kernels on gfx950: Sgemm / SgemmStridedBatched, and the
// level-1/2 routines (saxpy, sscal, sgemv).
//
// Sgemm replaces the reference's one-thread-per-output kernel
// (ref: src/libs/grxblas/kernels/sgemm.cpp:22-89; 2 global loads per
// multiply-add) with an fp32 matrix-core kernel (v_mfma_f32_32x32x2_f32): a
// 128x128 (or, for problems too small to fill the chip, 64x64) tile of C per
// 256-thread workgroup, 16-deep K stages double-buffered through LDS with
// guarded loads that apply op() while staging (all four transposes, ragged
// shapes, any leading dimension). The batch is the grid's z dimension with
// signed element strides (a zero stride broadcasts an operand), exactly the
// reference's one-launch batching (ref: src/libs/grxblas/grxblas.cpp:936-938).
// beta == 0 never reads C (ref: kernels/sgemm.cpp:80-85). Problems that
// fill the GPU with 256x256 tiles run gemm_mfma.hip's TN kernel on fp32
// instead (grxblas.cpp sgemm_batched).
//
// Level 1/2 follow the reference's semantics (ref: kernels/blas12.cpp:41-132):
// BLAS increments (negative walks backwards), sgemv beta == 0 never reads y.

#include "../launch.h"
#include "device_common.h"

namespace grxk {
namespace {

constexpr int kK = 16;   // K per stage

struct SParams {
  const float* a; const float* b; float* c;
  int64_t lda, ldb, ldc;
  int64_t sa, sb, sc;
  int m, n, k;
  int ta, tb;
  int tiles_m;
  float alpha, beta;
  grxCycleSlot* probe;
};

// One workgroup = 4 waves (2 x 2) computes an MT x MT tile of C with
// v_mfma_f32_32x32x2_f32 (each wave MT/2 x MT/2, i.e. (MT/64)^2 .. 4 MFMA
// tiles). K advances 16 at a time through double-buffered LDS tiles
// As[kk][i] = op(A)[row0+i][k0+kk] and Bs[kk][j] = op(B)[k0+kk][col0+j]; the
// next stage's loads (op() applied while loading, zeros outside the matrix)
// are issued before the current stage's MFMAs and stored after them, one
// barrier per stage. An MFMA k-step reads one float per lane per operand:
// lane l takes row/column l%32 at k = 2s + l/32.
// TA/TB are template parameters, so the staging code has no run-time
// transpose switch. VEC: leading dimensions, strides and base pointers are
// multiples of 4 floats, so 4 consecutive elements along an operand's
// contiguous dimension are one aligned 16-byte load; a stage wholly inside
// the matrices (decided once per stage, uniformly) takes those loads with no
// per-element guard, other stages the guarded path. (Measured at 4096^3:
// 91 -> 129 TFLOP/s against one kernel with run-time transposes and guards,
// 129 -> 134 with the fragment reads one k-step ahead. Slower, same output:
// a pitch that puts k-rows 2s and 2s+1 half the banks apart (3 %: 3 instead
// of 4 workgroups per CU), an XOR-swizzled unpadded layout (4 %), 32-deep
// stages (2 workgroups per CU, 5-9 %), 256x256 tiles (one wave per SIMD,
// 4 %), the next stage's LDS stores moved to mid-stage (no change).)
//
// MT = 32 (problems of few 64x64 tiles, 512^3 among them): each wave one
// 16x16 tile with v_mfma_f32_16x16x4_f32, K 32 deep per stage (so that the
// staging keeps one 4-element group per thread and operand), rows 33 floats
// apart: over 64 banks that keeps every access of the tile at most 2-way
// conflicted -- the fragment reads (four 16-lane groups at k = 4s .. 4s+3),
// the transposing stores of a K-contiguous operand (8-way at a pitch of 48)
// and the direct stores (4-way at 48); 512^3 30.7 -> 32.0 TFLOP/s.
template <int MT, bool VEC, bool TA, bool TB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8)))
void sgemm_mfma(SParams p) {
  constexpr int kK = MT == 32 ? 32 : grxk::kK;   // K per stage
  constexpr int WT = MT / 2;            // wave tile edge
  constexpr int NF = WT / 32;           // 32x32 MFMA tiles per wave edge (0 at MT = 32)
  constexpr int PITCH = MT == 32 ? 33 : MT + 4;  // MT + 4: 16-byte aligned rows, 4 workgroups fit a CU's LDS at MT=128
  constexpr int PER = MT * kK / 256;    // elements per thread per operand per stage
  __shared__ float As[2][kK][PITCH];
  __shared__ float Bs[2][kK][PITCH];

  const uint64_t t0 = p.probe ? cycle_now() : 0;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int tm = blockIdx.x % p.tiles_m;
  const int tn = blockIdx.x / p.tiles_m;
  const int row0 = tm * MT, col0 = tn * MT;
  const int64_t bz = blockIdx.z;
  const float* A = p.a + bz * p.sa;
  const float* B = p.b + bz * p.sb;
  float* C = p.c + bz * p.sc;
  const bool interior = row0 + MT <= p.m && col0 + MT <= p.n;

  // Staging: an operand stage is MT x 16 elements read along its storage's
  // contiguous dimension (op(A): i for N, k for T; op(B): k for N, j for T)
  // in groups of 4 consecutive elements; thread t handles groups
  // t + 256*q. Element (cont, other) of a group maps to LDS [kk][i or j].
  constexpr int GPT = PER / 4;  // groups per thread per operand
  float ra[PER], rb[PER];
  // Element (c, o) of a group is X[o*ld + c], valid iff c < lim_cont, o < lim_other.
  auto load_group = [&](const float* X, int64_t ld, bool full, int lim_cont, int lim_other,
                        int cont, int other, float* out) {
    const float* q = X + (int64_t)other * ld + cont;
    if (VEC && (full || (other < lim_other && cont + 3 < lim_cont))) {
      const float4 v = *(const float4*)q;
      out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) out[v] = (other < lim_other && cont + v < lim_cont) ? q[v] : 0.0f;
    }
  };
  // op(A) (m x k): N stores A[k*lda + i] (cont = i), T stores A[i*lda + k] (cont = k).
  // op(B) (k x n): N stores B[j*ldb + k] (cont = k), T stores B[k*ldb + j] (cont = j).
  auto load_all = [&](int k0, bool full) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < GPT; ++q) {
      const int e = 4 * (tid + 256 * q);
      if (TA) load_group(A, p.lda, full, p.k, p.m, k0 + e % kK, row0 + e / kK, &ra[4 * q]);
      else load_group(A, p.lda, full, p.m, p.k, row0 + e % MT, k0 + e / MT, &ra[4 * q]);
      if (TB) load_group(B, p.ldb, full, p.n, p.k, col0 + e % MT, k0 + e / MT, &rb[4 * q]);
      else load_group(B, p.ldb, full, p.k, p.n, k0 + e % kK, col0 + e / kK, &rb[4 * q]);
    }
  };
  auto load = [&](int k0) {
    // One uniform decision per stage: the unguarded path is straight-line code.
    if (VEC && interior && k0 + kK <= p.k) load_all(k0, true);
    else load_all(k0, false);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int q = 0; q < GPT; ++q) {
      const int e = 4 * (tid + 256 * q);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (TA) As[buf][e % kK + v][e / kK] = ra[4 * q + v];
        else As[buf][e / MT][e % MT + v] = ra[4 * q + v];
        if (TB) Bs[buf][e / MT][e % MT + v] = rb[4 * q + v];
        else Bs[buf][e % kK + v][e / kK] = rb[4 * q + v];
      }
    }
  };

  // C = alpha*acc + beta*C (col-major) for a lane's run of 4 rows i0.. of
  // column gj: one 16-byte non-temporal store where the run lies inside C and
  // C's columns are 16-byte aligned, element by element otherwise (same
  // arithmetic).
  const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)C & 15) == 0;
  auto run4 = [&](int i0, int gj, const float* v) __attribute__((always_inline)) {
    float* cp = C + (int64_t)gj * p.ldc + i0;
    if (vec && i0 + 4 <= p.m) {
      f32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = __fmul_rn(p.alpha, v[q]);
      if (p.beta != 0.0f) {
        const f32x4 old = *(const f32x4*)cp;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = __fadd_rn(o[q], __fmul_rn(p.beta, old[q]));
      }
      __builtin_nontemporal_store(o, (f32x4*)cp);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (i0 + q >= p.m) break;
        const float x = __fmul_rn(p.alpha, v[q]);
        cp[q] = (p.beta == 0.0f) ? x : __fadd_rn(x, __fmul_rn(p.beta, cp[q]));
      }
    }
  };

  if constexpr (MT == 32) {
    // One 16x16 tile per wave: lane l reads op(A) row 16*wm + l%16 and op(B)
    // column 16*wn + l%16 at k = 4s + l/16, and holds rows 4*(l/16) .. +3 of
    // column l%16 of the result.
    const int r16 = lane & 15, kq = lane >> 4;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    load(0);
    store(0);
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 < p.k; k0 += kK) {
      const bool more = k0 + kK < p.k;
      if (more) load(k0 + kK);
      float av[kK / 4], bv[kK / 4];
#pragma unroll
      for (int st = 0; st < kK / 4; ++st) {
        av[st] = As[buf][4 * st + kq][16 * wm + r16];
        bv[st] = Bs[buf][4 * st + kq][16 * wn + r16];
      }
#pragma unroll
      for (int st = 0; st < kK / 4; ++st)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[st], bv[st], acc, 0, 0, 0);
      if (more) store(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
    const int gj = col0 + 16 * wn + r16;
    const int i0 = row0 + 16 * wm + 4 * kq;
    if (gj < p.n && i0 < p.m) {
      const float v[4] = {acc[0], acc[1], acc[2], acc[3]};
      run4(i0, gj, v);
    }
  } else {
    f32x16 acc[NF][NF];
#pragma unroll
    for (int fm = 0; fm < NF; ++fm)
#pragma unroll
      for (int fn = 0; fn < NF; ++fn)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;

    load(0);
    store(0);
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 < p.k; k0 += kK) {
      const bool more = k0 + kK < p.k;
      if (more) load(k0 + kK);
      // Fragments one k-step ahead: step s+1's LDS reads are issued before
      // step s's MFMAs (the scheduling barriers keep that order), so each
      // wait covers reads issued a whole step earlier.
      float av[2][NF], bv[2][NF];
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        av[0][f] = As[buf][hh][WT * wm + 32 * f + l32];
        bv[0][f] = Bs[buf][hh][WT * wn + 32 * f + l32];
      }
#pragma unroll
      for (int s = 0; s < kK / 2; ++s) {
        if (s + 1 < kK / 2) {
#pragma unroll
          for (int f = 0; f < NF; ++f) {
            av[(s + 1) & 1][f] = As[buf][2 * s + 2 + hh][WT * wm + 32 * f + l32];
            bv[(s + 1) & 1][f] = Bs[buf][2 * s + 2 + hh][WT * wn + 32 * f + l32];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int fm = 0; fm < NF; ++fm)
#pragma unroll
          for (int fn = 0; fn < NF; ++fn)
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[s & 1][fm], bv[s & 1][fn], acc[fm][fn],
                                                               0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (more) store(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }

    // A lane holds column l32 of each MFMA tile and rows 8*(r/4) + 4*hh +
    // r%4: runs of 4 rows.
#pragma unroll
    for (int fm = 0; fm < NF; ++fm)
#pragma unroll
      for (int fn = 0; fn < NF; ++fn) {
        const int gj = col0 + WT * wn + 32 * fn + l32;
        if (gj >= p.n) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int i0 = row0 + WT * wm + 32 * fm + 8 * g + 4 * hh;
          if (i0 >= p.m) continue;
          const float v[4] = {acc[fm][fn][4 * g], acc[fm][fn][4 * g + 1], acc[fm][fn][4 * g + 2],
                              acc[fm][fn][4 * g + 3]};
          run4(i0, gj, v);
        }
      }
  }
  cycle_record(p.probe, t0, (uint32_t)((bz * gridDim.x + blockIdx.x) * 4 + wave), wave);
}

__device__ __forceinline__ int64_t blas_index(int i, int n, int inc) {
  return inc > 0 ? (int64_t)i * inc : (int64_t)(n - 1 - i) * (int64_t)(-inc);
}

// Level-1/2 kernels run 256-thread workgroups; with a cycle probe attached
// every wave writes slot blockIdx*4 + wave, like the GEMM kernels.
__device__ __forceinline__ void l12_record(grxCycleSlot* probe, uint64_t t0) {
  cycle_record(probe, t0, blockIdx.x * 4 + (threadIdx.x >> 6), threadIdx.x >> 6);
}

__global__ void saxpy_kernel(int n, float alpha, const float* x, int incx, float* y, int incy,
                             grxCycleSlot* probe) {
  const uint64_t t0 = probe ? cycle_now() : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t xi = blas_index((int)i, n, incx), yi = blas_index((int)i, n, incy);
    y[yi] = fmaf(alpha, x[xi], y[yi]);
  }
  l12_record(probe, t0);
}

__global__ void sscal_kernel(int n, float alpha, float* x, int incx, grxCycleSlot* probe) {
  const uint64_t t0 = probe ? cycle_now() : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    x[(int64_t)i * incx] *= alpha;
  l12_record(probe, t0);
}

// y = alpha*A*x + beta*y (A m x n col-major): one thread per output row; the
// column walk keeps lanes on consecutive rows of A, so each step coalesces.
__global__ void sgemv_n_kernel(int m, int n, float alpha, const float* A, int lda,
                               const float* x, int incx, float beta, float* y, int incy,
                               grxCycleSlot* probe) {
  const uint64_t t0 = probe ? cycle_now() : 0;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < m) {
    float acc = 0.0f;
    for (int j = 0; j < n; ++j) acc = fmaf(A[(int64_t)j * lda + i], x[blas_index(j, n, incx)], acc);
    const int64_t yi = blas_index(i, m, incy);
    y[yi] = (beta == 0.0f) ? alpha * acc : fmaf(beta, y[yi], alpha * acc);
  }
  l12_record(probe, t0);
}

// y = alpha*A^T*x + beta*y: one 256-thread workgroup per output, the lanes
// stride down a column of A together and reduce in LDS.
__global__ __launch_bounds__(256) void sgemv_t_kernel(int m, int n, float alpha, const float* A,
                                                      int lda, const float* x, int incx, float beta,
                                                      float* y, int incy, grxCycleSlot* probe) {
  const uint64_t t0 = probe ? cycle_now() : 0;
  __shared__ float part[4];
  const int j = blockIdx.x;
  float acc = 0.0f;
  for (int i = threadIdx.x; i < m; i += 256)
    acc = fmaf(A[(int64_t)j * lda + i], x[blas_index(i, m, incx)], acc);
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float t = (part[0] + part[1]) + (part[2] + part[3]);
    const int64_t yi = blas_index(j, n, incy);
    y[yi] = (beta == 0.0f) ? alpha * t : fmaf(beta, y[yi], alpha * t);
  }
  l12_record(probe, t0);
}

}  // namespace

hipError_t launch_sgemm(const SgemmDesc& d, hipStream_t s) {
  SParams p{};
  p.a = d.a; p.b = d.b; p.c = d.c;
  p.lda = d.lda; p.ldb = d.ldb; p.ldc = d.ldc;
  p.sa = d.stride_a; p.sb = d.stride_b; p.sc = d.stride_c;
  p.m = d.m; p.n = d.n; p.k = d.k;
  p.ta = d.ta; p.tb = d.tb;
  p.alpha = d.alpha; p.beta = d.beta;
  p.probe = d.probe;
  if (d.batch > 65535) return hipErrorInvalidValue;
  // 128-wide tiles once they fill the chip, 64-wide below that, 32-wide
  // where 64-wide tiles would leave half the CUs idle (without a cycle
  // probe, whose slots are counted for 64x64 tiles).
  const int64_t big = ((int64_t)(d.m + 127) / 128) * ((d.n + 127) / 128) * d.batch;
  const int64_t mid = ((int64_t)(d.m + 63) / 64) * ((d.n + 63) / 64) * d.batch;
  const int mt = big >= 256 ? 128 : (mid >= 128 || d.probe ? 64 : 32);
  p.tiles_m = (d.m + mt - 1) / mt;
  const int64_t tiles = (int64_t)p.tiles_m * ((d.n + mt - 1) / mt);
  if (tiles > 0x7fffffff) return hipErrorInvalidValue;
  const bool vec = d.lda % 4 == 0 && d.ldb % 4 == 0 && d.stride_a % 4 == 0 && d.stride_b % 4 == 0 &&
                   (uintptr_t)d.a % 16 == 0 && (uintptr_t)d.b % 16 == 0;
  const dim3 grid((unsigned)tiles, 1, (unsigned)d.batch);
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, p); };
  const int sel = (mt == 128 ? 8 : mt == 32 ? 16 : 0) | (vec ? 4 : 0) | (d.ta ? 2 : 0) | (d.tb ? 1 : 0);
  switch (sel) {
    case 16: go(sgemm_mfma<32, false, false, false>); break;
    case 17: go(sgemm_mfma<32, false, false, true>); break;
    case 18: go(sgemm_mfma<32, false, true, false>); break;
    case 19: go(sgemm_mfma<32, false, true, true>); break;
    case 20: go(sgemm_mfma<32, true, false, false>); break;
    case 21: go(sgemm_mfma<32, true, false, true>); break;
    case 22: go(sgemm_mfma<32, true, true, false>); break;
    case 23: go(sgemm_mfma<32, true, true, true>); break;
    case 0:  go(sgemm_mfma<64, false, false, false>); break;
    case 1:  go(sgemm_mfma<64, false, false, true>); break;
    case 2:  go(sgemm_mfma<64, false, true, false>); break;
    case 3:  go(sgemm_mfma<64, false, true, true>); break;
    case 4:  go(sgemm_mfma<64, true, false, false>); break;
    case 5:  go(sgemm_mfma<64, true, false, true>); break;
    case 6:  go(sgemm_mfma<64, true, true, false>); break;
    case 7:  go(sgemm_mfma<64, true, true, true>); break;
    case 8:  go(sgemm_mfma<128, false, false, false>); break;
    case 9:  go(sgemm_mfma<128, false, false, true>); break;
    case 10: go(sgemm_mfma<128, false, true, false>); break;
    case 11: go(sgemm_mfma<128, false, true, true>); break;
    case 12: go(sgemm_mfma<128, true, false, false>); break;
    case 13: go(sgemm_mfma<128, true, false, true>); break;
    case 14: go(sgemm_mfma<128, true, true, false>); break;
    case 15: go(sgemm_mfma<128, true, true, true>); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int64_t l1_blocks(int n) { return std::min<int64_t>(((int64_t)n + 255) / 256, 65536); }

int64_t sgemv_blocks(bool trans, int m, int n) { return trans ? n : ((int64_t)m + 255) / 256; }

hipError_t launch_saxpy(int n, float alpha, const float* x, int incx, float* y, int incy,
                        grxCycleSlot* probe, hipStream_t s) {
  hipLaunchKernelGGL(saxpy_kernel, dim3((unsigned)l1_blocks(n)), dim3(256), 0, s, n, alpha, x, incx,
                     y, incy, probe);
  return hipGetLastError();
}

hipError_t launch_sscal(int n, float alpha, float* x, int incx, grxCycleSlot* probe,
                        hipStream_t s) {
  hipLaunchKernelGGL(sscal_kernel, dim3((unsigned)l1_blocks(n)), dim3(256), 0, s, n, alpha, x, incx,
                     probe);
  return hipGetLastError();
}

hipError_t launch_sgemv(bool trans, int m, int n, float alpha, const float* A, int lda,
                        const float* x, int incx, float beta, float* y, int incy,
                        grxCycleSlot* probe, hipStream_t s) {
  const unsigned blocks = (unsigned)sgemv_blocks(trans, m, n);
  if (!trans) {
    hipLaunchKernelGGL(sgemv_n_kernel, dim3(blocks), dim3(256), 0, s, m, n, alpha, A, lda, x, incx,
                       beta, y, incy, probe);
  } else {
    hipLaunchKernelGGL(sgemv_t_kernel, dim3(blocks), dim3(256), 0, s, m, n, alpha, A, lda, x, incx,
                       beta, y, incy, probe);
  }
  return hipGetLastError();
}

}  // namespace grxk
