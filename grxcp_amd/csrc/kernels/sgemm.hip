// grxBLAS fp32 kernels on gfx950: Sgemm / SgemmStridedBatched, and the
// level-1/2 routines (saxpy, sscal, sgemv).
//
// Sgemm replaces the reference's one-thread-per-output kernel
// (ref: src/libs/grxblas/kernels/sgemm.cpp:22-89; 2 global loads per
// multiply-add) with an LDS-tiled kernel: a 64x64 tile of C per 256-thread
// workgroup, 4x4 outputs per thread, 16-deep K stages staged through LDS with
// guarded loads that apply op() while staging (all four transposes, ragged
// shapes, any leading dimension). The batch is the grid's z dimension with
// signed element strides (a zero stride broadcasts an operand), exactly the
// reference's one-launch batching (ref: src/libs/grxblas/grxblas.cpp:936-938).
// beta == 0 never reads C (ref: kernels/sgemm.cpp:80-85).
//
// Level 1/2 follow the reference's semantics (ref: kernels/blas12.cpp:41-132):
// BLAS increments (negative walks backwards), sgemv beta == 0 never reads y.

#include "../launch.h"
#include "device_common.h"

namespace grxk {
namespace {

constexpr int kT = 64;   // C tile edge
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

__global__ __launch_bounds__(256) void sgemm_tiled(SParams p) {
  __shared__ float As[kK][kT + 4];   // As[kk][i] = op(A)[row0+i][k0+kk]
  __shared__ float Bs[kK][kT + 4];   // Bs[kk][j] = op(B)[k0+kk][col0+j]

  const uint64_t t0 = p.probe ? cycle_now() : 0;
  const int tid = threadIdx.x;
  const int tm = blockIdx.x % p.tiles_m;
  const int tn = blockIdx.x / p.tiles_m;
  const int row0 = tm * kT, col0 = tn * kT;
  const int64_t bz = blockIdx.z;
  const float* A = p.a + bz * p.sa;
  const float* B = p.b + bz * p.sb;
  float* C = p.c + bz * p.sc;

  // Thread (ti, tj) owns rows ti + 16*r and columns tj + 16*c: consecutive
  // lanes own consecutive rows, so C stores coalesce along its columns.
  const int ti = tid & 15, tj = tid >> 4;
  float acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = 0.0f;

  for (int k0 = 0; k0 < p.k; k0 += kK) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = tid + 256 * q;   // 1024 elements per operand stage
      // op(A): stored m x k (N, contiguous in i) or k x m (T, contiguous in k)
      int i, kk;
      if (p.ta) { kk = e % kK; i = e / kK; } else { i = e % kT; kk = e / kT; }
      const int gi = row0 + i, gk = k0 + kk;
      float va = 0.0f;
      if (gi < p.m && gk < p.k)
        va = p.ta ? A[(int64_t)gi * p.lda + gk] : A[(int64_t)gk * p.lda + gi];
      As[kk][i] = va;
      // op(B): stored k x n (N, contiguous in k) or n x k (T, contiguous in j)
      int j;
      if (!p.tb) { kk = e % kK; j = e / kK; } else { j = e % kT; kk = e / kT; }
      const int gj = col0 + j;
      const int gk2 = k0 + kk;
      float vb = 0.0f;
      if (gj < p.n && gk2 < p.k)
        vb = p.tb ? B[(int64_t)gk2 * p.ldb + gj] : B[(int64_t)gj * p.ldb + gk2];
      Bs[kk][j] = vb;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) av[r] = As[kk][ti + 16 * r];
#pragma unroll
      for (int c = 0; c < 4; ++c) bv[c] = Bs[kk][tj + 16 * c];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(av[r], bv[c], acc[r][c]);
    }
    __syncthreads();
  }

#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int gj = col0 + tj + 16 * c;
    if (gj >= p.n) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gi = row0 + ti + 16 * r;
      if (gi >= p.m) continue;
      float* cp = C + (int64_t)gj * p.ldc + gi;
      const float s = __fmul_rn(p.alpha, acc[r][c]);
      *cp = (p.beta == 0.0f) ? s : __fadd_rn(s, __fmul_rn(p.beta, *cp));
    }
  }
  cycle_record(p.probe, t0,
               (uint32_t)((bz * gridDim.x + blockIdx.x) * 4 + (tid >> 6)), tid >> 6);
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
  p.tiles_m = (d.m + kT - 1) / kT;
  const int64_t tiles = (int64_t)p.tiles_m * ((d.n + kT - 1) / kT);
  if (tiles > 0x7fffffff || d.batch > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sgemm_tiled, dim3((unsigned)tiles, 1, (unsigned)d.batch), dim3(256), 0, s, p);
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
