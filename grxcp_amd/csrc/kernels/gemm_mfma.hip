// grxBLAS GemmEx on gfx950 matrix cores.
//
// Replaces the reference's tensor-unit GEMM (ref: src/libs/grxblas/kernels/
// hgemm_tcu.cpp:215-372, a single persistent CTA walking 8x4x8 WMMA tiles fed
// by DXA descriptor copies) with two MFMA kernels:
//
//  * gemm_tn_fast: op(A) and op(B) both K-contiguous (transa=T, transb=N in
//    grxBLAS's column-major terms, i.e. row-major A times column-major B). A
//    256x256 macro tile per 256-thread workgroup (4 waves, 128x128 each: 8x8
//    v_mfma 16x16 tiles per wave for bf16/fp16/int8, 4x4 32x32 tiles for
//    fp32), 128 bytes of K per stage (64 bf16/fp16 or 128 int8), two LDS
//    stages of 64 KB, 16-byte buffer loads, an XOR swizzle that keeps
//    ds_read_b128 / ds_write_b128 free of bank conflicts, and an XCD-aware
//    tile order. Ragged m/n are handled by the buffer descriptor's
//    range check (out-of-range rows read as zero) plus masked stores; a ragged
//    k is masked per 16-byte chunk, so k only has to be a multiple of 16 bytes.
//
//  * gemm_general: every transpose combination, any m/n/k, any leading
//    dimension and alignment. 64x64 tiles, element-wise guarded staging into
//    LDS in the same [row][k] layout the matrix cores read, 4 waves of one
//    32x32 MFMA tile each. This is the path the reference's ragged and
//    transposed gate cases exercise.
//
// Both kernels are byte-generic: every matrix-core step consumes 16 bytes of
// A and 16 bytes of B per lane (8 bf16/fp16 or 16 int8 in one v_mfma, 4 fp32
// in four v_mfma_f32_32x32x2_f32) and produces the same 32x32 accumulator
// layout, so one body serves all four input types; gemm_tn_fast's 16x16
// path likewise for the 16-bit and int8 types. fp32 serves Sgemm's problems
// that fill the GPU (grxblas.cpp sgemm_batched).
//
// Accumulator layouts (verified on gfx950 by tests/test_gpu_gemm.py): 32x32
// MFMA, lane l, element r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32;
// 16x16 MFMA, row 4*(l/16) + r, column l%16.

#include "../launch.h"
#include "device_common.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

namespace grxk {
namespace {

// ---------------------------------------------------------------------------
// matrix-core ops: 16 bytes of A and B per lane, 32x32 output per wave
// ---------------------------------------------------------------------------

struct OpBF16 {
  static constexpr const char* kName = "bf16";
  using Acc = f32x16;
  using Elem = float;
  static constexpr int kElemBytes = 2;
  __device__ static Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // gemm_tn_fast: 16x16 tiles, accumulated in place in AGPRs (assembly, so
  // that the register allocator cannot move an accumulator between k-steps:
  // with the builtin it copied 80 of them per loop trip).
  static constexpr bool kM16 = true;
  using Acc16 = f32x4;
  __device__ static void mma16(i32x4 a, i32x4 b, Acc16& c) {
    asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};

struct OpF16 {
  static constexpr const char* kName = "f16";
  using Acc = f32x16;
  using Elem = float;
  static constexpr int kElemBytes = 2;
  __device__ static Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // gemm_tn_fast: 16x16 tiles, accumulated in place in AGPRs (assembly, so
  // that the register allocator cannot move an accumulator between k-steps:
  // with the builtin it copied 80 of them per loop trip).
  static constexpr bool kM16 = true;
  using Acc16 = f32x4;
  __device__ static void mma16(i32x4 a, i32x4 b, Acc16& c) {
    asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};

struct OpI8 {
  static constexpr const char* kName = "i8";
  using Acc = i32x16;
  using Elem = int;
  static constexpr int kElemBytes = 1;
  __device__ static Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  // gemm_tn_fast: 16x16 tiles, accumulated in place in AGPRs (assembly, so
  // that the register allocator cannot move an accumulator between k-steps:
  // with the builtin it copied 80 of them per loop trip).
  static constexpr bool kM16 = true;
  using Acc16 = i32x4;
  __device__ static void mma16(i32x4 a, i32x4 b, Acc16& c) {
    asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};

// fp32 (Sgemm): a 16-byte fragment is 4 floats, k = 4*(lane/32) + s of an
// 8-float slice of K; v_mfma_f32_32x32x2_f32 step s pairs k = s (lanes 0-31)
// with k = 4 + s (lanes 32-63), so 4 steps cover the slice.
struct OpF32 {
  static constexpr const char* kName = "f32";
  using Acc = f32x16;
  using Elem = float;
  static constexpr int kElemBytes = 4;
  __device__ static Acc mma(i32x4 a, i32x4 b, Acc c) {
    // Whole-vector casts: a bit cast of one element (a[s]) reads element 0.
    const f32x4 af = __builtin_bit_cast(f32x4, a), bf = __builtin_bit_cast(f32x4, b);
#pragma unroll
    for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s], bf[s], c, 0, 0, 0);
    return c;
  }
  // gemm_tn_fast keeps 32x32 tiles for fp32 (with v_mfma_f32_16x16x4 one
  // wave per SIMD runs out of registers).
  static constexpr bool kM16 = false;
};

struct KParams {
  const uint8_t* a;
  const uint8_t* b;
  void* c;
  int64_t lda, ldb, ldc;  // elements
  int m, n, k;
  int tiles_m, tiles_n;
  int ta, tb;             // general kernel only
  float alpha, beta;
  int32_t ialpha, ibeta;
  int64_t sa, sb, sc;     // batch strides in bytes (grid.y is the batch)
  int k_last;             // split-K: k of the last grid.y slice (0: every slice has k)
  const float* scale;
  grxCycleSlot* probe;
  int group;              // tile-rows per group of the XCD-aware tile order
};

// ---------------------------------------------------------------------------
// epilogue. C is column-major, so a run of consecutive rows i0.. of one column
// j is contiguous. Each Epi writes one element (put) or a full aligned run of
// kRun elements, 16 bytes, with one vector access (put_run). Runs are stored
// with the non-temporal (streaming) hint. Every CU finishes its tile at about
// the same time, so C leaves as a burst of 256 tiles while the matrix cores
// idle; with the hint the bursts cost less (measured: +4 % on int8 with a
// 4096x28672 C, +11 % at 16384^2 x 1024, +1-2 % at 8192^3). Split-K
// partials, which the reduction reads back at once, take plain stores.
// ---------------------------------------------------------------------------

// One 16-byte run of C: streamed (non-temporal) unless STREAM is false, for
// an output that is read back right away (split-K partials).
template <bool STREAM, class V>
__device__ __forceinline__ void put16(void* c, V o) {
  if constexpr (STREAM) __builtin_nontemporal_store(o, (V*)c);
  else *(V*)c = o;
}

template <MmaOut OUT>
struct Epi;

template <>
struct Epi<MmaOut::F32> {
  using T = float;
  static constexpr int kRun = 4;
  __device__ static float apply(const KParams& p, float acc, float c_old) {
    // alpha*acc (+ beta*C) with each operation rounded separately, as the
    // reference's CPU gate writes it (no contraction into an FMA).
    const float s = __fmul_rn(p.alpha, acc);
    return p.beta == 0.0f ? s : __fadd_rn(s, __fmul_rn(p.beta, c_old));
  }
  __device__ static void put(const KParams& p, T* c, float v, int) {
    *c = apply(p, v, p.beta != 0.0f ? *c : 0.0f);
  }
  template <bool STREAM = true>
  __device__ static void put_run(const KParams& p, T* c, const float* v, int) {
    f32x4 o;
    if (p.beta == 0.0f) {
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = __fmul_rn(p.alpha, v[q]);
    } else {
      const f32x4 old = *(const f32x4*)c;
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = apply(p, v[q], old[q]);
    }
    put16<STREAM>(c, o);
  }
};

template <MmaOut OUT>
struct EpiNarrow {
  using T = uint16_t;
  static constexpr int kRun = 8;
  __device__ static uint16_t cvt(float x) {
    if constexpr (OUT == MmaOut::BF16) return f32_to_bf16(x);
    else return f32_to_f16(x);
  }
  __device__ static float back(uint16_t x) {
    if constexpr (OUT == MmaOut::BF16) return bf16_to_f32(x);
    else return f16_to_f32(x);
  }
  __device__ static float apply(const KParams& p, float acc, uint16_t c_old) {
    const float s = __fmul_rn(p.alpha, acc);
    return p.beta == 0.0f ? s : __fadd_rn(s, __fmul_rn(p.beta, back(c_old)));
  }
  __device__ static void put(const KParams& p, T* c, float v, int) {
    *c = cvt(apply(p, v, p.beta != 0.0f ? *c : (uint16_t)0));
  }
  __device__ static uint32_t pack(float a, float b) {
    if constexpr (OUT == MmaOut::BF16) return pack_bf16x2(a, b);
    else return pack_f16x2(a, b);
  }
  template <bool STREAM = true>
  __device__ static void put_run(const KParams& p, T* c, const float* v, int) {
    u32x4 o;
    if (p.beta == 0.0f) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
        o[h] = pack(__fmul_rn(p.alpha, v[2 * h]), __fmul_rn(p.alpha, v[2 * h + 1]));
    } else {
      const u32x4 old = *(const u32x4*)c;
#pragma unroll
      for (int h = 0; h < 4; ++h)
        o[h] = pack(apply(p, v[2 * h], (uint16_t)(old[h] & 0xffff)),
                    apply(p, v[2 * h + 1], (uint16_t)(old[h] >> 16)));
    }
    put16<STREAM>(c, o);
  }
};
template <> struct Epi<MmaOut::BF16> : EpiNarrow<MmaOut::BF16> {};
template <> struct Epi<MmaOut::F16> : EpiNarrow<MmaOut::F16> {};

template <>
struct Epi<MmaOut::I32> {
  using T = int;
  static constexpr int kRun = 4;
  __device__ static int apply(const KParams& p, int acc, int c_old) {
    uint32_t r = (uint32_t)p.ialpha * (uint32_t)acc;
    if (p.ibeta != 0) r += (uint32_t)p.ibeta * (uint32_t)c_old;
    return (int)r;
  }
  __device__ static void put(const KParams& p, T* c, int v, int) {
    *c = apply(p, v, p.ibeta != 0 ? *c : 0);
  }
  template <bool STREAM = true>
  __device__ static void put_run(const KParams& p, T* c, const int* v, int) {
    i32x4 old = {0, 0, 0, 0};
    if (p.ibeta != 0) old = *(const i32x4*)c;
    i32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = apply(p, v[q], old[q]);
    put16<STREAM>(c, o);
  }
};

template <>
struct Epi<MmaOut::DEQ_BF16> {
  using T = uint16_t;
  static constexpr int kRun = 8;
  // bf16_rne(f32_rne(f32_rne(acc) * scale[j])): v_cvt_f32_i32 rounds to
  // nearest even, __fmul_rn is one correctly rounded product.
  __device__ static uint16_t apply(float s, int acc) {
    return f32_to_bf16(__fmul_rn((float)acc, s));
  }
  __device__ static void put(const KParams& p, T* c, int v, int j) { *c = apply(p.scale[j], v); }
  template <bool STREAM = true>
  __device__ static void put_run(const KParams& p, T* c, const int* v, int j) {
    put_run_scaled<STREAM>(c, v, p.scale[j]);
  }
  // The same with column j's scale already in a register.
  template <bool STREAM = true>
  __device__ static void put_run_scaled(T* c, const int* v, float s) {
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h)
      o[h] = pack_bf16x2(__fmul_rn((float)v[2 * h], s), __fmul_rn((float)v[2 * h + 1], s));
    put16<STREAM>(c, o);
  }
};

// `count` consecutive rows i0.. of column j (j < n). With `vec`, the caller
// guarantees a run of kRun elements starting at i0 is 16-byte aligned.
template <MmaOut OUT, bool STREAM = true, class E>
__device__ __forceinline__ void store_run(const KParams& p, int i0, int j, const E* v, int count,
                                          bool vec) {
  using P = Epi<OUT>;
  typename P::T* c = (typename P::T*)p.c + (int64_t)j * p.ldc + i0;
  if (vec && count == P::kRun && i0 + P::kRun <= p.m) {
    P::template put_run<STREAM>(p, c, v, j);
  } else {
    for (int q = 0; q < count; ++q)
      if (i0 + q < p.m) P::put(p, c + q, v[q], j);
  }
}

// Spread a 32x32 accumulator tile (rows base_i.., cols base_j..) to C, four
// rows per lane and store (general path: no alignment assumed).
template <class Op, MmaOut OUT>
__device__ __forceinline__ void store_acc_tile(const KParams& p, const typename Op::Acc& acc,
                                               int base_i, int base_j, int lane) {
  using E = typename Op::Elem;
  const int j = base_j + (lane & 31);
  if (j >= p.n) return;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int i0 = base_i + 8 * g + 4 * (lane >> 5);
    if (i0 >= p.m) continue;
    E v[4] = {(E)acc[4 * g + 0], (E)acc[4 * g + 1], (E)acc[4 * g + 2], (E)acc[4 * g + 3]};
    store_run<OUT>(p, i0, j, v, 4, false);
  }
}

// 32-bit reinterpretation through a by-value copy. (hipcc lowers
// __builtin_bit_cast applied directly to an element of an ext_vector_type
// as a cast of element 0, so vector elements always pass through these.)
template <int N>
struct IntC { static constexpr int value = N; };

template <class T>
__device__ __forceinline__ int bits_of(T x) { return __builtin_bit_cast(int, x); }
template <class T>
__device__ __forceinline__ T from_bits(int x) { return __builtin_bit_cast(T, x); }

// The problem of batch blockIdx.y: operands and C moved by its strides. A
// split-K launch uses the same mechanism: slice z reads K range
// [z*k, (z+1)*k) (the last one k_last long) and writes its own partial C.
__device__ __forceinline__ KParams batch_view(const KParams& in) {
  KParams p = in;
  const int64_t z = blockIdx.y;
  p.a += z * in.sa;
  p.b += z * in.sb;
  p.c = (uint8_t*)in.c + z * in.sc;
  if (in.k_last && blockIdx.y == gridDim.y - 1) p.k = in.k_last;
  return p;
}

// Probe slot of a wave: workgroups of all batches in launch order.
__device__ __forceinline__ int64_t probe_slot(int wave) {
  return ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * 4 + wave;
}

// XCD-aware tile order. Consecutive workgroup ids are dispatched round-robin
// over the 8 XCDs; remapping gives each XCD a contiguous run of logical tiles,
// and the logical order walks groups of `kgroup` tile-rows (8 by default) so
// that neighbours share A and B panels in that XCD's L2: 32 concurrent tiles
// per XCD as 8 rows x 4 columns stream 12 operand panels per round, the
// fewest for 32 tiles (8192^3 bf16: FETCH_SIZE 1.61 GB per launch against
// 2.47 GB for 16 x 2 and 4.45 GB for 32 x 1, which cost 0 % and 4 % of the
// rate: the L2 egress is not what bounds this kernel).
__device__ __forceinline__ void map_tile(int bid, int nblocks, int tiles_m, int tiles_n,
                                         int kgroup, int& tm, int& tn) {
  int logical = bid;
  if ((nblocks & 7) == 0) logical = (bid & 7) * (nblocks >> 3) + (bid >> 3);
  const int kGroup = kgroup > 0 ? kgroup : 8;
  const int per_group = kGroup * tiles_n;
  const int group = logical / per_group;
  const int first_m = group * kGroup;
  const int gsize = min(tiles_m - first_m, kGroup);
  const int in_group = logical - group * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// ---------------------------------------------------------------------------
// TN fast path
// ---------------------------------------------------------------------------

constexpr int kFastTile = 256;   // rows of op(A) and columns of op(B) per workgroup
constexpr int kFastKBytes = 128; // bytes of K per stage
constexpr int kChunks = kFastKBytes / 16;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }
// gemm_tn128's [k][m] layout of an M-contiguous A: 16-byte chunk XOR for
// k-row k of a stage.
__device__ __forceinline__ int an_swz(int k) { return 2 * ((k & 3) | ((k >> 2) & 4)); }
// The same for int8 (k-rows of 128 bytes, 8 chunks): ((k >> 1) & 3) | bit 5
// of k in bit 2.
__device__ __forceinline__ int an_swz8(int k) { return ((k >> 1) & 3) | ((k >> 3) & 4); }
template <int EB> __device__ __forceinline__ int nswz(int k) { return EB == 2 ? an_swz(k) : an_swz8(k); }
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <class Op, MmaOut OUT, bool STREAM = true>
__global__ __launch_bounds__(256, 1) void gemm_tn_fast(KParams batch_p) {
  const KParams p = batch_view(batch_p);
  // [A | B][stage][row * 8 + physical chunk], 16 bytes per entry: 128 KB.
  // Operand-major, so the two stages of one operand are 32 KB apart: an
  // offset that fits the immediate field of ds_read.
  __shared__ __attribute__((aligned(1024))) i32x4 lds[2][2][kFastTile * kChunks];

  const uint64_t t0 = p.probe ? cycle_now() : 0;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  int tm, tn;
  map_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, p.group, tm, tn);
  const int row0 = tm * kFastTile;
  const int col0 = tn * kFastTile;

  const int lda_b = (int)(p.lda * Op::kElemBytes);
  const int ldb_b = (int)(p.ldb * Op::kElemBytes);
  const int kbytes = p.k * Op::kElemBytes;
  const int ktiles = (kbytes + kFastKBytes - 1) / kFastKBytes;

  // Buffer descriptors start at this tile's first row; the record count ends
  // at row m (n), so rows past the matrix read as zero without a branch, and
  // an offset of 2^31 (always past the end) reads zero for a masked k chunk.
  const int rows_a = min(kFastTile, p.m - row0);
  const int rows_b = min(kFastTile, p.n - col0);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.a + (int64_t)row0 * lda_b), (short)0, (rows_a - 1) * lda_b + kbytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.b + (int64_t)col0 * ldb_b), (short)0, (rows_b - 1) * ldb_b + kbytes, kRsrcWord3);
  constexpr uint32_t kOff = 0x80000000u;

  // Direct-to-LDS staging (buffer_load_dwordx4 ... lds): instruction i of
  // wave w fills the 1 KB block of rows 8*(4i+w) .. +7, lane L landing in
  // row +L/8 at physical chunk L%8. The swizzle is applied on the global
  // side: that lane fetches logical chunk (L%8) ^ swz(row). No VGPRs hold
  // the tile, and nothing waits for the data until the stage's barrier.
  const int lr = lane >> 3;
  const int pc = lane & 7;
  // The stage-invariant part of each DMA's offset (row and swizzled chunk),
  // per 8-row block group i and operand. A stage that lies wholly inside K
  // needs no mask: its DMAs pass this offset and the stage's K offset in
  // the instruction's scalar soffset, so the K loop spends no VALU
  // instruction on DMA addresses (measured 2-3 % faster than recomputing and
  // masking every offset per stage).
  uint32_t base_a[8], base_b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int blk = 4 * i + wave;
    const int row = 8 * blk + lr;
    const int c = pc ^ lr ^ (blk & 7);
    base_a[i] = (uint32_t)(row * lda_b + 16 * c);
    base_b[i] = (uint32_t)(row * ldb_b + 16 * c);
  }
  // One DMA instruction: 1 KB (8 rows) of operand `op` for stage kt. `full`
  // (compile-time) says the stage lies wholly inside K. Rows past m/n read
  // zero either way: their stage-invariant offset alone is past the
  // descriptor's record count.
  auto dma = [&](int kt, int st, int i, int op, auto full) {
    const int kb = kt * kFastKBytes;
    const int blk = 4 * i + wave;               // 8-row block index, 0..31
    if constexpr (decltype(full)::value) {
      if (op == 0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&lds[0][st][blk * 64], 16, base_a[i], kb, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)&lds[1][st][blk * 64], 16, base_b[i], kb, 0, 0);
    } else {
      const int c = pc ^ lr ^ (blk & 7);          // == pc ^ swz(row)
      const bool ok = kt < ktiles && kb + 16 * c < kbytes;
      if (op == 0) {
        const uint32_t va = ok ? base_a[i] + (uint32_t)kb : kOff;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&lds[0][st][blk * 64], 16, va, 0, 0, 0);
      } else {
        const uint32_t vb = ok ? base_b[i] + (uint32_t)kb : kOff;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)&lds[1][st][blk * 64], 16, vb, 0, 0, 0);
      }
    }
  };

  const int wm = wave >> 1;
  const int wn = wave & 1;
  typedef __attribute__((address_space(3))) const i32x4* lds_frag_t;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)&lds[0][0][0];
  constexpr uint32_t kStageBytes = kFastTile * kChunks * 16;    // 32 KB

  // A stage is 16 DMA instructions, d = 0..15: 8-row block group
  // 4*(d/8) + d%4 of operand (d/4)%2.
  auto dma_d = [&](int kt, int st, int d, auto full) __attribute__((always_inline)) {
    dma(kt, st, 4 * (d >> 3) + (d & 3), (d >> 2) & 1, full);
  };
  // While the stages an iteration loads lie wholly inside K, its DMAs need
  // no mask and its stage is known at compile time (two iterations per
  // trip); the rest take the masked form.
  const int kfull = kbytes / kFastKBytes;

  // Epilogue through LDS. A lane's accumulators are 4-row pieces of 16 or 32
  // different columns; stored as they are, every vector store would touch
  // that many cache lines 16 bytes at a time. Instead each wave parks one
  // 128x32 column block of raw 32-bit accumulators in its own LDS region
  // ([col][row], pitch 132 words; `park` writes it) and reads it back as
  // runs of kRun rows of one column, so one store instruction writes whole
  // 256-byte (or 512-byte) column segments. Rows 64..127 sit 4 words further
  // on (row r at r + 4*(r/64 & 1)): that keeps the 16 lanes of one column on
  // distinct banks when they read their runs, with every offset on the
  // write side a compile-time constant.
  using E = typename Op::Elem;
  constexpr int kRun = Epi<OUT>::kRun;            // 8 (16-bit C) or 4 (32-bit C)
  constexpr int kPitch = 128 + 4;
  constexpr int kLanesPerCol = 128 / kRun;        // 16 or 32
  constexpr int kColsPerRound = 64 / kLanesPerCol;
  int* stage = (int*)&lds[0][0][0] + wave * 32 * kPitch;   // 16.5 KB per wave
  auto epilogue = [&](auto park) __attribute__((always_inline)) {
    const int run = lane % kLanesPerCol;
    const int rcol = lane / kLanesPerCol;
    const int run_pos = run * kRun + 4 * ((run * kRun >> 6) & 1);
    const int gi = row0 + wm * 128 + run * kRun;
    // One column block per call; J is a compile-time constant so that the
    // accumulators stay in registers (a run-time index would move them to
    // scratch).
    auto column_block = [&](auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      park(jc);
      // LDS operations of one wave complete in order; the compiler only must
      // not move the reads above the writes (or the next writes above them).
      asm volatile("" ::: "memory");
      auto read_run = [&](int col, E* v) __attribute__((always_inline)) {
        const int* src = &stage[col * kPitch + run_pos];
#pragma unroll
        for (int h = 0; h < kRun / 4; ++h) {
          const i32x4 w = *(const i32x4*)(src + 4 * h);
#pragma unroll
          for (int q = 0; q < 4; ++q) v[4 * h + q] = from_bits<E>(w[q]);
        }
      };
      const int gj0 = col0 + wn * 128 + 32 * j;
      if (row0 + wm * 128 + 128 <= p.m && gj0 + 32 <= p.n) {
        // Interior block (the common case): unrolled, no masks.
        using T = typename Epi<OUT>::T;
        T* cbase = (T*)p.c + (int64_t)gj0 * p.ldc + gi;
#pragma unroll
        for (int rd = 0; rd < 32 / kColsPerRound; ++rd) {
          const int col = rd * kColsPerRound + rcol;
          E v[kRun];
          read_run(col, v);
          Epi<OUT>::template put_run<STREAM>(p, cbase + (int64_t)col * p.ldc, v, gj0 + col);
        }
      } else {
        for (int rd = 0; rd < 32 / kColsPerRound; ++rd) {
          const int col = rd * kColsPerRound + rcol;
          E v[kRun];
          read_run(col, v);
          const int gj = gj0 + col;
          if (gj < p.n && gi < p.m) store_run<OUT, STREAM>(p, gi, gj, v, kRun, true);
        }
      }
      asm volatile("" ::: "memory");
    };
    column_block(IntC<0>{});
    column_block(IntC<1>{});
    column_block(IntC<2>{});
    column_block(IntC<3>{});
  };

  if constexpr (Op::kM16) {
    // 16-bit and int8 inputs: 8 x 8 tiles of 16x16 per wave, 64-byte
    // k-steps (two per stage). Against 4 x 4 tiles of 32x32 (the fp32 path
    // below) the same operand bytes move, and the matrix cores draw less
    // power per FLOP: rocprofv3 over bf16 8192^3 read the same matrix-busy
    // cycles at a 1.91 GHz clock against 1.65 (+7.5 % sustained).
    using Acc = typename Op::Acc16;
    Acc acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = 0;
    const int r16 = lane & 15;
    // The k-step's four 16-byte chunks go to the four 16-lane groups in the
    // order 0, 2, 1, 3 (A and B alike, so every product is unchanged): a
    // ds_read_b128 serves 32 lanes at a time, and under the row swizzle
    // chunks c and c+2 of rows 0-15 land on distinct banks where c and c+1
    // would share them (rocprofv3: 6.8e7 bank-conflict cycles per launch at
    // 8192^3 in the plain order, none here).
    const int kq = ((lane >> 3) & 2) | ((lane >> 5) & 1);

    // Fragment reads: A rows wm*128 + 16t + r16, B rows wn*128 + 16t + r16,
    // 16 bytes at logical chunk 4*ks + kq. A fragments roll: the next
    // k-step's fragment t is read into the same registers once row t's last
    // MFMA has issued. B fragments are double-buffered. The LDS byte address
    // of every stage-0 fragment is computed once; stage 1 adds 32 KB, in the
    // instruction's offset field where the stage is a compile-time constant.
    i32x4 fa[8], fb[2][8];
    uint32_t ad_a[8][2], ad_b[8][2];                               // stage 0, [tile][k-step]
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int kc = 4 * ks + kq;
        const int ar = wm * 128 + t * 16 + r16;
        const int br = wn * 128 + t * 16 + r16;
        ad_a[t][ks] = lds0 + 16u * (uint32_t)(ar * kChunks + (kc ^ swz(ar)));
        ad_b[t][ks] = lds0 + 2 * kStageBytes + 16u * (uint32_t)(br * kChunks + (kc ^ swz(br)));
      }
    auto frag_a = [&](auto st, int ks, int t) __attribute__((always_inline)) {
      if constexpr (std::is_integral<decltype(st)>::value)
        fa[t] = *(lds_frag_t)(uintptr_t)(ad_a[t][ks] + (uint32_t)st * kStageBytes);
      else
        fa[t] = *(lds_frag_t)(uintptr_t)(ad_a[t][ks] + decltype(st)::value * kStageBytes);
    };
    auto frag_b = [&](auto st, int ks, int buf, int t) __attribute__((always_inline)) {
      if constexpr (std::is_integral<decltype(st)>::value)
        fb[buf][t] = *(lds_frag_t)(uintptr_t)(ad_b[t][ks] + (uint32_t)st * kStageBytes);
      else
        fb[buf][t] = *(lds_frag_t)(uintptr_t)(ad_b[t][ks] + decltype(st)::value * kStageBytes);
    };

    // One k-step: 64 MFMAs in 32 slots of one MFMA pair (A row i = q/4).
    // DMA instructions d0 .. d0+cnt-1 are spread evenly, each ahead of its
    // slot's pair; behind the pair, the next k-step's B fragments (the even
    // slots of the first half) and A fragment i (behind row i's last pair).
    // The order is held by sched_barrier.
    auto phase = [&](int buf, auto rd_st, int rd_ks, int dma_kt, int dma_st, int d0, int cnt,
                     auto full) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        const int i = q >> 2;
        // int8: snake order (odd rows walk the B tiles backwards, so
        // consecutive MFMAs always share an operand; config-3 int8 +0.3 %,
        // four interleaved pairs, none slower). The 16-bit types keep the
        // plain order. Every accumulator's k order is the same either way.
        constexpr bool kSnake = std::is_same<Op, OpI8>::value;
        const bool rev = kSnake && (i & 1) != 0;
        const int ja = rev ? 7 - 2 * (q & 3) : 2 * (q & 3);
        const int jb = rev ? ja - 1 : ja + 1;
        if ((q + 1) * cnt / 32 > q * cnt / 32) dma_d(dma_kt, dma_st, d0 + q * cnt / 32, full);
        __builtin_amdgcn_sched_barrier(0);
        Op::mma16(fa[i], fb[buf][ja], acc[i][ja]);
        Op::mma16(fa[i], fb[buf][jb], acc[i][jb]);
        __builtin_amdgcn_sched_barrier(0);
        if ((q & 1) == 0 && q < 16) frag_b(rd_st, rd_ks, buf ^ 1, q >> 1);
        if ((q & 3) == 3) frag_a(rd_st, rd_ks, i);
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    // Stage s lives in LDS buffer s & 1. Iteration kt runs k-step 0 of stage
    // kt, one barrier (stage kt+1 landed, stage kt no longer read), then
    // k-step 1 with stage kt+2's 16 DMAs (into the buffer stage kt just
    // vacated) spread over it, so each load has one to two k-steps of MFMA
    // time to land. (Measured against this: half of the DMAs in the k-step
    // before the barrier, as the fp32 path does with its four k-steps per
    // stage, left the last loads no cover: 67 % matrix-busy against 80 %;
    // all 16 in the first half of the k-step: -5 %.)
#pragma unroll
    for (int d = 0; d < 16; ++d) dma_d(0, 0, d, std::false_type{});
#pragma unroll
    for (int d = 0; d < 16; ++d) dma_d(1, 1, d, std::false_type{});
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");  // stage 0 landed
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      frag_a(IntC<0>{}, 0, t);
      frag_b(IntC<0>{}, 0, 0, t);
    }
    auto iter_c = [&](int kt, auto stage_c) __attribute__((always_inline)) {
      constexpr int cur = decltype(stage_c)::value;
      phase(0, IntC<cur>{}, 1, 0, 0, 0, 0, std::true_type{});
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // stage kt+1 landed
      __syncthreads();
      phase(1, IntC<cur ^ 1>{}, 0, kt + 2, cur, 0, 16, std::true_type{});
    };
    auto iter_r = [&](int kt) __attribute__((always_inline)) {
      const int cur = kt & 1;
      phase(0, cur, 1, 0, 0, 0, 0, std::false_type{});
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // stage kt+1 landed
      __syncthreads();
      phase(1, cur ^ 1, 0, kt + 2, cur, 0, 16, std::false_type{});
    };
    int kt = 0;
    for (; kt + 3 < kfull; kt += 2) {
      iter_c(kt, IntC<0>{});
      iter_c(kt + 1, IntC<1>{});
    }
    for (; kt < ktiles; ++kt) iter_r(kt);
    // The MFMAs are assembly, so the compiler places the epilogue's reads of
    // their results without knowing what wrote them: 18 wait states first.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" ::: "memory");
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");    // no LDS write may outlive the loop
    __syncthreads();                                     // and no wave still reads a stage

    // Lane l holds rows 16i + 4*(l/16) .. +3 of column 16*jj + l%16.
    if constexpr (OUT == MmaOut::DEQ_BF16) {
      // Dequantised int8: each value is scaled and rounded to bf16 in
      // registers (the same correctly rounded operations as
      // Epi<DEQ_BF16>::put_run_scaled, so the bits are unchanged) before it
      // is parked, and the LDS round trip moves half the bytes of the
      // 32-bit form: config-3 int8 2945 -> 2975 TOP/s (+1.0 %, six runs of
      // each in ABBA order, one box). The same for 16-bit C at beta = 0
      // measured -0.2 % (bf16 8192^3) and -0.5 % (4096^3), so those keep
      // the 32-bit park.
      // Per wave, a 128x32 column block at a time: [col][row] bf16, 68
      // words per column. A lane parks 4 rows (8 bytes) of one column per
      // 16x16 tile: the 32 lanes of a ds_write_b64 cycle put columns on
      // banks 4*c and their 4 words beside them, all 64 banks once. Read
      // back as runs of 8 rows (16 bytes), 16 lanes per column: one
      // column's 64 consecutive words per ds_read_b128 cycle.
      {
        constexpr int kPitchH = 64 + 4;
        uint32_t* sh = (uint32_t*)&lds[0][0][0] + wave * 32 * kPitchH;   // 8.5 KB per wave
        const int run = lane & 15;
        const int rcol = lane >> 4;
        const int gr0 = row0 + wm * 128;
        const bool rows_full = gr0 + 128 <= p.m;
        // The 8 column scales this lane parks, loaded together.
        float dsc[4][2];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int gj = col0 + wn * 128 + 32 * j + 16 * h + r16;
            dsc[j][h] = gj < p.n ? p.scale[gj] : 0.0f;
          }
        auto narrow2 = [&](int a, int b, float s) __attribute__((always_inline)) -> uint32_t {
          return pack_bf16x2(__fmul_rn((float)a, s), __fmul_rn((float)b, s));
        };
        auto column_block16 = [&](auto jc) __attribute__((always_inline)) {
          constexpr int j = decltype(jc)::value;
          // This block's accumulators are read only from here on: without
          // the fence the compiler converts later blocks early and spills.
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 8; ++i) asm volatile("" : "+a"(acc[i][2 * j + h]));
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const auto& a = acc[i][2 * j + h];
              u32x2 w;
              w[0] = narrow2(a[0], a[1], dsc[j][h]);
              w[1] = narrow2(a[2], a[3], dsc[j][h]);
              *(u32x2*)&sh[(16 * h + r16) * kPitchH + 8 * i + 2 * (lane >> 4)] = w;
            }
          asm volatile("" ::: "memory");
          const int gj0 = col0 + wn * 128 + 32 * j;
          uint16_t* cb = (uint16_t*)p.c + (int64_t)gj0 * p.ldc + gr0 + 8 * run;
          if (rows_full && gj0 + 32 <= p.n) {
#pragma unroll
            for (int rd = 0; rd < 8; ++rd) {
              const int col = 4 * rd + rcol;
              put16<STREAM>(cb + (int64_t)col * p.ldc, *(const u32x4*)&sh[col * kPitchH + 4 * run]);
            }
          } else {
            for (int rd = 0; rd < 8; ++rd) {
              const int col = 4 * rd + rcol;
              const u32x4 w = *(const u32x4*)&sh[col * kPitchH + 4 * run];
              if (gj0 + col >= p.n) continue;
              for (int q = 0; q < 8; ++q)
                if (gr0 + 8 * run + q < p.m)
                  cb[(int64_t)col * p.ldc + q] = (uint16_t)(w[q >> 1] >> (16 * (q & 1)));
            }
          }
          asm volatile("" ::: "memory");
        };
        column_block16(IntC<0>{});
        column_block16(IntC<1>{});
        column_block16(IntC<2>{});
        column_block16(IntC<3>{});
      }
    } else {
      epilogue([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            i32x4 w;
#pragma unroll
            for (int q = 0; q < 4; ++q) w[q] = bits_of(acc[i][2 * j + h][q]);
            *(i32x4*)&stage[(16 * h + r16) * kPitch + 16 * i + 4 * (lane >> 4) + 4 * (i >> 2)] = w;
          }
      });
    }
  } else {
    // fp32: 4 x 4 tiles of 32x32 per wave, 32-byte k-steps (four per stage).
    using Acc = typename Op::Acc;
    Acc acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    const int r32 = lane & 31;
    const int hh = lane >> 5;

    // Fragment reads: A rows wm*128 + 32t + r32, B rows wn*128 + 32t + r32,
    // 16 bytes at logical chunk 2*ks + hh. Two register sets: the reads for
    // k-step ks+1 are in flight while the 16 MFMAs of k-step ks run. Read
    // slot q follows first use in the next k-step (A0, B0..B3, A1..A3), so
    // each read has at least five MFMA pairs to land before an MFMA needs it.
    // The LDS byte address of every stage-0 fragment a lane reads ([tile]
    // [k-step], A and B) is computed once; a read of stage 1 adds 32 KB in
    // the instruction's offset field. With the stage a compile-time constant
    // (the main loop below is unrolled by two), fragment reads cost no VALU
    // instruction (measured 1-2 % faster than computing each address); the
    // masked tail reads with a run-time stage.
    i32x4 fa[2][4], fb[2][4];
    uint32_t ad_a[4][4], ad_b[4][4];                               // stage 0, [tile][k-step]
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int kc = 2 * ks + hh;
        const int ar = wm * 128 + t * 32 + r32;
        const int br = wn * 128 + t * 32 + r32;
        ad_a[t][ks] = lds0 + 16u * (uint32_t)(ar * kChunks + (kc ^ swz(ar)));
        ad_b[t][ks] = lds0 + 2 * kStageBytes + 16u * (uint32_t)(br * kChunks + (kc ^ swz(br)));
      }
    auto frag = [&](auto st, int ks, int buf, int q) __attribute__((always_inline)) {
      const int t = (q >= 1 && q <= 4) ? q - 1 : (q == 0 ? 0 : q - 4);
      if constexpr (std::is_integral<decltype(st)>::value) {
        const int kc = 2 * ks + hh;
        if (q >= 1 && q <= 4) {
          const int br = wn * 128 + t * 32 + r32;
          fb[buf][t] = lds[1][st][br * kChunks + (kc ^ swz(br))];
        } else {
          const int ar = wm * 128 + t * 32 + r32;
          fa[buf][t] = lds[0][st][ar * kChunks + (kc ^ swz(ar))];
        }
      } else {
        constexpr uint32_t off = decltype(st)::value * kStageBytes;
        if (q >= 1 && q <= 4) fb[buf][t] = *(lds_frag_t)(uintptr_t)(ad_b[t][ks] + off);
        else fa[buf][t] = *(lds_frag_t)(uintptr_t)(ad_a[t][ks] + off);
      }
    };

    // One k-step: 16 MFMAs on register set `buf` in 8 slots of one MFMA
    // pair. In the phases that carry DMA, DMA instructions d0 .. d0+cnt-1
    // are spread evenly over the slots, each issued ahead of its slot's MFMA
    // pair: a DMA issue that waits for the address unit then waits while the
    // previous pair still runs (measured 1-3 % faster than issuing it after
    // the pair; moving the fragment read ahead as well is 3 % slower).
    // Behind every pair one fragment read for the next k-step. The order is
    // held by sched_barrier.
    auto phase = [&](int buf, auto rd_st, int rd_ks, int dma_kt, int dma_st, int d0, int cnt,
                     auto full) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int i = q >> 1;
        const int ja = 2 * (q & 1), jb = ja + 1;
        if ((q + 1) * cnt / 8 > q * cnt / 8) dma_d(dma_kt, dma_st, d0 + q * cnt / 8, full);
        __builtin_amdgcn_sched_barrier(0);
        acc[i][ja] = Op::mma(fa[buf][i], fb[buf][ja], acc[i][ja]);
        acc[i][jb] = Op::mma(fa[buf][i], fb[buf][jb], acc[i][jb]);
        frag(rd_st, rd_ks, buf ^ 1, q);
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    // Stage s lives in LDS buffer s & 1. Iteration kt runs k-steps 0..2 of
    // stage kt, one barrier, then k-step 3. Stage kt+2's DMA (into the
    // buffer stage kt just vacated) is issued half right after that barrier
    // and half during k-step 0 of the next iteration, so each load has two to
    // four k-steps of MFMA time to land before the barrier that publishes it.
    // (Measured: moving part of it into k-step 1 saves less DMA issue time
    // than the late loads then cost at the barrier.)
    constexpr int kDmaD = 8, kDmaA = 8;
#pragma unroll
    for (int d = 0; d < 16; ++d) dma_d(0, 0, d, std::false_type{});
#pragma unroll
    for (int d = 0; d < kDmaD; ++d) dma_d(1, 1, d, std::false_type{});
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaD) : "memory");  // stage 0 landed
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) frag(IntC<0>{}, 0, 0, q);

    auto iter_c = [&](int kt, auto stage_c) __attribute__((always_inline)) {
      constexpr int cur = decltype(stage_c)::value;
      phase(0, IntC<cur>{}, 1, kt + 1, cur ^ 1, kDmaD, kDmaA, std::true_type{});
      phase(1, IntC<cur>{}, 2, 0, 0, 0, 0, std::true_type{});
      phase(0, IntC<cur>{}, 3, 0, 0, 0, 0, std::true_type{});
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // stage kt+1 landed
      __syncthreads();
      phase(1, IntC<cur ^ 1>{}, 0, kt + 2, cur, 0, kDmaD, std::true_type{});
    };
    auto iter_r = [&](int kt) __attribute__((always_inline)) {
      const int cur = kt & 1;
      phase(0, cur, 1, kt + 1, cur ^ 1, kDmaD, kDmaA, std::false_type{});
      phase(1, cur, 2, 0, 0, 0, 0, std::false_type{});
      phase(0, cur, 3, 0, 0, 0, 0, std::false_type{});
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // stage kt+1 landed
      __syncthreads();
      phase(1, cur ^ 1, 0, kt + 2, cur, 0, kDmaD, std::false_type{});
    };
    int kt = 0;
    for (; kt + 3 < kfull; kt += 2) {
      iter_c(kt, IntC<0>{});
      iter_c(kt + 1, IntC<1>{});
    }
    for (; kt < ktiles; ++kt) iter_r(kt);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");    // no LDS write may outlive the loop
    __syncthreads();                                     // and no wave still reads a stage

    // Lane l holds rows 32i + 8g + 4*(l/32) .. +3 of column 32j + l%32.
    epilogue([&](auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          i32x4 w;
#pragma unroll
          for (int q = 0; q < 4; ++q) w[q] = bits_of(acc[i][j][4 * g + q]);
          *(i32x4*)&stage[r32 * kPitch + 32 * i + 8 * g + 4 * hh + 4 * (i >> 1)] = w;
        }
    });
  }

  cycle_record(p.probe, t0, probe_slot(wave), wave);
}

// ---------------------------------------------------------------------------
// TN path, 128x128 tiles
// ---------------------------------------------------------------------------

// For 16-bit and int8 TN problems of up to 512 tiles of 128x128 (make_plan:
// one pass, or slices of K), where gemm_tn_fast's 256x256 tiles would leave
// CUs idle. 4 waves of 64x64 per 128x128 tile, each wave 4 x 4 tiles of
// 16x16 MFMAs accumulated in place in AGPRs (gemm_tn_fast's assembly MFMA,
// fragment chunk order and stage swizzle at half the rows). K streams
// through a ring of NS 128-byte LDS stages: with NS = 4 (128 KB, one
// workgroup per CU) three stages are in flight while one is read, so a load
// has three stages of MFMA time to land; with NS = 2 (64 KB) two workgroups
// share a CU and each SIMD's second wave hides the shorter cover. One
// barrier per stage both publishes the next stage and frees the one the DMA
// refills. Fragments are double-buffered one k-step ahead,
// read between the MFMAs. The DMA is issued as inline assembly: through the
// builtin, the compiler's wait-count pass cannot tell the stage reads from
// the DMA still landing in the other stages and waits for all of it before
// every barrier. C is stored from registers, 4 rows of one column per lane
// (8 or 16 bytes).
constexpr int kT128 = 128;

// AN: op(A) = A stored M-contiguous (transa = N, 16-bit inputs), read
// without a transposed copy: its stage holds 64 k-rows of the tile's 128 m
// ([k][m], 256 bytes a row, 16-byte chunks XOR-swizzled by 2 * ((k & 3) |
// ((k >> 2) & 4))), each A fragment is two transposing reads
// (ds_read_b64_tr_b16: a 16-lane group reads 4 k-rows x 16 m, each lane
// receiving the 4 k of its m), at the same k chunk as the B fragment of its
// lanes, so every product is unchanged; over the 32 lanes of a read cycle
// the swizzle puts the 8 rows' 16 chunks on distinct banks. BN: the same
// for op(B) = B^T stored N-contiguous (transb = T). int8: 128 k-rows of 128
// bytes per stage, chunks XOR-swizzled by an_swz8(k), each 16x16x64
// fragment two ds_read_b64_tr_b8 (8 k-rows x 16 m, each lane receiving the 8
// k of its m); over a read cycle's 32 lanes the 16 rows' chunks again fall
// on distinct banks.
template <class Op, MmaOut OUT, int NS, bool STREAM = true, bool AN = false, bool BN = false>
__global__ __launch_bounds__(256, NS == 2 ? 2 : 1) void gemm_tn128(KParams batch_p) {
  static_assert(NS == 2 || NS == 4, "stages in the ring: 4 (one workgroup per CU) or 2 (two)");
  static_assert((!AN && !BN) || Op::kElemBytes <= 2, "M/N-contiguous operands: 16-bit or int8 inputs");
  constexpr uint32_t kStage = kT128 * kChunks * 16;       // 16 KB per operand and stage
  const KParams p = batch_view(batch_p);
  // [A | B][stage][row * 8 + physical chunk], 16 bytes per entry.
  __shared__ __attribute__((aligned(1024))) i32x4 lds[2][NS][kT128 * kChunks];
  const uint64_t t0 = p.probe ? cycle_now() : 0;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int tm, tn;
  map_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, p.group, tm, tn);
  const int row0 = tm * kT128, col0 = tn * kT128;
  const int lda_b = (int)(p.lda * Op::kElemBytes);
  const int ldb_b = (int)(p.ldb * Op::kElemBytes);
  const int kbytes = p.k * Op::kElemBytes;
  const int ktiles = (kbytes + kFastKBytes - 1) / kFastKBytes;
  // Buffer descriptors as in gemm_tn_fast (record count ending at row m or
  // n, so rows past the matrix read zero; offset 2^31 reads zero for a
  // masked k chunk or a stage past K), as the four words the assembly takes.
  const int rows_a = min(kT128, p.m - row0);
  const int rows_b = min(kT128, p.n - col0);
  constexpr uint32_t kOff = 0x80000000u;
  constexpr int EB = Op::kElemBytes;
  constexpr int kRowsAN = kFastKBytes / EB;               // k-rows of an AN stage (64 or 128)
  constexpr int kRowChunks = kT128 * EB / 16;             // 16-byte chunks of a k-row (16 or 8)
  constexpr int kRowsDma = 64 / kRowChunks;               // k-rows per 1 KB DMA block (4 or 8)
  auto rsrc_words = [&](const uint8_t* base, int bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xffff);
    r[2] = __builtin_amdgcn_readfirstlane(bytes);
    r[3] = (int)kRsrcWord3;
    return r;
  };
  // AN: from the tile's first m; every k-row of A, to the end of the matrix
  // (m past the matrix within a row reads the next row's values, which only
  // reach rows of C that are never stored). BN likewise from the first n.
  const i32x4 rsa = AN ? rsrc_words(p.a + (int64_t)row0 * EB, (p.k - 1) * lda_b + (p.m - row0) * EB)
                       : rsrc_words(p.a + (int64_t)row0 * lda_b, (rows_a - 1) * lda_b + kbytes);
  const i32x4 rsb = BN ? rsrc_words(p.b + (int64_t)col0 * EB, (p.k - 1) * ldb_b + (p.n - col0) * EB)
                       : rsrc_words(p.b + (int64_t)col0 * ldb_b, (rows_b - 1) * ldb_b + kbytes);
  // DMA instruction d (0..7) of a stage: operand d / 4, the 1 KB block of
  // rows 8*(4*(d%4) + wave) .. +7, lane L landing in row +L/8 at physical
  // chunk L%8 and fetching logical chunk (L%8) ^ swz(row).
  const int lr = lane >> 3, pc = lane & 7;
  uint32_t base_a[4], base_b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = 4 * i + wave;
    const int row = 8 * blk + lr;
    const int c = pc ^ lr ^ (blk & 7);
    const int nrow = kRowsDma * blk + lane / kRowChunks;  // AN / BN: k-row of the stage
    base_a[i] = AN ? (uint32_t)(nrow * lda_b + 16 * ((lane % kRowChunks) ^ nswz<EB>(nrow)))
                   : (uint32_t)(row * lda_b + 16 * c);
    base_b[i] = BN ? (uint32_t)(nrow * ldb_b + 16 * ((lane % kRowChunks) ^ nswz<EB>(nrow)))
                   : (uint32_t)(row * ldb_b + 16 * c);
  }
  auto dma = [&](int kt, int st, int d) __attribute__((always_inline)) {
    const int i = d & 3;
    const int blk = 4 * i + wave;
    const int kb = kt * kFastKBytes;
    const int c = pc ^ lr ^ (blk & 7);
    const bool ok = kt < ktiles && kb + 16 * c < kbytes;
    // One wait state between the M0 write and the DMA that reads it (the
    // hazard pass does not look inside inline assembly).
    if ((d < 4 && AN) || (d >= 4 && BN)) {
      // 4 k-rows of 256 bytes (int8: 8 of 128): lane L -> k-row
      // kRowsDma*blk + L/kRowChunks, physical chunk L%kRowChunks
      const int krow = kt * kRowsAN + kRowsDma * blk + lane / kRowChunks;
      const uint32_t ld = (uint32_t)(d < 4 ? lda_b : ldb_b);
      const uint32_t v = krow < p.k ? (d < 4 ? base_a[i] : base_b[i]) + (uint32_t)(kt * kRowsAN) * ld : kOff;
      const uint32_t l = (uint32_t)(uintptr_t)(lds_ptr_t)&lds[d < 4 ? 0 : 1][st][blk * 64];
      if (d < 4)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                     :: "s"(l), "v"(v), "s"(rsa) : "memory");
      else
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                     :: "s"(l), "v"(v), "s"(rsb) : "memory");
    } else if (d < 4) {
      const uint32_t v = ok ? base_a[i] + (uint32_t)kb : kOff;
      const uint32_t l = (uint32_t)(uintptr_t)(lds_ptr_t)&lds[0][st][blk * 64];
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                   :: "s"(l), "v"(v), "s"(rsa) : "memory");
    } else {
      const uint32_t v = ok ? base_b[i] + (uint32_t)kb : kOff;
      const uint32_t l = (uint32_t)(uintptr_t)(lds_ptr_t)&lds[1][st][blk * 64];
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                   :: "s"(l), "v"(v), "s"(rsb) : "memory");
    }
  };

  using Acc = typename Op::Acc16;
  Acc acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0;
  const int wm = wave >> 1, wn = wave & 1, r16 = lane & 15;
  // Chunks of a 64-byte k-step to the four 16-lane groups in the order
  // 0, 2, 1, 3 (A and B alike), as in gemm_tn_fast: conflict-free reads.
  const int kq = ((lane >> 3) & 2) | ((lane >> 5) & 1);
  typedef __attribute__((address_space(3))) const i32x4* lds_frag_t;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)&lds[0][0][0];
  uint32_t ad_a[4][2], ad_b[4][2];                        // stage 0, [tile][k-step]
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kc = 4 * ks + kq;
      const int ar = wm * 64 + 16 * t + r16;
      const int br = wn * 64 + 16 * t + r16;
      ad_a[t][ks] = lds0 + 16u * (uint32_t)(ar * kChunks + (kc ^ swz(ar)));
      ad_b[t][ks] = lds0 + NS * kStage + 16u * (uint32_t)(br * kChunks + (kc ^ swz(br)));
    }
  // AN / BN: per tile and k-step, the two transposing reads' addresses
  // (k-rows 8c .. 8c+3 and 8c+4 .. 8c+7 of chunk c = 4*ks + kq, m (or n) =
  // 16t + 4*(j&3) for lane j of its 16-lane group; int8: k-rows 16c .. +7
  // and 16c+8 .. +15, m = 16t + 8*(j&1)).
  uint32_t ad_an[AN ? 4 : 1][2][2], ad_bn[BN ? 4 : 1][2][2];
  auto tr_addrs = [&](uint32_t (*ad)[2][2], int w, uint32_t base) __attribute__((always_inline)) {
    const int j = lane & 15;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if constexpr (EB == 2) {
            const int krow = 8 * (4 * ks + kq) + 4 * h + (j >> 2);
            const int m = w * 64 + 16 * t + 4 * (j & 3);
            ad[t][ks][h] = base + 256u * (uint32_t)krow + 16u * (uint32_t)((m >> 3) ^ an_swz(krow)) +
                           2u * (uint32_t)(m & 7);
          } else {
            const int krow = 16 * (4 * ks + kq) + 8 * h + (j >> 1);
            const int m = w * 64 + 16 * t + 8 * (j & 1);
            ad[t][ks][h] = base + 128u * (uint32_t)krow + 16u * (uint32_t)((m >> 4) ^ an_swz8(krow)) +
                           (uint32_t)(m & 15);
          }
        }
  };
  if constexpr (AN) tr_addrs(ad_an, wm, lds0);
  if constexpr (BN) tr_addrs(ad_bn, wn, lds0 + NS * kStage);
  typedef __attribute__((address_space(3))) s16x4* lds_s16x4_t;
  auto frag_tr = [&](const uint32_t (*ad)[2][2], int t, int rks, uint32_t off)
      __attribute__((always_inline)) -> i32x4 {
    u32x2 w0, w1;
    if constexpr (EB == 2) {
      w0 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t)(uintptr_t)(ad[t][rks][0] + off)));
      w1 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t)(uintptr_t)(ad[t][rks][1] + off)));
    } else {
      typedef __attribute__((address_space(3))) i32x2* lds_i32x2_t;
      w0 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t)(uintptr_t)(ad[t][rks][0] + off)));
      w1 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t)(uintptr_t)(ad[t][rks][1] + off)));
    }
    return i32x4{(int)w0.x, (int)w0.y, (int)w1.x, (int)w1.y};
  };
  i32x4 fa[2][4], fb[2][4];
  // One k-step: 16 MFMAs (A tile q/4 x B tile q%4). Behind the odd slots,
  // the next k-step's 8 fragments (stage offset `off`, k-step `rks`) into
  // the other register set; ahead of the even slots, DMA instruction q/2
  // of stage `dkt` into ring slot `dst` when `dma_on`.
  auto kstep = [&](auto bufc, uint32_t off, int rks, bool dma_on, int dkt, int dst)
      __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (dma_on && (q & 1) == 0) dma(dkt, dst, q >> 1);
      __builtin_amdgcn_sched_barrier(0);
      Op::mma16(fa[buf][q >> 2], fb[buf][q & 3], acc[q >> 2][q & 3]);
      __builtin_amdgcn_sched_barrier(0);
      if (q & 1) {
        const int f = q >> 1;
        if (f < 4 && AN) fa[buf ^ 1][f] = frag_tr(ad_an, f & (AN ? 3 : 0), rks, off);
        else if (f < 4) fa[buf ^ 1][f] = *(lds_frag_t)(uintptr_t)(ad_a[f][rks] + off);
        else if (BN) fb[buf ^ 1][f - 4] = frag_tr(ad_bn, (f - 4) & (BN ? 3 : 0), rks, off);
        else fb[buf ^ 1][f - 4] = *(lds_frag_t)(uintptr_t)(ad_b[f - 4][rks] + off);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Stages 0 .. NS-1 in flight, then stage 0 landed. Stage s lives in ring
  // slot s % NS; a stage past K is a zero fill, so every stage issues the
  // same 8 DMA instructions per wave and the waits below count uniformly.
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int d = 0; d < 8; ++d) dma(s, s, d);
  if constexpr (NS == 4) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    fa[0][t] = AN ? frag_tr(ad_an, t & (AN ? 3 : 0), 0, 0) : *(lds_frag_t)(uintptr_t)ad_a[t][0];
    fb[0][t] = BN ? frag_tr(ad_bn, t & (BN ? 3 : 0), 0, 0) : *(lds_frag_t)(uintptr_t)ad_b[t][0];
  }
  for (int kt = 0; kt < ktiles; ++kt) {
    const int st = kt & (NS - 1);
    // k-step 0 of stage kt; its k-step 1 fragments read alongside
    kstep(IntC<0>{}, (uint32_t)st * kStage, 1, false, 0, 0);
    // Stage kt+1 landed (with four stages, kt+2 and kt+3 may still be in
    // flight), and no wave reads stage kt any more: its slot takes stage
    // kt+NS.
    if constexpr (NS == 4) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    kstep(IntC<1>{}, (uint32_t)((kt + 1) & (NS - 1)) * kStage, 0, true, kt + NS, st);
  }
  // The MFMAs are assembly, so the compiler places the epilogue's reads of
  // their results without knowing what wrote them: 18 wait states first.
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" ::: "memory");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");    // no LDS write may outlive the workgroup

  // Lane l holds rows 16i + 4*(l/16) .. +3 of column 16j + l%16.
  using E = typename Op::Elem;
  using T = typename Epi<OUT>::T;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gj = col0 + wn * 64 + 16 * j + r16;
      const int i0 = row0 + wm * 64 + 16 * i + 4 * (lane >> 4);
      if (gj >= p.n || i0 >= p.m) continue;
      const E v[4] = {(E)acc[i][j][0], (E)acc[i][j][1], (E)acc[i][j][2], (E)acc[i][j][3]};
      if constexpr (Epi<OUT>::kRun == 4) {
        store_run<OUT, STREAM>(p, i0, gj, v, 4, true);
      } else if (i0 + 4 <= p.m) {
        // 16-bit C: the run's 8 bytes, each value as Epi<OUT>::put_run
        // (or put_run_scaled) rounds it.
        T* c = (T*)p.c + (int64_t)gj * p.ldc + i0;
        u32x2 o;
        if constexpr (OUT == MmaOut::DEQ_BF16) {
          const float s = p.scale[gj];
          o[0] = pack_bf16x2(__fmul_rn((float)v[0], s), __fmul_rn((float)v[1], s));
          o[1] = pack_bf16x2(__fmul_rn((float)v[2], s), __fmul_rn((float)v[3], s));
        } else if (p.beta == 0.0f) {
          o[0] = Epi<OUT>::pack(__fmul_rn(p.alpha, v[0]), __fmul_rn(p.alpha, v[1]));
          o[1] = Epi<OUT>::pack(__fmul_rn(p.alpha, v[2]), __fmul_rn(p.alpha, v[3]));
        } else {
          const u32x2 old = *(const u32x2*)c;
          o[0] = Epi<OUT>::pack(Epi<OUT>::apply(p, v[0], (uint16_t)(old[0] & 0xffff)),
                                Epi<OUT>::apply(p, v[1], (uint16_t)(old[0] >> 16)));
          o[1] = Epi<OUT>::pack(Epi<OUT>::apply(p, v[2], (uint16_t)(old[1] & 0xffff)),
                                Epi<OUT>::apply(p, v[3], (uint16_t)(old[1] >> 16)));
        }
        *(u32x2*)c = o;
      } else {
        store_run<OUT, STREAM>(p, i0, gj, v, 4, false);
      }
    }
  cycle_record(p.probe, t0, probe_slot(wave), wave);
}

// ---------------------------------------------------------------------------
// general path
// ---------------------------------------------------------------------------

constexpr int kGenTile = 64;
constexpr int kGenKBytes = 64;                 // two MFMA k-steps per stage
constexpr int kGenRowBytes = kGenKBytes + 16;  // padded row: conflict-free b128 reads

template <class Op, MmaOut OUT>
__global__ __launch_bounds__(256) void gemm_general(KParams batch_p) {
  const KParams p = batch_view(batch_p);
  constexpr int EB = Op::kElemBytes;
  using U = std::conditional_t<EB == 4, uint32_t, std::conditional_t<EB == 2, uint16_t, uint8_t>>;
  constexpr int KT = kGenKBytes / EB;  // elements of K per stage
  __shared__ __attribute__((aligned(16))) uint8_t sa[kGenTile * kGenRowBytes];
  __shared__ __attribute__((aligned(16))) uint8_t sb[kGenTile * kGenRowBytes];

  const uint64_t t0 = p.probe ? cycle_now() : 0;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tm = blockIdx.x % p.tiles_m;
  const int tn = blockIdx.x / p.tiles_m;
  const int row0 = tm * kGenTile;
  const int col0 = tn * kGenTile;

  using Acc = typename Op::Acc;
  Acc acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0;

  const int wm = wave >> 1, wn = wave & 1;
  const int ktiles = (p.k + KT - 1) / KT;
  constexpr int kPerThread = kGenTile * KT / 256;

  for (int kt = 0; kt < ktiles; ++kt) {
    const int k0 = kt * KT;
    // Stage op(A)[row0.., k0..] as [row][k] and op(B)[k0.., col0..] as [col][k].
    // The thread -> element map follows the operand's contiguous dimension so
    // that global reads coalesce.
#pragma unroll
    for (int q = 0; q < kPerThread; ++q) {
      const int e = tid + 256 * q;
      int r, kk;
      if (p.ta) { r = e / KT; kk = e % KT; } else { kk = e / kGenTile; r = e % kGenTile; }
      const int gi = row0 + r, gk = k0 + kk;
      uint8_t* dst = sa + r * kGenRowBytes + kk * EB;
      if (gi < p.m && gk < p.k) {
        const int64_t off = p.ta ? ((int64_t)gi * p.lda + gk) : ((int64_t)gk * p.lda + gi);
        *(U*)dst = ((const U*)p.a)[off];
      } else {
        *(U*)dst = 0;
      }
    }
#pragma unroll
    for (int q = 0; q < kPerThread; ++q) {
      const int e = tid + 256 * q;
      int c, kk;
      if (!p.tb) { c = e / KT; kk = e % KT; } else { kk = e / kGenTile; c = e % kGenTile; }
      const int gj = col0 + c, gk = k0 + kk;
      uint8_t* dst = sb + c * kGenRowBytes + kk * EB;
      if (gj < p.n && gk < p.k) {
        const int64_t off = p.tb ? ((int64_t)gk * p.ldb + gj) : ((int64_t)gj * p.ldb + gk);
        *(U*)dst = ((const U*)p.b)[off];
      } else {
        *(U*)dst = 0;
      }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kGenKBytes / 32; ++ks) {
      const int kb = ks * 32 + (lane >> 5) * 16;
      const i32x4 fa = *(const i32x4*)(sa + (wm * 32 + (lane & 31)) * kGenRowBytes + kb);
      const i32x4 fb = *(const i32x4*)(sb + (wn * 32 + (lane & 31)) * kGenRowBytes + kb);
      acc = Op::mma(fa, fb, acc);
    }
    __syncthreads();
  }

  store_acc_tile<Op, OUT>(p, acc, row0 + wm * 32, col0 + wn * 32, lane);
  cycle_record(p.probe, t0, probe_slot(wave), wave);
}

// ---------------------------------------------------------------------------
// operand transpose (for layouts the TN kernel cannot read directly)
// ---------------------------------------------------------------------------

// Y[c + r*ldy] = X[r + c*ldx] for r < R, c < C, elements of EB bytes, with
// X read only for c < Cin (columns Cin .. C-1 of Y are zeros: K padded to a
// multiple of 16 bytes); batch blockIdx.z at X + z*sx, Y + z*sy (elements).
// 64x64-element tiles through LDS: 16-byte loads along r, 16-byte stores
// along c. C is a multiple of 16/EB, so an output chunk is wholly inside or
// outside.
template <int EB>
__global__ __launch_bounds__(256) void transpose_k(const uint8_t* X, int64_t ldx, int64_t sx,
                                                   uint8_t* Y, int64_t ldy, int64_t sy, int R,
                                                   int C, int Cin, int vec_in) {
  constexpr int T = 64;
  constexpr int VE = 16 / EB;        // elements per 16-byte chunk
  constexpr int CPS = T / VE;        // chunks per 64-element segment
  constexpr int PITCH = T * EB + 16; // LDS bytes per c-row
  __shared__ __attribute__((aligned(16))) uint8_t tile[T][PITCH];  // [c][r]
  const int r0 = blockIdx.x * T, c0 = blockIdx.y * T;
  X += (int64_t)blockIdx.z * sx * EB;
  Y += (int64_t)blockIdx.z * sy * EB;
  for (int q = threadIdx.x; q < T * CPS; q += 256) {
    const int c = q / CPS, ch = q % CPS;
    const int gc = c0 + c, gr = r0 + ch * VE;
    uint8_t* dst = &tile[c][ch * 16];
    const uint8_t* src = X + ((int64_t)gc * ldx + gr) * EB;
    if (vec_in && gc < Cin && gr + VE <= R) {
      *(u32x4*)dst = *(const u32x4*)src;
    } else {
#pragma unroll
      for (int e = 0; e < VE; ++e)
#pragma unroll
        for (int b = 0; b < EB; ++b) dst[e * EB + b] = (gc < Cin && gr + e < R) ? src[e * EB + b] : 0;
    }
  }
  __syncthreads();
  for (int q = threadIdx.x; q < T * CPS; q += 256) {
    const int r = q / CPS, ch = q % CPS;
    const int gr = r0 + r, gc = c0 + ch * VE;
    if (gr >= R || gc >= C) continue;
    u32x4 w;
    if constexpr (EB == 4) {
#pragma unroll
      for (int h = 0; h < 4; ++h) w[h] = *(const uint32_t*)&tile[ch * VE + h][4 * r];
    } else if constexpr (EB == 2) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
        w[h] = (uint32_t)*(const uint16_t*)&tile[ch * VE + 2 * h][2 * r] |
               ((uint32_t)*(const uint16_t*)&tile[ch * VE + 2 * h + 1][2 * r] << 16);
    } else {
#pragma unroll
      for (int h = 0; h < 4; ++h)
        w[h] = (uint32_t)tile[ch * VE + 4 * h][r] | ((uint32_t)tile[ch * VE + 4 * h + 1][r] << 8) |
               ((uint32_t)tile[ch * VE + 4 * h + 2][r] << 16) |
               ((uint32_t)tile[ch * VE + 4 * h + 3][r] << 24);
    }
    *(u32x4*)(Y + ((int64_t)gr * ldy + gc) * EB) = w;
  }
}

template <int EB>
hipError_t launch_transpose(const void* x, int64_t ldx, int64_t sx, void* y, int64_t ldy,
                            int64_t sy, int R, int C, int Cin, int batch, hipStream_t s) {
  const int vec_in = ((uintptr_t)x % 16 == 0) && (ldx * EB) % 16 == 0 && (sx * EB) % 16 == 0;
  const dim3 grid((unsigned)((R + 63) / 64), (unsigned)((C + 63) / 64), (unsigned)batch);
  hipLaunchKernelGGL((transpose_k<EB>), grid, dim3(256), 0, s, (const uint8_t*)x, ldx, sx,
                     (uint8_t*)y, ldy, sy, R, C, Cin, vec_in);
  return hipGetLastError();
}

// Y[c + r*ldy] = X[c + r*ldx] for r < R, c < Cin, zeros for Cin <= c < C
// (C a multiple of 16/EB): an operand that is already K-contiguous but whose
// K, leading dimension or base the TN kernels cannot take, re-laid in rows of
// C elements (K padded to 16 bytes). One 16-byte output chunk per thread; a
// chunk wholly inside the row reads the aligned dwords that hold its 16
// bytes (four, or five when the source is not 4-byte aligned) and shifts
// them into place with v_alignbyte; every dword read holds at least one of
// the chunk's own bytes, so none can fall outside the source's mapped pages.
// The row's last, partial chunk is read element by element. Batch
// blockIdx.y at X + z*sx, Y + z*sy (elements).
template <int EB>
__global__ __launch_bounds__(256) void repitch_k(const uint8_t* X, int64_t ldx, int64_t sx,
                                                 uint8_t* Y, int64_t ldy, int64_t sy, int R,
                                                 int C, int Cin) {
  constexpr int VE = 16 / EB;
  const int cpr = C / VE;                                  // chunks per row
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= (int64_t)R * cpr) return;
  const int r = (int)(q / cpr), c0 = (int)(q % cpr) * VE;
  const uint8_t* src = X + ((int64_t)blockIdx.y * sx + (int64_t)r * ldx + c0) * EB;
  u32x4 o;
  if (c0 + VE <= Cin) {
    const uintptr_t a = (uintptr_t)src;
    const uint32_t sh = (uint32_t)(a & 3);
    const uint32_t* w = (const uint32_t*)(a - sh);
    uint32_t d[5];
#pragma unroll
    for (int i = 0; i < 4; ++i) d[i] = w[i];
    d[4] = sh ? w[4] : 0u;                   // the dword holding byte a+15 when unaligned
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
  } else {
    uint8_t w[16];
#pragma unroll
    for (int e = 0; e < VE; ++e)
#pragma unroll
      for (int b = 0; b < EB; ++b) w[e * EB + b] = c0 + e < Cin ? src[e * EB + b] : 0;
    o = *(const u32x4*)w;
  }
  *(u32x4*)(Y + ((int64_t)blockIdx.y * sy + (int64_t)r * ldy + c0) * EB) = o;
}

template <int EB>
hipError_t launch_repitch(const void* x, int64_t ldx, int64_t sx, void* y, int64_t ldy, int64_t sy,
                          int R, int C, int Cin, int batch, hipStream_t s) {
  const int64_t chunks = (int64_t)R * (C / (16 / EB));
  const dim3 grid((unsigned)((chunks + 255) / 256), (unsigned)batch);
  hipLaunchKernelGGL((repitch_k<EB>), grid, dim3(256), 0, s, (const uint8_t*)x, ldx, sx,
                     (uint8_t*)y, ldy, sy, R, C, Cin);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// split-K reduction
// ---------------------------------------------------------------------------

// C = epilogue(sum over s of W[s]), W[s] column-major with leading dimension
// ldw (a multiple of 8, so every run is 16-byte aligned) and slice stride
// sstride (elements). One thread per run of kRun rows of one column; slices
// are summed in order s = 0, 1, ..., so the result does not depend on timing.
// The loads of kBatch slices are issued before their adds (the sum is
// latency-bound otherwise: few threads, one dependent HBM read per slice).
// int32 partials add with two's complement wrap (unsigned arithmetic).
template <MmaOut OUT, class E>
__global__ __launch_bounds__(256) void reduce_splits(KParams p, const E* ws, int64_t ldw,
                                                     int64_t sstride, int nsplit) {
  constexpr int R = Epi<OUT>::kRun;
  constexpr int H = R / 4;          // 16-byte loads per slice
  constexpr int kBatch = 4;
  const int runs = (p.m + R - 1) / R;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)runs * p.n) return;
  const int j = (int)(idx / runs);
  const int i0 = (int)(idx % runs) * R;
  const E* src = ws + (int64_t)j * ldw + i0;
  E v[R];
#pragma unroll
  for (int q = 0; q < R; ++q) v[q] = 0;
  auto add = [&](const i32x4 (&w)[H]) {
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (std::is_integral<E>::value)
          v[4 * h + q] = (E)((uint32_t)v[4 * h + q] + (uint32_t)w[h][q]);
        else
          v[4 * h + q] += from_bits<E>(w[h][q]);
      }
  };
  int z = 0;
  for (; z + kBatch <= nsplit; z += kBatch) {
    i32x4 w[kBatch][H];
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int h = 0; h < H; ++h) w[b][h] = *(const i32x4*)(src + (z + b) * sstride + 4 * h);
#pragma unroll
    for (int b = 0; b < kBatch; ++b) add(w[b]);
  }
  for (; z < nsplit; ++z) {
    i32x4 w[H];
#pragma unroll
    for (int h = 0; h < H; ++h) w[h] = *(const i32x4*)(src + z * sstride + 4 * h);
    add(w);
  }
  // Runs of C are 16-byte aligned unless C is staged (ldc or base off 16 bytes).
  using T = typename Epi<OUT>::T;
  store_run<OUT>(p, i0, j, v, R, ((uintptr_t)((T*)p.c + (int64_t)j * p.ldc + i0) & 15) == 0);
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------

constexpr int64_t kTransposeMinWork = 1ll << 25;  // m*n*k below this: general path

template <MmaOut OUT>
constexpr int out_bytes() { return (OUT == MmaOut::F32 || OUT == MmaOut::I32) ? 4 : 2; }

// The TN kernel's requirements: K-contiguous operands whose rows start on
// 16-byte boundaries (so every staged chunk is one aligned 16-byte load),
// 32-bit buffer offsets within a 256-row panel, and a C whose columns start
// on 16-byte boundaries (ldc * sizeof(C) % 16 == 0, aligned C), so that a run of 4 (32-bit)
// or 8 (16-bit) rows of one column is one vector store.
template <class Op, MmaOut OUT>
bool tn_ready(const GemmDesc& d) {
  constexpr int EB = Op::kElemBytes;
  constexpr int OB = out_bytes<OUT>();
  return d.ta && !d.tb && d.k > 0 && ((int64_t)d.k * EB) % 16 == 0 &&
         (d.lda * EB) % 16 == 0 && (d.ldb * EB) % 16 == 0 &&
         ((uintptr_t)d.a % 16) == 0 && ((uintptr_t)d.b % 16) == 0 &&
         (d.ldc * OB) % 16 == 0 && ((uintptr_t)d.c % 16) == 0 &&
         (d.stride_a * EB) % 16 == 0 && (d.stride_b * EB) % 16 == 0 &&
         (d.stride_c * OB) % 16 == 0 &&
         (int64_t)kFastTile * d.lda * EB < (1ll << 31) &&
         (int64_t)kFastTile * d.ldb * EB < (1ll << 31);
}

// Other layouts run the TN kernel behind K-contiguous copies of the operands
// that are not: op(A) = A (transa N) is copied as A^T, op(B) = B^T (transb T)
// as B. Worth it once the GEMM dwarfs the copy (one more read and write of
// that operand). A TN problem too small to fill the GPU with 256x256 tiles
// (fewer than kSplitTiles) and long in K is split along K: slice z computes
// raw partials of its K range into the workspace (grid.y = slice) and
// reduce_splits applies the epilogue to their sum. Workspace layout: copy of
// A, copy of B, partials, each 256-byte aligned.
constexpr int kSplitTiles = 256;
constexpr int kTn128MaxTiles = 256;   // gemm_tn128's four-stage ring up to this many 128x128 tiles, two-stage up to twice it
constexpr int kMaxSplit = 16;
constexpr int64_t kFixNs = 8000, kStageNs = 1030, kReduceNs = 6000, kPartialBytesPerNs = 10000;
// An fp32 stage (32 elements of K) is 8x the MFMA work of a 16-bit one; measured
// 905 us for 128 stages per workgroup at 4096^3 (the chip holds ~2.4 GHz there).
constexpr int64_t kStageNsF32 = 7070;

struct Plan {
  bool copy_a = false, copy_b = false;
  int kp = 0;                     // the copies' K (row length): K, or K padded to 16 bytes
  bool c_staged = false;          // C reached through raw partials and reduce_splits
  int batch_a = 0, batch_b = 0;   // copies made (1 when the stride broadcasts)
  size_t a_bytes = 0, b_bytes = 0;
  int split = 1;                  // K slices
  int kslice = 0, k_last = 0;     // elements
  int64_t ldw = 0;                // partials' leading dimension
  size_t w_bytes = 0;
  bool tn = false;                // the TN kernel runs (directly or on copies)
  int64_t split_ns = 0;           // the split's modelled time (fp32 problems of 256+ tiles)
  bool tn128 = false;             // the TN problem runs on 128x128 tiles (gemm_tn128)
  int tn128_stages = 4;           // its LDS ring: 4 stages (one workgroup per CU) or 2 (two)
  bool a_direct = false;          // gemm_tn128 reads a 16-bit A (transa N) where it lies
  bool b_direct = false;          // ... and a 16-bit B (transb T)
  GemmDesc e;                     // the TN problem (over the copies; ws unset)
  size_t bytes() const { return a_bytes + b_bytes + w_bytes; }
};

inline size_t round256(size_t v) { return (v + 255) & ~(size_t)255; }

inline bool split128_enabled() { return true; }

template <class Op, MmaOut OUT>
Plan make_plan_core(const GemmDesc& d) {
  constexpr int EB = Op::kElemBytes;
  Plan t;
  t.e = d;
  t.e.ws = nullptr;
  t.e.ws_bytes = 0;
  if (tn_ready<Op, OUT>(d)) {
    t.tn = true;
  } else if (d.k > 0 && ((int64_t)d.k * EB) % 16 == 0 &&
             (int64_t)d.m * d.n * d.k >= kTransposeMinWork) {
    Plan c = t;
    c.copy_a = !d.ta;
    c.copy_b = d.tb;
    if (c.copy_a) {
      c.batch_a = d.stride_a == 0 ? 1 : d.batch;
      c.a_bytes = round256((size_t)c.batch_a * d.m * d.k * EB);
      c.e.ta = true;
      c.e.lda = d.k;
      c.e.stride_a = d.stride_a == 0 ? 0 : (int64_t)d.m * d.k;
    }
    if (c.copy_b) {
      c.batch_b = d.stride_b == 0 ? 1 : d.batch;
      c.b_bytes = round256((size_t)c.batch_b * d.n * d.k * EB);
      c.e.tb = false;
      c.e.ldb = d.k;
      c.e.stride_b = d.stride_b == 0 ? 0 : (int64_t)d.n * d.k;
    }
    // The copies are 256-byte aligned, so only the kept operand and C decide.
    GemmDesc q = c.e;
    if (c.copy_a) q.a = (const void*)(uintptr_t)256;
    if (c.copy_b) q.b = (const void*)(uintptr_t)256;
    if (tn_ready<Op, OUT>(q)) {
      c.tn = true;
      c.kp = d.k;
      t = c;
    }
  }
  // (16-bit and int8 inputs; fp32 keeps sgemm_mfma, whose guarded staging
  // takes any K at its usual rate.)
  if (!std::is_same<Op, OpF32>::value && !t.tn && d.pad_copies && d.k > 0 &&
      (int64_t)d.m * d.n * d.k >= kTransposeMinWork) {
    // K not a multiple of 16 bytes, or the K-contiguous operand unaligned:
    // both operands copied K-contiguous into rows of K rounded up to 16
    // bytes, the pad zero in both (so every padded product is an exact
    // zero), then the TN kernels on K' (4096^2 x 4095 bf16: 47 TFLOP/s on
    // the 64x64 general kernel). An operand stored K-contiguous is re-laid
    // row by row (repitch_k), the other transposed (transpose_k).
    constexpr int VE = 16 / EB;
    const int kp = (d.k + VE - 1) / VE * VE;
    Plan c = t;
    c.copy_a = c.copy_b = true;
    c.kp = kp;
    c.batch_a = d.stride_a == 0 ? 1 : d.batch;
    c.a_bytes = round256((size_t)c.batch_a * d.m * kp * EB);
    c.batch_b = d.stride_b == 0 ? 1 : d.batch;
    c.b_bytes = round256((size_t)c.batch_b * d.n * kp * EB);
    c.e.ta = true;
    c.e.tb = false;
    c.e.k = kp;
    c.e.lda = kp;
    c.e.ldb = kp;
    c.e.stride_a = d.stride_a == 0 ? 0 : (int64_t)d.m * kp;
    c.e.stride_b = d.stride_b == 0 ? 0 : (int64_t)d.n * kp;
    GemmDesc q = c.e;
    q.a = (const void*)(uintptr_t)256;
    q.b = (const void*)(uintptr_t)256;
    if (tn_ready<Op, OUT>(q)) {
      c.tn = true;
      t = c;
    }
  }
  if (!t.tn || d.probe) return t;
  // Split K where a cost model (times in ns, fitted to kernel traces of
  // 256x256 tiles at up to 256 workgroups) predicts at least 10 % less time.
  // One pass: kFixNs (launch, prologue, epilogue) + kStageNs per 128-byte K
  // stage. With s slices of at least 8 stages each (shorter slices measured
  // slower than the model says: the K-loop's fill and drain dominate) and
  // tiles * s <= 256 (one workgroup per CU), every workgroup runs
  // ceil(stages/s) stages, plus the reduction: kReduceNs and the fp32
  // partials written by the slices and read back, 8 * s * m * n bytes at
  // kPartialBytesPerNs (mostly served from the last-level cache, hence above
  // the HBM rate).
  // fp32 stages are long enough (8x the MFMA work) that slices may also run
  // in several waves of 256 workgroups: there the model charges each wave
  // its fill and drain (kFixNs) and ceil(stages/s) stages (3072^3: 144 tiles
  // in 7 slices, 4 waves; 99 -> 114 TFLOP/s against the 128x128 kernel).
  // fp32 problems of 256 tiles or more split only into slices of at least
  // 32 stages (shorter ones measured slower than the model), and the caller
  // takes such a split only where it beats the 128x128 kernel's best rate
  // (fp32_mma_wanted).
  constexpr bool kF32 = std::is_same<Op, OpF32>::value;
  const int64_t tiles = (int64_t)((d.m + kFastTile - 1) / kFastTile) * ((d.n + kFastTile - 1) / kFastTile);
  const int64_t stages = ((int64_t)d.k * EB + kFastKBytes - 1) / kFastKBytes;
  // 16-bit and int8 problems of at most 512 tiles of 128x128 run on them
  // unless K is long against the tile count: up to 32 stages always, beyond
  // that while 25 * stages <= 16 * tiles; the rest keep the 256x256 kernel,
  // split or not. Up to 256 tiles (one pass over the CUs) the kernel's
  // four-stage ring, one workgroup per CU; up to 512 its two-stage ring, two
  // workgroups per CU (2304^2 x 2048 669 against 530 on the 256x256 kernel,
  // 3072 x 2048 x 2048 736 / 625, 4096 x 2048 x 2048 886 / 798, 2048 x 4096
  // x 4096 1044 / 949; 2048^3 631 against 695 with four stages; past 512
  // tiles the 256x256 kernel: 3072^2 x 1024 718 against 588). Measured (bf16
  // TFLOP/s, 128x128 kernel against the alternative, same runs): 1024^3 170
  // / 89, 2048^3 706 / 462, 768^3 85 / 45, 1024^2 x 2048 214 / 162;
  // 1536^2 x 4096 (144 tiles, 64 stages) 540 / 464, 2048^2 x 4096 839 /
  // 674, 1280^2 x 4096 (100, 64) 384 / 353, 768 x 2048 x 4096 (96, 64) 372
  // / 384, 1024^2 x 3072 (64, 48) 237 / 240, 2048 x 1024 x 8192 (128, 128)
  // 544 / 676, 2048^2 x 8192 (256, 128) 967 / 963; past 256 tiles the
  // four-stage ring ties or loses to the 256x256 kernel (2304^2 x 2048 530 /
  // 527, 2048 x 4096 x 1024 616 / 640, 4096^2 x 1024 671 / 1057).
  // Batches of small problems (at most 16 tiles of 128x128 each) count their
  // workgroups, batch x tiles: bf16 TFLOP/s against the 256x256 kernel,
  // same runs, 16 x 256^2 x 64 23 / 14.5, 64 x 256^2 x 128 147 / 101, 32 x
  // 512^2 x 128 210 / 193 (torch bmm 7.4, 60, 115); batches of larger ones
  // keep the 256x256 kernel (8 x 1024^3 586 against 625, 12 x 768^3 406
  // against 454 on 128x128 tiles).
  const int64_t per128 = (int64_t)((d.m + kT128 - 1) / kT128) * ((d.n + kT128 - 1) / kT128);
  const int64_t tiles128 = per128 * d.batch;
  if (!kF32 && (d.batch == 1 || per128 <= 16) && tiles128 <= 2 * kTn128MaxTiles &&
      (stages <= 32 || 25 * stages <= 16 * tiles128)) {
    t.tn128 = true;
    t.tn128_stages = tiles128 <= kTn128MaxTiles ? 4 : 2;
    return t;
  }
  if (d.batch != 1) return t;                       // split K: one problem only
  // Long K on at most 128 tiles of 128x128: slices of at least 16 stages on
  // them, at most 256 workgroups in all, partials summed by reduce_splits.
  if (!kF32 && 2 * tiles128 <= kTn128MaxTiles && stages >= 32 && split128_enabled()) {
    const int64_t sl = std::min<int64_t>({kTn128MaxTiles / tiles128, stages / 16, (int64_t)kMaxSplit});
    const int64_t per = (stages + sl - 1) / sl;
    const int64_t slices = (stages + per - 1) / per;
    const int kslice = (int)per * (kFastKBytes / EB);
    t.tn128 = true;
    t.tn128_stages = 4;
    t.split = (int)slices;
    t.kslice = kslice;
    t.k_last = t.e.k - (t.split - 1) * kslice;
    t.ldw = ((int64_t)d.m + 7) / 8 * 8;
    t.w_bytes = round256((size_t)t.split * t.ldw * d.n * 4);
    return t;
  }
  if ((!kF32 && tiles >= kSplitTiles) || stages < 16) return t;
  const int64_t min_per = tiles >= kSplitTiles ? 32 : 8;
  const int64_t mn = ((int64_t)d.m + 7) / 8 * 8 * d.n;
  constexpr int64_t kStage = kF32 ? kStageNsF32 : kStageNs;
  auto cost = [&](int64_t sl, int64_t per) {
    const int64_t waves = kF32 ? (tiles * sl + 255) / 256 : 1;
    return (kFixNs + kStage * per) * waves +
           (sl > 1 ? kReduceNs + 8 * sl * mn / kPartialBytesPerNs : 0);
  };
  const int64_t one = cost(1, stages);
  int split = 1, per_best = (int)stages;
  int64_t best = one;
  for (int sl = 2; sl <= kMaxSplit && (kF32 || tiles * sl <= 256); ++sl) {
    const int64_t per = (stages + sl - 1) / sl;
    if (per < min_per) break;
    const int64_t slices = (stages + per - 1) / per;   // after rounding the slice up
    const int64_t c = cost(slices, per);
    if (c < best) {
      best = c;
      split = (int)slices;
      per_best = (int)per;
    }
  }
  if (split < 2 || best * 100 > one * 90) return t;
  const int kslice = per_best * (kFastKBytes / EB);
  t.split = split;
  t.split_ns = best;
  t.kslice = kslice;
  t.k_last = t.e.k - (split - 1) * kslice;
  t.ldw = ((int64_t)d.m + 7) / 8 * 8;
  t.w_bytes = round256((size_t)split * t.ldw * d.n * 4);
  return t;
}

// C whose leading dimension, base or batch stride is not on 16 bytes, which
// the TN kernels' stores need (bf16 C with m = 4095, or ldc = 500): 16-bit
// and int8 problems of one batch above the copy threshold keep the TN plan
// they would have with C aligned, their K loop writing raw partials (one
// slice, or the plan's split) to the workspace, and reduce_splits applies
// alpha, beta and the conversion into C, run by run.
template <MmaOut OUT>
bool c_ready(const GemmDesc& d) {
  constexpr int OB = out_bytes<OUT>();
  return (d.ldc * OB) % 16 == 0 && ((uintptr_t)d.c % 16) == 0 && (d.stride_c * OB) % 16 == 0;
}

// A 16-bit op(A) = A (transa N, M-contiguous) or op(B) = B^T (transb T,
// N-contiguous) on gemm_tn128 (one pass, its K slices, or a staged C) is
// read where it lies, through
// transposing LDS reads, instead of through a transposed copy (bf16 N,N
// 2048^3: 540 TFLOP/s behind the copy, 643-681 without). The 256x256
// kernel keeps the copies: read in place there (the same layout at 512-byte
// k-rows), bf16 N,N 8192^3 ran at 730 TFLOP/s against 1334 behind the copy,
// and at 4096^3 its waves waited 14x as long (SQ_WAIT_ANY) with no more LDS
// bank conflicts: every workgroup reads the same 64 k-rows of A per stage,
// one 512 KB (4096^2) or 1 MB (8192^2) window of HBM at a time, where the
// K-contiguous copy spreads a stage over the whole matrix, and its
// two-stage ring has one stage of cover against the 128x128 kernel's three.
// 16-byte chunks of m (n): m (n) a multiple of 8, so that no chunk straddles
// the end of the matrix (whose buffer record ends at the last element) and
// every chunk holding valid values is read whole; DMA offsets within the
// 2^31 bytes a buffer offset reaches below the zero-fill offset (the last
// k-row, plus a 128-row stage of slack).
inline bool direct_ok(int eb, int rows, const void* x, int64_t ld, int64_t stride, int k) {
  return (rows * eb) % 16 == 0 && (uintptr_t)x % 16 == 0 && (ld * eb) % 16 == 0 && (stride * eb) % 16 == 0 &&
         ((int64_t)k + kT128) * ld * eb + 4096 < (1ll << 31);
}

template <class Op>
Plan direct_operands(const GemmDesc& d, Plan t) {
  constexpr int EB = Op::kElemBytes;
  if (EB > 2 || !t.tn || !t.tn128 || t.kp != d.k) return t;
  if (t.copy_a && !d.ta && direct_ok(EB, d.m, d.a, d.lda, d.stride_a, d.k)) {
    t.copy_a = false;
    t.a_direct = true;
    t.batch_a = 0;
    t.a_bytes = 0;
    t.e.a = d.a;
    t.e.ta = false;
    t.e.lda = d.lda;
    t.e.stride_a = d.stride_a;
  }
  if (t.copy_b && d.tb && direct_ok(EB, d.n, d.b, d.ldb, d.stride_b, d.k)) {
    t.copy_b = false;
    t.b_direct = true;
    t.batch_b = 0;
    t.b_bytes = 0;
    t.e.b = d.b;
    t.e.tb = true;
    t.e.ldb = d.ldb;
    t.e.stride_b = d.stride_b;
  }
  return t;
}

template <class Op, MmaOut OUT>
Plan make_plan(const GemmDesc& d) {
  Plan t = make_plan_core<Op, OUT>(d);
  if (t.tn) return direct_operands<Op>(d, t);
  if (std::is_same<Op, OpF32>::value || d.batch != 1 || d.probe || !d.pad_copies ||
      d.k <= 0 || (int64_t)d.m * d.n * d.k < kTransposeMinWork || c_ready<OUT>(d))
    return t;
  GemmDesc q = d;
  q.c = (void*)(uintptr_t)256;
  q.ldc = ((int64_t)d.m + 7) / 8 * 8;
  q.stride_c = 0;
  Plan c = make_plan_core<Op, OUT>(q);
  if (!c.tn) return t;
  c.e.c = d.c;
  c.e.ldc = d.ldc;
  c.e.stride_c = d.stride_c;
  c.c_staged = true;
  if (c.split <= 1) {
    c.split = 1;
    c.kslice = c.e.k;
    c.k_last = c.e.k;
    c.ldw = ((int64_t)d.m + 7) / 8 * 8;
    c.w_bytes = round256((size_t)c.ldw * d.n * 4);
  }
  return direct_operands<Op>(d, c);
}

// GRXBLAS_LOG set (and not "0"): one line on stderr per GemmEx-family call
// naming the path it took. Read on every call, so it can be switched at run time.
inline bool log_plans() {
  const char* v = std::getenv("GRXBLAS_LOG");
  return v && *v && !(v[0] == '0' && v[1] == 0);
}

// GRXBLAS_TILE_GROUP=n (1..64): tile-rows per group of the XCD-aware tile
// order (map_tile); default 8. A tuning variable, read on every call.
inline int tile_group() {
  const char* v = std::getenv("GRXBLAS_TILE_GROUP");
  if (!v || !*v) return 8;
  const int g = std::atoi(v);
  return (g >= 1 && g <= 64) ? g : 8;
}

template <MmaOut OUT>
constexpr const char* out_name() {
  return OUT == MmaOut::F32 ? "f32" : OUT == MmaOut::I32 ? "i32" : OUT == MmaOut::F16 ? "f16"
       : OUT == MmaOut::BF16 ? "bf16" : "bf16(dequant)";
}

template <class Op, MmaOut OUT>
hipError_t run(const GemmDesc& d, hipStream_t s) {
  constexpr int EB = Op::kElemBytes;
  // The raw accumulator type of this input type, for split-K partials.
  constexpr MmaOut RAW = std::is_same<Op, OpI8>::value ? MmaOut::I32 : MmaOut::F32;
  using E = typename Op::Elem;
  Plan t = make_plan<Op, OUT>(d);
  if (t.bytes() > 0 && !(d.ws && d.ws_bytes >= t.bytes())) {
    // No workspace for copies or partials: the kernel that fits d as it is.
    t = Plan{};
    t.e = d;
    t.tn = tn_ready<Op, OUT>(d);
  }
  uint8_t* ws = (uint8_t*)d.ws;
  if (t.copy_a) {
    // op(A) as rows of kp: A (m x k, m contiguous) transposed, or A^T (rows
    // of k) re-laid; columns k .. kp-1 zero
    const hipError_t e =
        d.ta ? launch_repitch<EB>(d.a, d.lda, d.stride_a, ws, t.kp, (int64_t)d.m * t.kp, d.m, t.kp,
                                  d.k, t.batch_a, s)
             : launch_transpose<EB>(d.a, d.lda, d.stride_a, ws, t.kp, (int64_t)d.m * t.kp, d.m,
                                    t.kp, d.k, t.batch_a, s);
    if (e != hipSuccess) return e;
    t.e.a = ws;
  }
  if (t.copy_b) {
    // op(B) as rows of kp per column j: B (k x n, k contiguous) re-laid, or
    // B^T (n contiguous) transposed
    const hipError_t e =
        !d.tb ? launch_repitch<EB>(d.b, d.ldb, d.stride_b, ws + t.a_bytes, t.kp, (int64_t)d.n * t.kp,
                                   d.n, t.kp, d.k, t.batch_b, s)
              : launch_transpose<EB>(d.b, d.ldb, d.stride_b, ws + t.a_bytes, t.kp,
                                     (int64_t)d.n * t.kp, d.n, t.kp, d.k, t.batch_b, s);
    if (e != hipSuccess) return e;
    t.e.b = ws + t.a_bytes;
  }
  const GemmDesc* g = &t.e;
  if (log_plans()) {
    std::fprintf(stderr,
                 "grxblas: gemm %s->%s ta=%d tb=%d m=%d n=%d k=%d batch=%d kernel=%s copy_a=%d "
                 "copy_b=%d split=%d ring=%d staged=%d direct_a=%d direct_b=%d\n",
                 Op::kName, out_name<OUT>(), (int)d.ta, (int)d.tb, d.m, d.n, d.k, d.batch,
                 t.tn ? (t.tn128 ? "tn128" : "tn256") : "general64", (int)t.copy_a, (int)t.copy_b, t.split,
                 t.tn && t.tn128 ? t.tn128_stages : 0, (int)(t.tn && t.c_staged),
                 (int)(t.tn && t.a_direct), (int)(t.tn && t.b_direct));
  }

  KParams p{};
  p.a = (const uint8_t*)g->a;
  p.b = (const uint8_t*)g->b;
  p.c = g->c;
  p.lda = g->lda; p.ldb = g->ldb; p.ldc = g->ldc;
  p.m = g->m; p.n = g->n; p.k = g->k;
  p.ta = g->ta; p.tb = g->tb;
  p.alpha = g->alpha; p.beta = g->beta;
  p.ialpha = g->ialpha; p.ibeta = g->ibeta;
  p.scale = g->scale;
  p.probe = g->probe;
  p.group = tile_group();
  p.sa = g->stride_a * EB;
  p.sb = g->stride_b * EB;
  p.sc = g->stride_c * out_bytes<OUT>();

  if (t.tn && (t.split > 1 || t.c_staged)) {
    // Slices (or one, for a staged C): raw partials into the workspace, then
    // the epilogue over their sum.
    KParams q = p;
    E* w = (E*)(ws + t.a_bytes + t.b_bytes);
    q.c = w;
    q.ldc = t.ldw;
    q.k = t.kslice;
    q.k_last = t.k_last;
    // slice z starts kslice elements down K: along a row of the TN layout,
    // kslice rows down an operand read in place
    q.sa = (int64_t)t.kslice * EB * (t.a_direct ? g->lda : 1);
    q.sb = (int64_t)t.kslice * EB * (t.b_direct ? g->ldb : 1);
    q.sc = t.ldw * g->n * 4;
    q.alpha = 1.0f; q.beta = 0.0f; q.ialpha = 1; q.ibeta = 0;
    q.scale = nullptr;
    q.probe = nullptr;
    if constexpr (Op::kM16) {
      if (t.tn128) {                  // slices on 128x128 tiles
        q.tiles_m = (g->m + kT128 - 1) / kT128;
        q.tiles_n = (g->n + kT128 - 1) / kT128;
        const dim3 grid(q.tiles_m * q.tiles_n, t.split);
        const int v = (t.tn128_stages == 2 ? 4 : 0) + (t.a_direct ? 1 : 0) + (t.b_direct ? 2 : 0);
        if constexpr (Op::kElemBytes <= 2) {      // operands read in place: 16-bit and int8
          switch (v) {
            case 1: hipLaunchKernelGGL((gemm_tn128<Op, RAW, 4, false, true, false>), grid, dim3(256), 0, s, q); break;
            case 2: hipLaunchKernelGGL((gemm_tn128<Op, RAW, 4, false, false, true>), grid, dim3(256), 0, s, q); break;
            case 3: hipLaunchKernelGGL((gemm_tn128<Op, RAW, 4, false, true, true>), grid, dim3(256), 0, s, q); break;
            case 5: hipLaunchKernelGGL((gemm_tn128<Op, RAW, 2, false, true, false>), grid, dim3(256), 0, s, q); break;
            case 6: hipLaunchKernelGGL((gemm_tn128<Op, RAW, 2, false, false, true>), grid, dim3(256), 0, s, q); break;
            case 7: hipLaunchKernelGGL((gemm_tn128<Op, RAW, 2, false, true, true>), grid, dim3(256), 0, s, q); break;
            default: break;
          }
        }
        if (v == 4)
          hipLaunchKernelGGL((gemm_tn128<Op, RAW, 2, false>), grid, dim3(256), 0, s, q);
        else if (v == 0)
          hipLaunchKernelGGL((gemm_tn128<Op, RAW, 4, false>), grid, dim3(256), 0, s, q);
      }
    }
    if (!t.tn128) {
      q.tiles_m = (g->m + kFastTile - 1) / kFastTile;
      q.tiles_n = (g->n + kFastTile - 1) / kFastTile;
      hipLaunchKernelGGL((gemm_tn_fast<Op, RAW, false>), dim3(q.tiles_m * q.tiles_n, t.split), dim3(256), 0,
                         s, q);
    }
    constexpr int R = Epi<OUT>::kRun;
    const int64_t items = (int64_t)((g->m + R - 1) / R) * g->n;
    hipLaunchKernelGGL((reduce_splits<OUT, E>), dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s,
                       p, (const E*)w, t.ldw, t.ldw * g->n, t.split);
  } else if (t.tn && t.tn128) {
    p.tiles_m = (g->m + kT128 - 1) / kT128;
    p.tiles_n = (g->n + kT128 - 1) / kT128;
    if constexpr (Op::kM16)   // the plan takes this path for 16-bit and int8 inputs only
    {
      if constexpr (Op::kElemBytes <= 2) {
        if (t.a_direct || t.b_direct) {
          const dim3 grid(p.tiles_m * p.tiles_n, g->batch);
          const int v = (t.tn128_stages == 2 ? 4 : 0) + (t.a_direct ? 1 : 0) + (t.b_direct ? 2 : 0);
          switch (v) {
            case 1: hipLaunchKernelGGL((gemm_tn128<Op, OUT, 4, true, true, false>), grid, dim3(256), 0, s, p); break;
            case 2: hipLaunchKernelGGL((gemm_tn128<Op, OUT, 4, true, false, true>), grid, dim3(256), 0, s, p); break;
            case 3: hipLaunchKernelGGL((gemm_tn128<Op, OUT, 4, true, true, true>), grid, dim3(256), 0, s, p); break;
            case 5: hipLaunchKernelGGL((gemm_tn128<Op, OUT, 2, true, true, false>), grid, dim3(256), 0, s, p); break;
            case 6: hipLaunchKernelGGL((gemm_tn128<Op, OUT, 2, true, false, true>), grid, dim3(256), 0, s, p); break;
            default: hipLaunchKernelGGL((gemm_tn128<Op, OUT, 2, true, true, true>), grid, dim3(256), 0, s, p); break;
          }
          return hipGetLastError();
        }
      }
      if (t.tn128_stages == 2)
        hipLaunchKernelGGL((gemm_tn128<Op, OUT, 2>), dim3(p.tiles_m * p.tiles_n, g->batch), dim3(256), 0, s, p);
      else
        hipLaunchKernelGGL((gemm_tn128<Op, OUT, 4>), dim3(p.tiles_m * p.tiles_n, g->batch), dim3(256), 0, s, p);
    }
    else
      return hipErrorInvalidValue;
  } else if (t.tn) {
    p.tiles_m = (g->m + kFastTile - 1) / kFastTile;
    p.tiles_n = (g->n + kFastTile - 1) / kFastTile;
    const int blocks = p.tiles_m * p.tiles_n;
    hipLaunchKernelGGL((gemm_tn_fast<Op, OUT>), dim3(blocks, g->batch), dim3(256), 0, s, p);
  } else {
    p.tiles_m = (g->m + kGenTile - 1) / kGenTile;
    p.tiles_n = (g->n + kGenTile - 1) / kGenTile;
    const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemm_general<Op, OUT>), dim3((unsigned)blocks, g->batch), dim3(256), 0, s,
                       p);
  }
  return hipGetLastError();
}

template <class Op, MmaOut OUT>
size_t workspace(const GemmDesc& d) {
  return make_plan<Op, OUT>(d).bytes();
}

}  // namespace

int64_t gemm_probe_slots(int m, int n) {
  if (m <= 0 || n <= 0) return 0;
  return ((int64_t)(m + kGenTile - 1) / kGenTile) * ((n + kGenTile - 1) / kGenTile) * 4;
}

hipError_t launch_mma_gemm(MmaIn in, MmaOut out, const GemmDesc& d, hipStream_t s) {
  switch (in) {
    case MmaIn::BF16:
      if (out == MmaOut::F32) return run<OpBF16, MmaOut::F32>(d, s);
      if (out == MmaOut::BF16) return run<OpBF16, MmaOut::BF16>(d, s);
      break;
    case MmaIn::F16:
      if (out == MmaOut::F32) return run<OpF16, MmaOut::F32>(d, s);
      if (out == MmaOut::F16) return run<OpF16, MmaOut::F16>(d, s);
      break;
    case MmaIn::I8:
      if (out == MmaOut::I32) return run<OpI8, MmaOut::I32>(d, s);
      if (out == MmaOut::DEQ_BF16) return run<OpI8, MmaOut::DEQ_BF16>(d, s);
      break;
    case MmaIn::F32:
      if (out == MmaOut::F32) return run<OpF32, MmaOut::F32>(d, s);
      break;
  }
  return hipErrorNotSupported;
}

size_t gemm_workspace_bytes(MmaIn in, MmaOut out, const GemmDesc& d) {
  switch (in) {
    case MmaIn::BF16:
      if (out == MmaOut::F32) return workspace<OpBF16, MmaOut::F32>(d);
      if (out == MmaOut::BF16) return workspace<OpBF16, MmaOut::BF16>(d);
      break;
    case MmaIn::F16:
      if (out == MmaOut::F32) return workspace<OpF16, MmaOut::F32>(d);
      if (out == MmaOut::F16) return workspace<OpF16, MmaOut::F16>(d);
      break;
    case MmaIn::I8:
      if (out == MmaOut::I32) return workspace<OpI8, MmaOut::I32>(d);
      if (out == MmaOut::DEQ_BF16) return workspace<OpI8, MmaOut::DEQ_BF16>(d);
      break;
    case MmaIn::F32:
      if (out == MmaOut::F32) return workspace<OpF32, MmaOut::F32>(d);
      break;
  }
  return 0;
}

// One workgroup per CU, so workgroups (tiles x batch x K slices) run in
// waves of 256; a last wave that is mostly empty costs a whole wave here,
// where sgemm_mfma (4 workgroups of 128x128 per CU) finishes such a tail
// sooner (4000x4100x1000: 68 against 87 TFLOP/s). Taken with at least 4
// waves, or a last wave at least 3/4 full.
bool fp32_mma_wanted(const GemmDesc& d) {
  if (d.probe || d.m <= 0 || d.n <= 0 || d.batch <= 0) return false;
  const Plan t = make_plan<OpF32, MmaOut::F32>(d);
  if (!t.tn) return false;
  const int64_t tiles = (int64_t)((d.m + kFastTile - 1) / kFastTile) * ((d.n + kFastTile - 1) / kFastTile);
  if (t.split > 1 && tiles >= kSplitTiles) {
    // A problem sgemm_mfma fills too: split only where the model beats that
    // kernel's best rate, ~134 TFLOP/s (6144^3: 134 -> 140, 4608^3: 112 ->
    // 132, 5120^3: 120 -> 132; 6144^2 x 2048 stays at 133, split 120).
    const double flops = 2.0 * d.m * d.n * d.k;
    return (double)t.split_ns * 134000.0 < flops;
  }
  const int64_t units = tiles * d.batch * t.split;
  const int64_t waves = (units + 255) / 256;
  const int64_t last = units - (waves - 1) * 256;
  return units >= 256 && (waves >= 4 || last >= 192);
}

}  // namespace grxk
