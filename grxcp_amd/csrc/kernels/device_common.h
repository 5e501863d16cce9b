// Device-side helpers shared by the gfx950 kernels: vector types, exact
// narrow-float conversions, wavefront reductions and the cycle probe.
#ifndef GRXCP_DEVICE_COMMON_H
#define GRXCP_DEVICE_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <grx/grx_cycles.h>

namespace grxk {

typedef int      i32x4  __attribute__((ext_vector_type(4)));
typedef int      i32x16 __attribute__((ext_vector_type(16)));
typedef float    f32x4  __attribute__((ext_vector_type(4)));
typedef float    f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16   bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8  __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2  __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4  __attribute__((ext_vector_type(4)));

// ---- narrow float formats (bit patterns in uint16_t) ----------------------

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t x = __float_as_uint(f);
  if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu))
    return (uint16_t)((x >> 16) | 0x40u);
  return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

// Two fp32 -> packed bf16x2 (low half = a) in one v_cvt_pk_bf16_f32: round
// to nearest even, NaN quieted -- the same bits as f32_to_bf16 on each half.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// fp32 <-> fp16 through the hardware converts (v_cvt_f16_f32 rounds to
// nearest even and keeps subnormals; v_cvt_f32_f16 is exact).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  const _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

// Two fp32 -> packed fp16x2 (low half = a), round to nearest even.
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  const f16x2 v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// ---- reductions over one 64-wide wavefront ---------------------------------

// A butterfly that stays in the ALU: DPP moves within each row of 16 lanes
// (quad permutes [1,0,3,2] and [2,3,0,1], then the half-row and row
// mirrors, each pairing lanes whose partial results are disjoint), then
// gfx950's row-swap instructions across rows of 16 and halves of 32. Every
// lane ends with the same value (each step combines the same two partials
// in every lane, and op is commutative). The shuffle form (__shfl_xor)
// compiles to six dependent ds_bpermute LDS round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp_f<0xb1>(v));    // quad_perm [1,0,3,2]: lane ^ 1
  v = op(v, dpp_f<0x4e>(v));    // quad_perm [2,3,0,1]: lane ^ 2
  v = op(v, dpp_f<0x141>(v));   // row_half_mirror: the other quad of 8
  v = op(v, dpp_f<0x140>(v));   // row_mirror: the other 8 of 16
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));   // the other row of 16
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));   // the other half of 32
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}

// ---- cycle probe -------------------------------------------------------------
// One grxCycleSlot per wave, written by lane 0 with an ordinary (vector)
// global store. `core` = XCD id << 16 | CU-level hardware id bits, so slots
// from different clock domains are distinguishable.

__device__ __forceinline__ uint64_t cycle_now() { return __builtin_amdgcn_s_memtime(); }

__device__ __forceinline__ uint32_t hw_core_id() {
  // HW_REG_HW_ID (id 4): bits [15:8] hold CU/SH/SE; HW_REG_XCC_ID (id 20)
  // bits [3:0] the XCD.
  const uint32_t hwid = __builtin_amdgcn_s_getreg((31 << 11) | (0 << 6) | 4);
  const uint32_t xcc = __builtin_amdgcn_s_getreg((15 << 11) | (0 << 6) | 20);
  return ((xcc & 0xfu) << 16) | ((hwid >> 8) & 0xffu);
}

__device__ __forceinline__ void cycle_record(grxCycleSlot* slots, uint64_t t0,
                                             uint32_t slot, uint32_t wave) {
  if (!slots) return;
  if ((threadIdx.x & 63) != 0) return;
  const uint64_t t1 = cycle_now();
  grxCycleSlot s;
  s.start = t0;
  s.end = t1;
  s.core = hw_core_id();
  s.warp = wave;
  slots[slot] = s;
}

}  // namespace grxk

#endif  // GRXCP_DEVICE_COMMON_H
