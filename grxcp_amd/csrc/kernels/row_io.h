// Element access for the grxDNN row kernels (norms, softmax, GELU): 16-byte
// chunks of bf16 / fp16 / fp32 unpacked to fp32 and packed back with round
// to nearest even, plus single-element access for unaligned rows.
#ifndef GRXCP_ROW_IO_H
#define GRXCP_ROW_IO_H

#include "../launch.h"
#include "device_common.h"

namespace grxk {

template <NormType T> struct Io;  // NormType doubles as the row element type
template <> struct Io<NormType::BF16> {
  static constexpr int kVec = 8;
  __device__ static float ld(const uint8_t* p, int64_t i) { return bf16_to_f32(((const uint16_t*)p)[i]); }
  __device__ static void st(uint8_t* p, int64_t i, float v) { ((uint16_t*)p)[i] = f32_to_bf16(v); }
  __device__ static void unpack(const u32x4 w, float* f) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f[2 * q] = __uint_as_float(w[q] << 16);
      f[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
    }
  }
  __device__ static u32x4 pack(const float* f) {
    // v_cvt_pk_bf16_f32: round to nearest even, NaN quieted -- the same
    // bits as f32_to_bf16.
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    u32x4 w;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bf16x2 v = {(__bf16)f[2 * q], (__bf16)f[2 * q + 1]};
      w[q] = __builtin_bit_cast(uint32_t, v);
    }
    return w;
  }
};
template <> struct Io<NormType::F16> {
  static constexpr int kVec = 8;
  __device__ static float ld(const uint8_t* p, int64_t i) { return f16_to_f32(((const uint16_t*)p)[i]); }
  __device__ static void st(uint8_t* p, int64_t i, float v) { ((uint16_t*)p)[i] = f32_to_f16(v); }
  __device__ static void unpack(const u32x4 w, float* f) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f[2 * q] = f16_to_f32((uint16_t)(w[q] & 0xffffu));
      f[2 * q + 1] = f16_to_f32((uint16_t)(w[q] >> 16));
    }
  }
  __device__ static u32x4 pack(const float* f) {
    u32x4 w;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w[q] = (uint32_t)f32_to_f16(f[2 * q]) | ((uint32_t)f32_to_f16(f[2 * q + 1]) << 16);
    return w;
  }
};
template <> struct Io<NormType::F32> {
  static constexpr int kVec = 4;
  __device__ static float ld(const uint8_t* p, int64_t i) { return ((const float*)p)[i]; }
  __device__ static void st(uint8_t* p, int64_t i, float v) { ((float*)p)[i] = v; }
  __device__ static void unpack(const u32x4 w, float* f) {
#pragma unroll
    for (int q = 0; q < 4; ++q) f[q] = __uint_as_float(w[q]);
  }
  __device__ static u32x4 pack(const float* f) {
    u32x4 w;
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = __float_as_uint(f[q]);
    return w;
  }
};

}  // namespace grxk

#endif  // GRXCP_ROW_IO_H
