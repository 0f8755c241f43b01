// Shared device helpers for the RoLaQ packed-INT2 MLA kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace rolaq {

constexpr int kGroup = 128;            // quantization group (elements)
constexpr int kCodesPerWord = 16;      // 2-bit codes per 32-bit word
constexpr float kZeroOffset = 1.5f;    // -C0 / (span / 3) of the Lloyd grid
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNeutralLse = -1.0e4f;  // empty split (SGLang decode convention)

// D = A(16x32) * B(32x16) + C on bf16 inputs, fp32 accumulate.
// Lane l holds A[l%16][8(l/16)+i], B[8(l/16)+i][l%16] (i = 0..7, two per dword,
// low half first) and C[4(l/16)+j][l%16] (j = 0..3).
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// The same product on fp16 inputs (same operand layout).
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f32x4 mfma16x16x32_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                0, 0);
}

// Two fp32 -> one dword of two fp16 (round to nearest even; beyond 65504 -> inf).
__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
  f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2_t));
}

// Two fp32 -> one dword of two bf16 (round to nearest even), low half = lo.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_float(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }
__device__ __forceinline__ uint16_t float_to_bf16(float f) {
  return uint16_t(pack_bf16(f, 0.0f) & 0xffffu);
}

// The correctly rounded FP32 quotient d / s from y = RN(1 / s) (one true
// division per divisor): q0 = RN(d y), the exact remainder r = d - q0 s, then
// RN(q0 + r y) (Markstein's quotient correction with a fused multiply-add,
// P. Markstein, IBM J. Res. Dev. 34(1), 1990). Used where many values share a
// divisor; checked against true division in tests/test_division_identity.py.
__device__ __forceinline__ float div_by(float d, float s, float y) {
  const float q0 = d * y;
  return fmaf(fmaf(-q0, s, d), y, q0);
}

// Load through a global (address space 1) pointer: a global_load, which only
// vmcnt tracks. A load through a generic pointer becomes flat_load, which LDS
// waits (lgkmcnt) must also drain.
template <typename T>
__device__ __forceinline__ T gload(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

// One dword of two bf16 -> the same two values as fp16 (exact for magnitudes
// in [2^-24, 65504] that fit fp16's 11-bit significand, which covers every bf16
// value in [2^-17, 65504]; beyond 65504 -> inf).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t v) { return pack_f16(bf16_lo(v), bf16_hi(v)); }
// One dword of two fp16 -> the same two values as bf16 (exact for fp16 values
// that are bf16 numbers, as the decode's levels and window rows are).
__device__ __forceinline__ uint32_t f16x2_to_bf16x2(uint32_t v) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, v);
  return pack_bf16((float)h[0], (float)h[1]);
}
__device__ __forceinline__ u32x4 bf16x8_to_f16x8(u32x4 v) {
  return u32x4{bf16x2_to_f16x2(v.x), bf16x2_to_f16x2(v.y), bf16x2_to_f16x2(v.z), bf16x2_to_f16x2(v.w)};
}

__device__ __forceinline__ float wave_max_over_groups(float v) {
  // max over lanes l, l^16, l^32, l^48 (the four 16-lane rows of a wave)
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
__device__ __forceinline__ float wave_sum_over_groups(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

}  // namespace rolaq
