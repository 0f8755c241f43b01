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

// D = A(16x128) * B(128x16) 2^(sb - 127) + C with A in fp4 (e2m1) and B in fp8
// (e4m3, OCP), fp32 accumulate (v_mfma_scale_f32_16x16x128_f8f6f4, 32 cycles).
// sb is the E8M0 block scale of the lane's 32 K-elements of B (A's scale is 1).
// Operand layouts (checked on the device):
//   A lane l (row l%16, G = l/16): dword d (0..3) nibble n <-> K = 64(G&1) + 16(G>>1) + 32(d>>1) + 8(d&1) + n
//   B lane l (col l%16, G = l/16): dword i (0..7) byte b  <-> K = 32G + 4i + b
//   C as for mfma16x16x32.
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mfma_f4_f8(u32x4 a, u32x8 b, f32x4 c, int sb) {
  typedef int i32x4_t __attribute__((ext_vector_type(4)));
  typedef int i32x8_t __attribute__((ext_vector_type(8)));
  const i32x4_t a4 = __builtin_bit_cast(i32x4_t, a);
  const i32x8_t a8 = __builtin_shufflevector(a4, a4, 0, 1, 2, 3, -1, -1, -1, -1);  // fp4 uses 4 dwords
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, __builtin_bit_cast(i32x8_t, b), c, 4, 0, 0, 127, 0,
                                                          sb);
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

// In-place unpack of one packed word (16 codes; code p at bits 2p) into eight
// dwords of two bf16 each. Dword k holds (code k, code k + 8) as the bf16
// values 4 + c * 2^(e_k - 5), e = {0, 2, 4, 0, 2, 4, 0, 2}: the code bits are
// masked straight into the mantissa of 4.0 (0x4080), so a dword costs one
// and-or (plus a shared shift for k >= 3).
__device__ __forceinline__ void unpack_word(uint32_t w, uint32_t d[8]) {
  const uint32_t base = 0x40804080u;
  d[0] = (w & 0x00030003u) | base;
  d[1] = (w & 0x000C000Cu) | base;
  d[2] = (w & 0x00300030u) | base;
  const uint32_t w6 = w >> 6;
  d[3] = (w6 & 0x00030003u) | base;
  d[4] = (w6 & 0x000C000Cu) | base;
  d[5] = (w6 & 0x00300030u) | base;
  const uint32_t w12 = w >> 12;
  d[6] = (w12 & 0x00030003u) | base;
  d[7] = (w12 & 0x000C000Cu) | base;
}

// Mantissa shift e_k of pair k in unpack_word; the decoded value is
// 4 + c * 2^(e_k - 5), so weights on pair k are scaled by 2^(5 - e_k).
__host__ __device__ constexpr int pair_shift(int k) { return k < 3 ? 2 * k : (k < 6 ? 2 * k - 6 : 2 * k - 12); }
__host__ __device__ constexpr float pair_weight(int k) { return float(1 << (5 - pair_shift(k))); }

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
