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

// Lloyd code thresholds moved from the quotient to its numerator. For a float
// threshold th and s > 0, RN(y / s) >= th holds exactly when y / s >= mu, or
// y / s > mu when th's significand is odd (the tie at mu then rounds to the
// float below th), mu being the midpoint of th and the next float below it.
// mu has at most 26 significant bits, so s * mu is exact in FP64, and the
// smallest float y passing the test is s * mu rounded up (one float further
// when the test is strict and s * mu is itself a float). Comparing y with
// these per-row floats gives the codes of the correctly rounded quotient
// (mla_quant/oscar.py:135-140) with no division per element; checked against
// true division in tests/test_division_identity.py.
__device__ __forceinline__ double below_midpoint(float th) {
  const uint32_t b = __float_as_uint(th);
  const uint32_t below = (b << 1) == 0 ? 0x80000001u : ((int32_t)b < 0 ? b + 1 : b - 1);
  return 0.5 * ((double)__uint_as_float(below) + (double)th);
}

__device__ __forceinline__ bool threshold_inclusive(float th) { return (__float_as_uint(th) & 1u) == 0; }

__device__ __forceinline__ float y_threshold(double s, double mu, bool incl) {
  const double p = s * mu;
  const float y = (float)p;
  const double yd = (double)y;
  if (incl ? !(yd < p) : !(yd <= p)) return y;  // also NaN: every test fails
  const uint32_t b = __float_as_uint(y);
  return __uint_as_float((b << 1) == 0 ? 1u : ((int32_t)b < 0 ? b - 1 : b + 1));
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

// In-place scaling of an output accumulator held in an AGPR tuple. The
// compiler prints an "a" operand of four floats as a[b:b+3]; the assembler
// macro ROLAQ_ACC_BASE recovers b by comparing that text with every even base
// (an operand anywhere else stops the assembly with an error), so that
// ROLAQ_ACC_SCALE can read, scale and write the four registers one by one
// (v_accvgpr_read / v_mul_f32 / v_accvgpr_write) without the compiler ever
// seeing the accumulators leave their registers. Inline asm blobs share one
// assembler state in order of emission, so the definitions are made once, at
// the start of each kernel.
#define ROLAQ_ACC_CASE(k, k3) "  .ifc \\t, a[" #k ":" #k3 "]\n    .set rolaq_acc_b, " #k "\n  .endif\n"
#define ROLAQ_ACC_CASES \
  ROLAQ_ACC_CASE(0, 3) ROLAQ_ACC_CASE(2, 5) ROLAQ_ACC_CASE(4, 7) ROLAQ_ACC_CASE(6, 9) ROLAQ_ACC_CASE(8, 11) ROLAQ_ACC_CASE(10, 13) \
  ROLAQ_ACC_CASE(12, 15) ROLAQ_ACC_CASE(14, 17) ROLAQ_ACC_CASE(16, 19) ROLAQ_ACC_CASE(18, 21) ROLAQ_ACC_CASE(20, 23) ROLAQ_ACC_CASE(22, 25) \
  ROLAQ_ACC_CASE(24, 27) ROLAQ_ACC_CASE(26, 29) ROLAQ_ACC_CASE(28, 31) ROLAQ_ACC_CASE(30, 33) ROLAQ_ACC_CASE(32, 35) ROLAQ_ACC_CASE(34, 37) \
  ROLAQ_ACC_CASE(36, 39) ROLAQ_ACC_CASE(38, 41) ROLAQ_ACC_CASE(40, 43) ROLAQ_ACC_CASE(42, 45) ROLAQ_ACC_CASE(44, 47) ROLAQ_ACC_CASE(46, 49) \
  ROLAQ_ACC_CASE(48, 51) ROLAQ_ACC_CASE(50, 53) ROLAQ_ACC_CASE(52, 55) ROLAQ_ACC_CASE(54, 57) ROLAQ_ACC_CASE(56, 59) ROLAQ_ACC_CASE(58, 61) \
  ROLAQ_ACC_CASE(60, 63) ROLAQ_ACC_CASE(62, 65) ROLAQ_ACC_CASE(64, 67) ROLAQ_ACC_CASE(66, 69) ROLAQ_ACC_CASE(68, 71) ROLAQ_ACC_CASE(70, 73) \
  ROLAQ_ACC_CASE(72, 75) ROLAQ_ACC_CASE(74, 77) ROLAQ_ACC_CASE(76, 79) ROLAQ_ACC_CASE(78, 81) ROLAQ_ACC_CASE(80, 83) ROLAQ_ACC_CASE(82, 85) \
  ROLAQ_ACC_CASE(84, 87) ROLAQ_ACC_CASE(86, 89) ROLAQ_ACC_CASE(88, 91) ROLAQ_ACC_CASE(90, 93) ROLAQ_ACC_CASE(92, 95) ROLAQ_ACC_CASE(94, 97) \
  ROLAQ_ACC_CASE(96, 99) ROLAQ_ACC_CASE(98, 101) ROLAQ_ACC_CASE(100, 103) ROLAQ_ACC_CASE(102, 105) ROLAQ_ACC_CASE(104, 107) ROLAQ_ACC_CASE(106, 109) \
  ROLAQ_ACC_CASE(108, 111) ROLAQ_ACC_CASE(110, 113) ROLAQ_ACC_CASE(112, 115) ROLAQ_ACC_CASE(114, 117) ROLAQ_ACC_CASE(116, 119) ROLAQ_ACC_CASE(118, 121) \
  ROLAQ_ACC_CASE(120, 123) ROLAQ_ACC_CASE(122, 125) ROLAQ_ACC_CASE(124, 127) ROLAQ_ACC_CASE(126, 129) ROLAQ_ACC_CASE(128, 131) ROLAQ_ACC_CASE(130, 133) \
  ROLAQ_ACC_CASE(132, 135) ROLAQ_ACC_CASE(134, 137) ROLAQ_ACC_CASE(136, 139) ROLAQ_ACC_CASE(138, 141) ROLAQ_ACC_CASE(140, 143) ROLAQ_ACC_CASE(142, 145) \
  ROLAQ_ACC_CASE(144, 147) ROLAQ_ACC_CASE(146, 149) ROLAQ_ACC_CASE(148, 151) ROLAQ_ACC_CASE(150, 153) ROLAQ_ACC_CASE(152, 155) ROLAQ_ACC_CASE(154, 157) \
  ROLAQ_ACC_CASE(156, 159) ROLAQ_ACC_CASE(158, 161) ROLAQ_ACC_CASE(160, 163) ROLAQ_ACC_CASE(162, 165) ROLAQ_ACC_CASE(164, 167) ROLAQ_ACC_CASE(166, 169) \
  ROLAQ_ACC_CASE(168, 171) ROLAQ_ACC_CASE(170, 173) ROLAQ_ACC_CASE(172, 175) ROLAQ_ACC_CASE(174, 177) ROLAQ_ACC_CASE(176, 179) ROLAQ_ACC_CASE(178, 181) \
  ROLAQ_ACC_CASE(180, 183) ROLAQ_ACC_CASE(182, 185) ROLAQ_ACC_CASE(184, 187) ROLAQ_ACC_CASE(186, 189) ROLAQ_ACC_CASE(188, 191) ROLAQ_ACC_CASE(190, 193) \
  ROLAQ_ACC_CASE(192, 195) ROLAQ_ACC_CASE(194, 197) ROLAQ_ACC_CASE(196, 199) ROLAQ_ACC_CASE(198, 201) ROLAQ_ACC_CASE(200, 203) ROLAQ_ACC_CASE(202, 205) \
  ROLAQ_ACC_CASE(204, 207) ROLAQ_ACC_CASE(206, 209) ROLAQ_ACC_CASE(208, 211) ROLAQ_ACC_CASE(210, 213) ROLAQ_ACC_CASE(212, 215) ROLAQ_ACC_CASE(214, 217) \
  ROLAQ_ACC_CASE(216, 219) ROLAQ_ACC_CASE(218, 221) ROLAQ_ACC_CASE(220, 223) ROLAQ_ACC_CASE(222, 225) ROLAQ_ACC_CASE(224, 227) ROLAQ_ACC_CASE(226, 229) \
  ROLAQ_ACC_CASE(228, 231) ROLAQ_ACC_CASE(230, 233) ROLAQ_ACC_CASE(232, 235) ROLAQ_ACC_CASE(234, 237) ROLAQ_ACC_CASE(236, 239) ROLAQ_ACC_CASE(238, 241) \
  ROLAQ_ACC_CASE(240, 243) ROLAQ_ACC_CASE(242, 245) ROLAQ_ACC_CASE(244, 247) ROLAQ_ACC_CASE(246, 249) ROLAQ_ACC_CASE(248, 251) ROLAQ_ACC_CASE(250, 253) \
  ROLAQ_ACC_CASE(252, 255)
// Defines the macros for the rest of the assembly (each kernel calls it first;
// the assembler keeps the definitions, and the guard skips a second one).
__device__ __forceinline__ void define_acc_macros() {
  asm volatile(
    ".ifndef rolaq_acc_macros\n"
    ".set rolaq_acc_macros, 1\n"
    ".macro ROLAQ_ACC_BASE t\n"
    "  .set rolaq_acc_b, -1\n" ROLAQ_ACC_CASES
    "  .if rolaq_acc_b < 0\n"
    "    .error \"ROLAQ_ACC_BASE: not an AGPR tuple\"\n"
    "  .endif\n"
    ".endm\n"
    ".macro ROLAQ_ACC_SCALE t, t0, t1, t2, t3, f0, f1, f2, f3\n"
    "  ROLAQ_ACC_BASE \\t\n"
    "  v_accvgpr_read_b32 \\t0, a[rolaq_acc_b]\n"
    "  v_accvgpr_read_b32 \\t1, a[rolaq_acc_b+1]\n"
    "  v_accvgpr_read_b32 \\t2, a[rolaq_acc_b+2]\n"
    "  v_accvgpr_read_b32 \\t3, a[rolaq_acc_b+3]\n"
    "  s_nop 1\n"
    "  v_mul_f32_e32 \\t0, \\t0, \\f0\n"
    "  v_mul_f32_e32 \\t1, \\t1, \\f1\n"
    "  v_mul_f32_e32 \\t2, \\t2, \\f2\n"
    "  v_mul_f32_e32 \\t3, \\t3, \\f3\n"
    "  s_nop 1\n"
    "  v_accvgpr_write_b32 a[rolaq_acc_b], \\t0\n"
    "  v_accvgpr_write_b32 a[rolaq_acc_b+1], \\t1\n"
    "  v_accvgpr_write_b32 a[rolaq_acc_b+2], \\t2\n"
    "  v_accvgpr_write_b32 a[rolaq_acc_b+3], \\t3\n"
    ".endm\n"
    ".endif\n");
}
#undef ROLAQ_ACC_CASES
#undef ROLAQ_ACC_CASE

// Four output accumulators, element j of each scaled by f_j in place when
// need (a lane mask) is not 0. The branch is inside the asm: for the compiler
// the accumulators flow through unchanged in their registers, so the rare
// rescale adds no copies at a join. The leading waits cover the output MFMA
// that last wrote them (tens of instructions earlier), the trailing ones an
// MFMA that reads them next.
__device__ __forceinline__ void scale_acc4(f32x4& a, f32x4& b, f32x4& c, f32x4& d, const float (&f)[4],
                                           uint64_t need) {
  float t0, t1, t2, t3;
  asm volatile(
      "s_cmp_lg_u64 %12, 0\n\t"
      "s_cbranch_scc0 1f\n\t"
      "s_nop 7\n\ts_nop 7\n\t"
      "ROLAQ_ACC_SCALE %0, %4, %5, %6, %7, %8, %9, %10, %11\n\t"
      "ROLAQ_ACC_SCALE %1, %4, %5, %6, %7, %8, %9, %10, %11\n\t"
      "ROLAQ_ACC_SCALE %2, %4, %5, %6, %7, %8, %9, %10, %11\n\t"
      "ROLAQ_ACC_SCALE %3, %4, %5, %6, %7, %8, %9, %10, %11\n\t"
      "s_nop 7\n"
      "1:"
      : "+a"(a), "+a"(b), "+a"(c), "+a"(d), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
      : "v"(f[0]), "v"(f[1]), "v"(f[2]), "v"(f[3]), "s"(need)
      : "scc");
}

// scale_acc4 over 16 accumulator tuples behind one test of the lane mask
// (one branch instead of four when nothing is scaled)
__device__ __forceinline__ void scale_acc16(f32x4 (&o)[16], const float (&f)[4], uint64_t need) {
  float t0, t1, t2, t3;
  asm volatile(
      "s_cmp_lg_u64 %24, 0\n\t"
      "s_cbranch_scc0 1f\n\t"
      "s_nop 7\n\ts_nop 7\n\t"
      "ROLAQ_ACC_SCALE %0, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %1, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %2, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %3, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %4, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %5, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %6, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %7, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %8, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %9, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %10, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %11, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %12, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %13, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %14, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "ROLAQ_ACC_SCALE %15, %16, %17, %18, %19, %20, %21, %22, %23\n\t"
      "s_nop 7\n"
      "1:"
      : "+a"(o[0]), "+a"(o[1]), "+a"(o[2]), "+a"(o[3]), "+a"(o[4]), "+a"(o[5]), "+a"(o[6]), "+a"(o[7]),
        "+a"(o[8]), "+a"(o[9]), "+a"(o[10]), "+a"(o[11]), "+a"(o[12]), "+a"(o[13]), "+a"(o[14]), "+a"(o[15]),
        "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
      : "v"(f[0]), "v"(f[1]), "v"(f[2]), "v"(f[3]), "s"(need)
      : "scc");
}

// acc + lo + hi of a packed pair of fp16 values (exact products by one,
// FP32 accumulation: v_dot2_f32_f16)
__device__ __forceinline__ float sum_f16x2(uint32_t v, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v), h2{(_Float16)1.0f, (_Float16)1.0f}, acc, false);
}

// all-ones when keep, else zero: a branch-free "keep ? v : 0" on bit patterns
__device__ __forceinline__ uint32_t keep_mask(bool keep) { return keep ? 0xFFFFFFFFu : 0u; }

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
