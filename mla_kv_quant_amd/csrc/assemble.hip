// Dequantize-rows ("assemble") kernel: cache rows of the packed pool as bf16
// [latent | rope] rows, the latent optionally rotated back to the model's
// frame. Serves MHA-style prefill over a quantized prefix, whose kv_b_proj
// consumes un-rotated latents (deployment/sglang/srt/mem_cache/rolaq_mla.py:60-61;
// the fork's _assemble_rows_kernel, deployment/patches/rolaq_sglang.patch:5-6,
// writes [latent | rope] per row).
//
// Row value: the BF16 window row when the slot still owns its window row
// (row_of_slot[slot] = r >= 0 and owner_of_row[r] == slot), else the INT2
// row dequantized as (code - zero) * scale and rounded to bf16 -- the cache's
// stored form (mla_quant/quantizer.py:117-121). Un-rotation multiplies that
// bf16 row by R_eff^T in FP32 (bf16 MFMA, exact products) and rounds to bf16,
// the cast order of rotate_quantize (quantizer.py:121-122).
#include "rolaq_common.h"
#include "rolaq_args.h"

namespace rolaq {

constexpr int kAsmRows = 64;  // rows per block

template <int D>
__global__ __launch_bounds__(256) void assemble_kernel(AssembleArgs a) {
  constexpr int NG = D / 128, STR = 2 * D + 16, CPR = D / 8;  // 16-byte chunks per latent row
  constexpr int KS = D / 32, MB = D / 4 / 16;                // K-steps; 16-column blocks per wave
  __shared__ __attribute__((aligned(16))) uint8_t s_x[kAsmRows * STR];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gq = lane >> 4, la = lane & 15;
  const int64_t row0 = (int64_t)blockIdx.x * kAsmRows;

  // ---- gather: window row or dequantized INT2 row, as bf16 -----------------------
  for (int c = tid; c < kAsmRows * CPR; c += 256) {
    const int r = c / CPR, ch = c % CPR;
    const int64_t row = row0 + r;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row < a.n) {
      const int64_t slot = a.slots[row];
      const int32_t hr = a.row_of_slot[slot];
      if (hr >= 0 && a.owner_of_row[hr] == (int32_t)slot) {
        v = *reinterpret_cast<const u32x4*>(a.hp + (int64_t)hr * D + 8 * ch);
      } else {
        const int d0 = 8 * ch, g = d0 / 128, e0 = d0 % 128;
        const uint32_t w = *reinterpret_cast<const uint32_t*>(a.codes + slot * (D / 4) + 4 * (NG * (e0 / 16) + g));
        const uint32_t bits = w >> (16 * ((e0 / 8) & 1));
        const f32x2 p = *reinterpret_cast<const f32x2*>(a.params + slot * 2 * NG + 2 * g);
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (float((bits >> (2 * e)) & 3u) - p.y) * p.x;
        v = u32x4{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])};
      }
    }
    if (a.rot) {
      *reinterpret_cast<u32x4*>(s_x + r * STR + 16 * ch) = v;
    } else if (row < a.n) {
      *reinterpret_cast<u32x4*>(a.out + row * a.out_st + 8 * ch) = v;
    }
  }
  // ---- rope columns ------------------------------------------------------------------
  for (int c = tid; c < kAsmRows * (a.R / 8); c += 256) {
    const int r = c / (a.R / 8), ch = c % (a.R / 8);
    const int64_t row = row0 + r;
    if (row < a.n) {
      const int64_t slot = a.slots[row];
      *reinterpret_cast<u32x4*>(a.out + row * a.out_st + D + 8 * ch) =
          *reinterpret_cast<const u32x4*>(a.rope + slot * a.R + 8 * ch);
    }
  }
  if (!a.rot) return;
  __syncthreads();

  // ---- un-rotate: out[row, col] = sum_k x[row, k] R_eff[col, k] ------------------------
  // wave w: columns [D/4 w, D/4 (w+1)); MFMA M = columns (A from R_eff rows),
  // N = rows (B from LDS), so lane (la, gq) ends with 4 consecutive columns of a row.
  const int c0 = (D / 4) * wave;
  f32x4 acc[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int ks = 0; ks < KS; ++ks) {
    u32x4 xb[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
      xb[nb] = *reinterpret_cast<const u32x4*>(s_x + (16 * nb + la) * STR + 64 * ks + 16 * gq);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const u32x4 ra = *reinterpret_cast<const u32x4*>(a.rot + (int64_t)(c0 + 16 * mb + la) * D + 32 * ks + 8 * gq);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mfma16x16x32(ra, xb[nb], acc[mb][nb]);
    }
  }
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int64_t row = row0 + 16 * nb + la;
    if (row >= a.n) continue;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const f32x4 v = acc[mb][nb];
      *reinterpret_cast<u32x2*>(a.out + row * a.out_st + c0 + 16 * mb + 4 * gq) =
          u32x2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
    }
  }
}

}  // namespace rolaq

hipError_t rolaq_launch_assemble(const rolaq::AssembleArgs& a, int D, hipStream_t stream) {
  using namespace rolaq;
  const dim3 grid((unsigned)((a.n + kAsmRows - 1) / kAsmRows)), block(256);
  if (D == 512) {
    hipLaunchKernelGGL((assemble_kernel<512>), grid, block, 0, stream, a);
  } else if (D == 256) {
    hipLaunchKernelGGL((assemble_kernel<256>), grid, block, 0, stream, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
