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

// Rows in the rotated frame (rot == null): a gather, 16 bytes per thread.
template <int D>
__global__ __launch_bounds__(256) void assemble_kernel(AssembleArgs a) {
  constexpr int NG = D / 128, CPR = D / 8;  // 16-byte chunks per latent row
  const int tid = threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * kAsmRows;

  // ---- window row or dequantized INT2 row, as bf16 ---------------------------------
  for (int c = tid; c < kAsmRows * CPR; c += 256) {
    const int r = c / CPR, ch = c % CPR;
    const int64_t row = row0 + r;
    if (row >= a.n) continue;
    const int64_t slot = a.slots[row];
    const int32_t hr = a.row_of_slot[slot];
    u32x4 v;
    if (hr >= 0 && a.owner_of_row[hr] == (int32_t)slot) {
      v = *reinterpret_cast<const u32x4*>(a.hp + (int64_t)hr * D + 8 * ch);
    } else {
      const int d0 = 8 * ch, g = d0 / 128;
      // elements d0 .. d0+7: bytes d0/4, d0/4 + 1 of the packed row
      const uint32_t bits = *reinterpret_cast<const uint16_t*>(a.codes + slot * (D / 4) + d0 / 4);
      const f32x2 p = *reinterpret_cast<const f32x2*>(a.params + slot * 2 * NG + 2 * g);
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (float((bits >> (2 * e)) & 3u) - p.y) * p.x;
      v = u32x4{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])};
    }
    *reinterpret_cast<u32x4*>(a.out + row * a.out_st + 8 * ch) = v;
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
}

// ---------------------------------------------------------------------------
// Rows rotated back (rot != null): a GEMM out[n, D] = X[n, D] R_eff^T with X
// the bf16 rows above. A block takes 128 rows: it gathers them into LDS once
// (per-row source first, then 16-byte chunks), and its 8 waves each own D/8
// output columns over all 128 rows -- MFMA 16x16x32 with R_eff rows as the A
// operand, streamed from global memory (L2-resident, shared by all blocks) one
// K-step ahead, and the LDS rows as the B operand. Per K-step and wave: D/128
// R loads of 16 bytes per lane (and 4 D/128 ds_bpermute), 8 LDS reads,
// 8 D/128 MFMAs.
// ---------------------------------------------------------------------------
constexpr int kAsmRotRows = 128;
constexpr int kAsmRotWaves = 8;

template <int D>
struct AsmRotGeo {
  static constexpr int STR = 2 * D + 16;  // bytes per LDS row (padded)
  static constexpr int LDS = kAsmRotRows * STR;
};

template <int D>
__global__ __launch_bounds__(64 * kAsmRotWaves, 1) void assemble_rot_kernel(AssembleArgs a) {
  constexpr int NG = D / 128, STR = AsmRotGeo<D>::STR, KS = D / 32;
  constexpr int CW = D / kAsmRotWaves, MB = CW / 16, NB = kAsmRotRows / 16;
  constexpr int NT = 64 * kAsmRotWaves;
  extern __shared__ __attribute__((aligned(16))) uint8_t s_x[];
  __shared__ int64_t s_slot[kAsmRotRows];
  __shared__ int32_t s_hr[kAsmRotRows];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gq = lane >> 4, la = lane & 15;
  const int64_t row0 = (int64_t)blockIdx.x * kAsmRotRows;

  // This wave's R_eff rows c0 + 16 mb + (0..15). They are loaded coalesced --
  // lanes 4r..4r+3 read the 64 contiguous bytes of row r for one K-step, so a
  // 16-lane pass touches 4 rows, not 16 -- and moved to the MFMA lane layout
  // (lane la + 16 gq <- lane 4 la + gq) with ds_bpermute. The first K-step's
  // loads are in flight during the gather.
  const int c0 = CW * wave;
  const uint16_t* rbase = a.rot + (int64_t)(c0 + (lane >> 2)) * D + 8 * (lane & 3);
  const int perm = 4 * (4 * la + gq);
  auto relayout = [&](u32x4 v) {
    return u32x4{(uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v.x),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v.y),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v.z),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v.w)};
  };
  u32x4 rr[2][MB];  // raw (load-layout) R chunks, one K-step ahead
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) rr[0][mb] = gload<u32x4>(rbase + 16 * mb * D);

  // ---- per-row source: the window row while the slot owns it, else INT2 ---------
  if (tid < kAsmRotRows) {
    const int64_t row = row0 + tid;
    int64_t slot = -1;
    int32_t hr = -1;
    if (row < a.n) {
      slot = a.slots[row];
      const int32_t r = a.row_of_slot[slot];
      if (r >= 0 && a.owner_of_row[r] == (int32_t)slot) hr = r;
    }
    s_slot[tid] = slot;
    s_hr[tid] = hr;
  }
  __syncthreads();
  // ---- gather the rows as bf16 into LDS (rows past n as zeros) --------------------
  // One item = row r and its 16-byte code chunk j: dword q = 4j + i is word q
  // of the row, columns 16 q + (0..15) of group q / 8; each dword gives two
  // 16-byte LDS chunks. Few, wide loads per thread keep many
  // in flight.
  constexpr int CCH = D / 64;  // 16-byte code chunks per row
  for (int c = tid; c < kAsmRotRows * CCH; c += NT) {
    const int r = c / CCH, j = c % CCH;
    const int64_t slot = s_slot[r];
    const int32_t hr = s_hr[r];
    u32x4 v[8];
    if (slot >= 0 && hr >= 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = 16 * (4 * j + i);
        v[2 * i] = *reinterpret_cast<const u32x4*>(a.hp + (int64_t)hr * D + col);
        v[2 * i + 1] = *reinterpret_cast<const u32x4*>(a.hp + (int64_t)hr * D + col + 8);
      }
    } else if (slot >= 0) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(a.codes + slot * (D / 4) + 16 * j);
      f32x2 pr[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) pr[g] = *reinterpret_cast<const f32x2*>(a.params + slot * 2 * NG + 2 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x2 p = pr[(4 * j + i) / 8];
        float f[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) f[e] = (float((w[i] >> (2 * e)) & 3u) - p.y) * p.x;
        v[2 * i] = u32x4{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])};
        v[2 * i + 1] =
            u32x4{pack_bf16(f[8], f[9]), pack_bf16(f[10], f[11]), pack_bf16(f[12], f[13]), pack_bf16(f[14], f[15])};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = 16 * (4 * j + i);
      *reinterpret_cast<u32x4*>(s_x + r * STR + 2 * col) = v[2 * i];
      *reinterpret_cast<u32x4*>(s_x + r * STR + 2 * col + 16) = v[2 * i + 1];
    }
  }
  // ---- rope columns -------------------------------------------------------------------
  for (int c = tid; c < kAsmRotRows * (a.R / 8); c += NT) {
    const int r = c / (a.R / 8), ch = c % (a.R / 8);
    const int64_t slot = s_slot[r];
    if (slot >= 0)
      *reinterpret_cast<u32x4*>(a.out + (row0 + r) * a.out_st + D + 8 * ch) =
          *reinterpret_cast<const u32x4*>(a.rope + slot * a.R + 8 * ch);
  }
  __syncthreads();

  // ---- out[row, c0 + col] = sum_k X[row, k] R_eff[c0 + col, k] --------------------------
  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // The B operands of K-step ks + 1 are read from LDS while the MFMAs of step
  // ks run (two register sets); one step per scheduling region, so the reads
  // stay a whole step ahead of their use.
  const uint8_t* xb = s_x + la * STR + 16 * gq;
  u32x4 xv[2][NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) xv[0][nb] = *reinterpret_cast<const u32x4*>(xb + 16 * nb * STR);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int cur = ks & 1;
    u32x4 ra[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) ra[mb] = relayout(rr[cur][mb]);
    if (ks + 1 < KS) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) rr[cur ^ 1][mb] = gload<u32x4>(rbase + 16 * mb * D + 32 * (ks + 1));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        xv[cur ^ 1][nb] = *reinterpret_cast<const u32x4*>(xb + 16 * nb * STR + 64 * (ks + 1));
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma16x16x32(ra[mb], xv[cur][nb], acc[mb][nb]);
    __builtin_amdgcn_sched_barrier(0);
  }
  // lane (la, gq) holds columns c0 + 16 mb + 4 gq + (0..3) of row 16 nb + la
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
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
  if (a.rot) {
    const dim3 grid((unsigned)((a.n + kAsmRotRows - 1) / kAsmRotRows)), block(64 * kAsmRotWaves);
#define ROLAQ_ASM_ROT(DD)                                                                                 \
    if (D == DD) {                                                                                        \
      const hipError_t e = hipFuncSetAttribute((const void*)assemble_rot_kernel<DD>,                      \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, AsmRotGeo<DD>::LDS); \
      if (e != hipSuccess) return e;                                                                      \
      hipLaunchKernelGGL((assemble_rot_kernel<DD>), grid, block, AsmRotGeo<DD>::LDS, stream, a);          \
      return hipGetLastError();                                                                           \
    }
    ROLAQ_ASM_ROT(512)
    ROLAQ_ASM_ROT(256)
#undef ROLAQ_ASM_ROT
    return hipErrorInvalidValue;
  }
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
