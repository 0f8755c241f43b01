// Fused RoLaQ cache writer (gfx950): rotate -> Lloyd INT2 quantize -> pack,
// plus the rope / BF16-window / ownership stores.
//
// Reference behaviour: try_fast_decode_store -> FP32 GEMM x @ R_eff and
// _pack_and_aux (deployment/sglang/QuantKernel/mla_fused_writer.py:16-51,
// 54-107, 110-224); codec mla_quant/oscar.py:130-144.
//
// Both GEMM operands are exactly representable in bf16 (the latent is bf16 and
// R_eff = fp32(bf16(R))), so bf16 MFMA with FP32 accumulation forms the same
// products as the reference's FP32 GEMM; only the summation order differs.
//
// Decomposition: a block owns one quantization group g (128 output columns)
// and keeps that slice of R_eff^T in LDS for its lifetime; its 4 waves each
// take 64-row tiles of a stripe of rows. Blocks of the NG groups of one stripe
// are numbered so that they land on the same XCD and read the same latent rows
// through one L2. Per tile a wave computes C^T[col, row] with MFMA 16x16x32
// (M = 16 columns, N = 16 rows, K = 32), so each lane ends up with 32 values of
// one row: row statistics need a 4-lane reduction and the codes of a packed
// word come from 4 lanes.
#include "rolaq_common.h"
#include "rolaq_args.h"

namespace rolaq {


template <int D>
__global__ __launch_bounds__(256, 1) void writer_kernel(WriterArgs a) {
  constexpr int NG = D / 128;
  constexpr int KS = D / 32;              // K-steps
  constexpr int LDS_STRIDE = 2 * D + 16;  // bytes per LDS column (padded)
  constexpr int WROWS = 64;               // rows per wave tile
  extern __shared__ __attribute__((aligned(16))) uint8_t s_rt[];

  // block -> (group, stripe); blocks of one stripe share w % 8 (same XCD)
  const int w = blockIdx.x;
  int g, stripe;
  if (a.nstripes % 8 == 0) {
    g = (w / 8) % NG;
    stripe = (w % 8) + 8 * (w / (8 * NG));
  } else {
    g = w % NG;
    stripe = w / NG;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int gq = lane >> 4, la = lane & 15;

  // ---- stage R_eff^T rows [128g, 128g + 128) into LDS ------------------------
  {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.rt + (int64_t)(128 * g) * D);
    constexpr int CHUNKS = 128 * D * 2 / 16;
    for (int c = tid; c < CHUNKS; c += 256) {
      const int col = c / (D * 2 / 16), off = (c % (D * 2 / 16)) * 16;
      *reinterpret_cast<u32x4*>(s_rt + col * LDS_STRIDE + off) =
          *reinterpret_cast<const u32x4*>(src + (int64_t)col * D * 2 + off);
    }
  }
  __syncthreads();

  const int64_t nrb = (a.n + 4 * WROWS - 1) / (4 * WROWS);
  for (int64_t rb = stripe; rb < nrb; rb += a.nstripes) {
    const int64_t row0 = rb * 4 * WROWS + wave * WROWS;
    if (row0 >= a.n) continue;
    f32x4 acc[8][4];
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint16_t* xr[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int64_t r = min(row0 + 16 * nb + la, a.n - 1);
      xr[nb] = a.x + r * a.xs + 8 * gq;
    }
    u32x4 bcur[4], bnext[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) bcur[nb] = *reinterpret_cast<const u32x4*>(xr[nb]);
#pragma unroll 2
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) bnext[nb] = *reinterpret_cast<const u32x4*>(xr[nb] + 32 * (ks + 1));
      }
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const u32x4 av = *reinterpret_cast<const u32x4*>(s_rt + (16 * mb + la) * LDS_STRIDE + (32 * ks + 8 * gq) * 2);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mfma16x16x32(av, bcur[nb], acc[mb][nb]);
      }
      if (ks + 1 < KS) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) bcur[nb] = bnext[nb];
      }
    }

    // ---- epilogue: one row per lane per N-block ------------------------------
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int64_t row = row0 + 16 * nb + la;
      const bool live = row < a.n;
      // acc[mb][nb][j]: column 16mb + 4gq + j of group g for this row
      float s = 0.f;
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) s += acc[mb][nb][j];
      s = wave_sum_over_groups(s);
      const float mean = s * (1.0f / 128.0f);
      float q = 0.f;
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float d = acc[mb][nb][j] - mean;
          q = fmaf(d, d, q);
        }
      q = wave_sum_over_groups(q);
      const float std_ = sqrtf(q * (1.0f / 128.0f) + 1e-08f);
      const float inv = 1.0f / std_;
      // byte gq of word mb: codes of columns 16mb + 4gq + j at bits 2j
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        uint32_t byte = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float nrm = (acc[mb][nb][j] - mean) * inv;
          const uint32_t c = uint32_t(nrm >= -a.thr) + uint32_t(nrm >= 0.f) + uint32_t(nrm >= a.thr);
          byte |= c << (2 * j);
        }
        if (mb < 4) lo |= byte << (8 * mb); else hi |= byte << (8 * (mb - 4));
      }
      // lane gq assembles words 2gq, 2gq+1 from the four lanes of this row
      const uint32_t mine = gq < 2 ? lo : hi;  // dword holding words 2gq, 2gq+1 bytes
      uint32_t src[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo_k = __shfl(lo, la + 16 * k);
        const uint32_t hi_k = __shfl(hi, la + 16 * k);
        src[k] = gq < 2 ? lo_k : hi_k;
      }
      (void)mine;
      const int bsel0 = (2 * gq) % 4, bsel1 = (2 * gq + 1) % 4;
      uint32_t w0 = 0, w1 = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        w0 |= ((src[k] >> (8 * bsel0)) & 0xffu) << (8 * k);
        w1 |= ((src[k] >> (8 * bsel1)) & 0xffu) << (8 * k);
      }
      const int64_t slot = live ? a.loc[row] : 0;
      if (live) {
        uint8_t* crow = a.codes + slot * (D / 4);
        *reinterpret_cast<uint32_t*>(crow + 4 * (NG * (2 * gq) + g)) = w0;
        *reinterpret_cast<uint32_t*>(crow + 4 * (NG * (2 * gq + 1) + g)) = w1;
        if (gq == 0) {
          const float scale = a.kscale * std_;
          const float zero = kZeroOffset - mean / scale;
          *reinterpret_cast<f32x2*>(a.params + slot * 2 * NG + 2 * g) = f32x2{scale, zero};
        }
        // window bookkeeping (mla_fused_writer.py:36-51)
        const int64_t seq = a.seq_lens[row];
        const int64_t pos = a.positions ? a.positions[row] : seq - 1;
        const int64_t req = a.req_idx[row];
        const bool keep = ((pos < a.P) || (pos >= seq - a.W)) && req < a.max_reqs && req >= 0 && slot > 0;
        const int64_t inner = pos < a.P ? pos : a.P + (pos - a.P > 0 ? pos - a.P : 0) % (a.W > 0 ? a.W : 1);
        const int64_t ring = 1 + req * (a.P + a.W) + inner;
        if (keep) {
          uint16_t* hrow = a.hp + ring * D + 128 * g;
#pragma unroll
          for (int mb = 0; mb < 8; ++mb) {
            const u32x2 v = {pack_bf16(acc[mb][nb][0], acc[mb][nb][1]), pack_bf16(acc[mb][nb][2], acc[mb][nb][3])};
            *reinterpret_cast<u32x2*>(hrow + 16 * mb + 4 * gq) = v;
          }
        }
        if (g == 0 && slot > 0) {
          for (int r = gq; r < a.R; r += 4)
            a.rope[slot * a.R + r] = a.k_pe[row * a.pe_s0 + r * a.pe_s1];
          if (gq == 0) {
            a.row_of_slot[slot] = keep ? int32_t(ring) : -1;
            if (keep) a.owner_of_row[ring] = int32_t(slot);
          }
        }
      }
    }
  }
}

}  // namespace rolaq

hipError_t rolaq_launch_writer(const rolaq::WriterArgs& args_in, int D, int num_cus, hipStream_t stream) {
  using namespace rolaq;
  WriterArgs a = args_in;
  const int NG = D / 128;
  const int64_t nrb = (a.n + 255) / 256;
  // enough stripes to give every CU one block, in multiples of 8 when large
  int64_t stripes = (num_cus + NG - 1) / NG;
  if (stripes >= 8) stripes = (stripes / 8) * 8;
  if (stripes > nrb) stripes = nrb;
  if (stripes < 1) stripes = 1;
  a.nstripes = (int)stripes;
  const dim3 grid((unsigned)(stripes * NG)), block(256);
  const size_t lds = (size_t)128 * (2 * D + 16);
  if (D == 512) {
    const hipError_t e = hipFuncSetAttribute((const void*)writer_kernel<512>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((writer_kernel<512>), grid, block, lds, stream, a);
  } else if (D == 256) {
    const hipError_t e = hipFuncSetAttribute((const void*)writer_kernel<256>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((writer_kernel<256>), grid, block, lds, stream, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
