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
// and keeps that slice of R_eff^T in LDS for its lifetime; its 8 waves (two per
// SIMD, so one wave's epilogue overlaps the other's MFMAs) each take 64-row
// tiles of a stripe of rows. Per tile a wave computes C^T[col, row] with MFMA
// 16x16x32 (M = 16 columns, N = 16 rows, K = 32) from LDS (R) and latent rows
// loaded straight into registers a few K-steps ahead; the LDS rows are
// permuted so that each lane ends up with whole packed words of one row.
#include "rolaq_common.h"
#include "rolaq_args.h"

#include <cstddef>
#include <type_traits>

namespace rolaq {

constexpr int kWriterWaves = 8;   // waves per block: two per SIMD, so one's epilogue overlaps the other's MFMAs
constexpr int kWriterRows = 64;   // latent rows per wave tile
constexpr int kWriterDepth = 2;   // K-steps of latent loads in flight per wave (divides D / 32)
constexpr int kBufferFlags = 0x00020000;  // buffer descriptor word 3 for gfx9 raw buffers

// Column (within group g) held by row m of the block's LDS copy of R_g^T.
// Output block mb of a tile gives lane (la, gq) the rows 4 gq + i (i = 0..3)
// of that block; mapping them to columns 32 gq + 16 (mb / 4) + 4 (mb % 4) + i
// hands every lane two whole packed words (words 2 gq, 2 gq + 1 of the group)
// and 32 consecutive columns, so packing and stores need no lane exchange.
__host__ __device__ constexpr int writer_col(int m) {
  return 32 * ((m & 15) >> 2) + 16 * ((m >> 4) >> 2) + 4 * ((m >> 4) & 3) + (m & 3);
}

// Sum over the lanes l, l ^ 16, l ^ 32, l ^ 48 (same la, all gq) with the
// gfx950 row-swap permutes: VALU only, no LDS round trip.
__device__ __forceinline__ float sum_over_rows(float v) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the four lanes 4r..4r+3 (DPP quad permutes); every lane of the
// quad gets the same bits, (v0 + v1) + (v2 + v3) up to commutation.
__device__ __forceinline__ float sum_over_quad(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));  // [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));  // [2,3,0,1]
  return v;
}

// Sum of squares of eight bf16 values, FP32.
__device__ __forceinline__ float sumsq8(u32x4 v) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s = fmaf(bf16_lo(v[i]), bf16_lo(v[i]), s);
    s = fmaf(bf16_hi(v[i]), bf16_hi(v[i]), s);
  }
  return s;
}

// kv_a_layernorm of eight bf16 values with the row's inverse RMS r and the
// weights gm: bf16(gamma * bf16(x * r)), each rounding to nearest even -- the
// cast order of DeepseekV2RMSNorm.forward (transformers
// models/deepseek_v2/modeling_deepseek_v2.py:166-171). The product of two
// bf16 values is exact in FP32, so the last step rounds once.
__device__ __forceinline__ u32x4 rms_apply8(u32x4 v, float r, u32x4 gm) {
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t h = pack_bf16(bf16_lo(v[i]) * r, bf16_hi(v[i]) * r);
    o[i] = pack_bf16(bf16_lo(h) * bf16_lo(gm[i]), bf16_hi(h) * bf16_hi(gm[i]));
  }
  return o;
}


// 2 w + (this lane's bit of the lane mask m): one add with carry-in.
__device__ __forceinline__ uint32_t twice_plus_bit(uint32_t w, uint64_t m) {
  uint32_t r;
  uint64_t carry_out;
  asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(r), "=s"(carry_out) : "v"(w), "s"(m));
  return r;
}

// A field of the kernel's WriterArgs argument, loaded from the kernel argument
// segment where it is used. This relies on WriterArgs being writer_kernel's only
// explicit argument (so it sits at offset 0 of the segment) with the host's
// layout: both are checked at compile time (here and after writer_kernel).
static_assert(std::is_standard_layout<WriterArgs>::value && std::is_trivially_copyable<WriterArgs>::value,
              "kernarg_field reads WriterArgs fields by offsetof");
template <typename T>
__device__ __forceinline__ T kernarg_field(size_t off) {
  const auto k = (const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr();
  T v = *(const __attribute__((address_space(4))) T*)(k + off);
  asm volatile("" : "+s"(v));  // not merged with the argument's first load
  return v;
}

template <int D>
struct WriterGeo {
  static constexpr int NG = D / 128;
  static constexpr int KS = D / 32;            // MFMA K-steps
  static constexpr int STRIDE = 2 * D + 16;    // bytes per LDS row (padded)
  static constexpr int LDS_BYTES = 128 * STRIDE;
  static constexpr int LDS_NORM_BYTES = LDS_BYTES + 2 * D;  // + the norm weight
};

// Block = one quantization group g x a stripe of 64-row tiles. The block's
// R_g^T slice stays in LDS; its eight waves each own whole tiles and never
// synchronise after staging. Blocks of the NG groups of one stripe get the same
// blockIdx % 8, i.e. the same XCD, so each latent row is fetched from HBM once
// and served to the other groups from that XCD's L2.
//
// NORM: the rows are kv_a_layernorm inputs. Before a tile's K loop the wave
// reads the tile's rows once more for their sums of squares (the four lanes
// of a row each sum 8 columns per K-step, then a quad sum), and every K-step
// chunk is normalized in registers before it becomes an MFMA operand; each
// group's block also stores a quarter (1/NG) of the normalized rows' columns to y.
template <int D, bool NORM>
__global__ __launch_bounds__(64 * kWriterWaves, 1) void writer_kernel(WriterArgs a) {
  using G = WriterGeo<D>;
  constexpr int NG = G::NG, KS = G::KS, STR = G::STRIDE;
  extern __shared__ __attribute__((aligned(16))) uint8_t s_rt[];

  const int w = blockIdx.x;
  int g, stripe;
  if (a.nstripes % 8 == 0) {
    g = (w / 8) % NG;
    stripe = (w % 8) + 8 * (w / (8 * NG));
  } else {
    g = w % NG;
    stripe = w / NG;
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gq = lane >> 4, la = lane & 15;

  // ---- stage the permuted rows of R_eff^T for group g ------------------------
  {
    constexpr int CPR = 2 * D / 16;  // 16-byte chunks per row
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.rt);
#pragma unroll 8
    for (int c = tid; c < 128 * CPR; c += 64 * kWriterWaves) {
      const int m = c / CPR, off = (c % CPR) * 16;
      const int64_t col = 128 * g + writer_col(m);
      *reinterpret_cast<u32x4*>(s_rt + m * STR + off) =
          *reinterpret_cast<const u32x4*>(src + col * (2 * D) + off);
    }
  }
  uint8_t* s_gamma = s_rt + G::LDS_BYTES;
  if constexpr (NORM) {
    for (int c = tid; c < D / 8; c += 64 * kWriterWaves)
      *reinterpret_cast<u32x4*>(s_gamma + 16 * c) = *reinterpret_cast<const u32x4*>(a.gamma + 8 * c);
  }
  __syncthreads();

  const int64_t ntiles = (a.n + kWriterRows - 1) / kWriterRows;
  const int64_t tstep = (int64_t)a.nstripes * kWriterWaves;
  const uint8_t* lds_a = s_rt + la * STR + 16 * gq;

  // Latent rows go into registers kWriterDepth K-steps ahead; the ring runs
  // on across tiles, so the next tile's first steps are in flight while this
  // tile's epilogue runs. The loads are coalesced -- lanes 4r..4r+3 read the
  // 64 contiguous bytes of row r for one K-step -- and each K-step's data is
  // moved to the MFMA lane layout (lane la + 16 gq <- lane 4 la + gq) with
  // ds_bpermute. (Loading the MFMA layout directly makes every 16-lane pass of
  // a load touch 16 rows, which leaves the texture path four times busier.)
  // They are buffer loads over the tile's rows: one per-lane offset for the
  // whole kernel, the row block and K-step in the scalar and immediate
  // offsets, rows at or past n read as zeros.
  const int xrow = (int)a.xs * 2;                          // bytes per latent row
  const int voff = (lane >> 2) * xrow + 16 * (lane & 3);
  const int perm = 4 * (4 * la + gq);                      // ds_bpermute source address
  auto tile_rsrc = [&](int64_t t0) {
    const int64_t rows = min((int64_t)kWriterRows, a.n - t0 * kWriterRows);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.x) + t0 * kWriterRows * a.xs, (short)0,
                                             (int)(rows > 0 ? rows * xrow : 0), kBufferFlags);
  };
  auto xload = [&](__amdgpu_buffer_rsrc_t rs, int nb, int k) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 64 * k, nb * 16 * xrow, 0));
  };
  auto relayout = [&](u32x4 v) {
    return u32x4{(uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v.x),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v.y),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v.z),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v.w)};
  };
  // normalized rows go out in the K-steps ks with ks % NG == g of each group's
  // block (the stores shared out, so no block's loads wait behind all of
  // them), lanes 4r..4r+3 storing the 64 contiguous bytes of row r of one
  // K-step (the load pattern)
  const bool ystore = NORM && a.y != nullptr;
  const int yrow = (int)a.ys * 2;
  const int yoff = (lane >> 2) * yrow + 16 * (lane & 3);
  u32x4 xb[kWriterDepth][4];
  int64_t t = (int64_t)stripe * kWriterWaves + wave;
  {
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(t);
#pragma unroll
    for (int d = 0; d < kWriterDepth; ++d)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) xb[d][nb] = xload(rs, nb, d);
  }
  // low dwords of the int64 row metadata (sequence lengths and positions are
  // below 2^31 tokens; request indices are checked to fit, -1 stays -1)
  const int32_t* seq32 = reinterpret_cast<const int32_t*>(a.seq_lens);
  // decode rows (no positions) sit at seq_len - 1: read seq_lens there instead
  const int32_t* pos32 = reinterpret_cast<const int32_t*>(a.positions ? a.positions : a.seq_lens);
  const int32_t pos_adj = a.positions ? 0 : -1;
  const int32_t* req32 = reinterpret_cast<const int32_t*>(a.req_idx);

  for (; t < ntiles; t += tstep) {
    const int64_t row0 = t * kWriterRows;
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(t), rn = tile_rsrc(t + tstep);

    // ---- NORM: inverse RMS of rows 16 nb + lane / 4 (rows past n read as 0) -----
    float rinv[4];
    __amdgpu_buffer_rsrc_t ys_rsrc;
    if constexpr (NORM) {
      if (ystore) {
        const int64_t rows = min((int64_t)kWriterRows, a.n - row0);
        ys_rsrc = __builtin_amdgcn_make_buffer_rsrc(a.y + row0 * a.ys, (short)0, (int)(rows * yrow), kBufferFlags);
      }
    }
    if constexpr (NORM) {
      float ss[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = 0; k0 < KS; k0 += 2) {
        u32x4 v[2][4];
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) v[k][nb] = xload(rs, nb, k0 + k);
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) ss[nb] += sumsq8(v[k][nb]);
      }
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        rinv[nb] = 1.0f / sqrtf(sum_over_quad(ss[nb]) * (1.0f / D) + a.eps);
    }

    // ---- C^T tile: 128 columns x 64 rows on MFMA 16x16x32 ----------------------
    f32x4 acc[8][4];
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // K-step k's latent slice (normalized under NORM) is moved to the MFMA
    // layout by stage(k), which then reuses its ring slot for the load
    // kWriterDepth steps further on. Under NORM the K loop is software
    // pipelined: stage(k) and the first half of step k's R_g rows are issued
    // between the two halves of step k - 1's MFMAs, the second half of its
    // R_g rows before its own first half.
    u32x4 xv[2][4], av[2][8];
    auto stage = [&](int k) {
      const int s = k % kWriterDepth;
      if constexpr (NORM) {
        const u32x4 gm = *reinterpret_cast<const u32x4*>(s_gamma + 64 * k + 16 * (lane & 3));
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          xb[s][nb] = rms_apply8(xb[s][nb], rinv[nb], gm);
          if (ystore && k % NG == g)  // rows at or past n fall outside the buffer and are dropped
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) uint32_t,
                                                                      xb[s][nb]),
                                                   ys_rsrc, yoff + 64 * k, nb * 16 * yrow, 0);
        }
      }
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) xv[k % 2][nb] = relayout(xb[s][nb]);
      const int kk = k + kWriterDepth;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) xb[s][nb] = kk < KS ? xload(rs, nb, kk) : xload(rn, nb, kk - KS);
    };
    auto rread = [&](int k, int m0) {
#pragma unroll
      for (int mb = m0; mb < m0 + 4; ++mb)
        av[k % 2][mb] = *reinterpret_cast<const u32x4*>(lds_a + 16 * mb * STR + 64 * k);
    };
    if constexpr (NORM) {
      stage(0);
      rread(0, 0);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int c = ks % 2;
        rread(ks, 4);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mfma16x16x32(av[c][mb], xv[c][nb], acc[mb][nb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x080, 1, 0);  // an LDS read
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // four MFMAs
        }
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 1 < KS) {
          stage(ks + 1);
          rread(ks + 1, 0);
        }
#pragma unroll
        for (int mb = 4; mb < 8; ++mb)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mfma16x16x32(av[c][mb], xv[c][nb], acc[mb][nb]);
        if (ks + 1 < KS) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x080, 1, 0);  // a relayout permute or LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // without the norm the staged operands' registers are worth more than
      // the overlap (measured): one K-step per scheduling region
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int c = ks % 2;
        rread(ks, 0);
        rread(ks, 4);
        stage(ks);
#pragma unroll
        for (int mb = 0; mb < 8; ++mb)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mfma16x16x32(av[c][mb], xv[c][nb], acc[mb][nb]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // ---- epilogue: lane (la, gq) holds columns 32gq..32gq+31 of row 16nb+la ---
    // The lane's row within the tile, recomputed here: kept from the kernel's
    // start, the compiler spills it, and every reload waits for all loads in
    // flight (the next tile's latent rows among them).
    int lane_now;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_now));
    const int lr = lane_now & 15, gr = lane_now >> 4;
    // the code thresholds -t, 0, t as midpoints (FP64) and tie rules
    const float thr = a.thr;
    const double mu_lo = below_midpoint(-thr), mu_hi = below_midpoint(thr), mu_zero = below_midpoint(0.0f);
    const bool incl_lo = threshold_inclusive(-thr), incl_hi = threshold_inclusive(thr);
    int64_t slot[4];
    int32_t seq[4], pos[4], req[4];
    u32x2 pes[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int64_t r = min(row0 + 16 * nb + lr, a.n - 1);
      pes[nb] = a.pe_vec ? *reinterpret_cast<const u32x2*>(a.k_pe + r * a.pe_s0 + 16 * g + 4 * gr) : u32x2{0u, 0u};

      slot[nb] = a.loc[r];
      seq[nb] = seq32[2 * r];
      pos[nb] = pos32[2 * r] + pos_adj;
      // a request index that does not fit 32 bits is outside [0, max_reqs):
      // no ring row (its high dword is not the sign extension of the low one)
      const int32_t rlo = req32[2 * r], rhi = req32[2 * r + 1];
      req[nb] = rhi == (rlo >> 31) ? rlo : -1;
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      __builtin_amdgcn_sched_barrier(0);
      const int64_t row = row0 + 16 * nb + lr;
      // rope columns [16 g, 16 g + 16) of the row, four per lane
      const u32x2 pe = pes[nb];
      const bool live = row < a.n;
      const int64_t sl = slot[nb];
      // window bookkeeping (mla_fused_writer.py:36-51)
      const int32_t p = pos[nb], sq = seq[nb], rq = req[nb];
      const bool keep = live && ((p < a.P) || (p >= sq - a.W)) && rq < a.max_reqs && rq >= 0 && sl > 0;
      const int32_t inner = p < a.P ? p : a.P + (p - a.P > 0 ? p - a.P : 0) % (a.W > 0 ? a.W : 1);
      const int64_t ring = 1 + (int64_t)rq * (a.P + a.W) + inner;
      if (keep) {
        // bf16 of the rotated FP32 row (columns 32gq..32gq+31 of group g)
        uint16_t* hrow = a.hp + ring * D + 128 * g + 32 * gq;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const f32x4 u = acc[2 * h][nb], v = acc[2 * h + 1][nb];
          const u32x4 pk = {pack_bf16(u[0], u[1]), pack_bf16(u[2], u[3]), pack_bf16(v[0], v[1]),
                            pack_bf16(v[2], v[3])};
          *reinterpret_cast<u32x4*>(hrow + 8 * h) = pk;
        }
      }
      // Lloyd statistics over the row's 128 group columns (4 lanes)
      float s = 0.f;
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) s += (acc[mb][nb][0] + acc[mb][nb][1]) + (acc[mb][nb][2] + acc[mb][nb][3]);
      s = sum_over_rows(s);
      const float mean = s * (1.0f / 128.0f);
      float q = 0.f;
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[mb][nb][i] -= mean;
          q = fmaf(acc[mb][nb][i], acc[mb][nb][i], q);
        }
      q = sum_over_rows(q);
      const float std_ = sqrtf(q * (1.0f / 128.0f) + 1e-08f);
      // code = #{-t, 0, t <= normalized}, normalized = (x - mean) / std, the
      // correctly rounded FP32 quotient (oscar.py:135-140): compared through
      // the row's exact thresholds on y = x - mean (no division per element).
      // Its two bits: high = (y >= y0), low = the parity of the three tests.
      const double sd = (double)std_;
      const float ylo = y_threshold(sd, mu_lo, incl_lo), y0 = y_threshold(sd, mu_zero, true),
                  yhi = y_threshold(sd, mu_hi, incl_hi);
      uint32_t word[2] = {0u, 0u};
#pragma unroll
      for (int wi = 0; wi < 2; ++wi)
#pragma unroll
        for (int e = 15; e >= 0; --e) {  // Horner, element e at bits 2e, 2e + 1
          const float y = acc[4 * wi + e / 4][nb][e % 4];
          const uint64_t hi = __builtin_amdgcn_ballot_w64(y >= y0);
          const uint64_t lo = __builtin_amdgcn_ballot_w64(y >= ylo) ^ hi ^ __builtin_amdgcn_ballot_w64(y >= yhi);
          word[wi] = twice_plus_bit(twice_plus_bit(word[wi], hi), lo);
        }
      if (live) {
        // words 2gq, 2gq+1 of group g: row words 8g + 2gq, 8g + 2gq + 1
        *reinterpret_cast<u32x2*>(a.codes + sl * (D / 4) + 4 * (8 * g + 2 * gq)) = u32x2{word[0], word[1]};
        if (gq == 0) {
          const float scale = a.kscale * std_;
          const float zero = kZeroOffset - mean / scale;
          *reinterpret_cast<f32x2*>(a.params + sl * 2 * NG + 2 * g) = f32x2{scale, zero};
        }
        if (sl > 0) {
          if (a.pe_vec) {
            // the rope pool's base read again from the kernel arguments here
            // (a scalar load), not held in a register that would be spilled
            // (as a global pointer: through a generic one the store is a flat
            // store, which the next LDS waits would also wait for)
            typedef __attribute__((address_space(1))) u32x2 g_u32x2;
            uint16_t* const rope = kernarg_field<uint16_t*>(offsetof(WriterArgs, rope));
            *(g_u32x2*)(rope + sl * a.R + 16 * g + 4 * gr) = pe;
          } else if (g == 0) {
            for (int r = gq; r < a.R; r += 4) a.rope[sl * a.R + r] = a.k_pe[row * a.pe_s0 + r * a.pe_s1];
          }
          if (g == 0 && gq == 0) {
            a.row_of_slot[sl] = keep ? int32_t(ring) : -1;
            if (keep) a.owner_of_row[ring] = int32_t(sl);
          }
        }
      }
    }
  }
}

// kernarg_field: WriterArgs must stay writer_kernel's one explicit argument
static_assert(std::is_same<decltype(&writer_kernel<512, false>), void (*)(WriterArgs)>::value &&
                  std::is_same<decltype(&writer_kernel<256, true>), void (*)(WriterArgs)>::value,
              "writer_kernel's only argument must be WriterArgs (read at kernel-argument offset 0)");

}  // namespace rolaq

hipError_t rolaq_launch_writer(const rolaq::WriterArgs& args_in, int D, int num_cus, hipStream_t stream) {
  using namespace rolaq;
  WriterArgs a = args_in;
  const int NG = D / 128;
  const int64_t ntiles = (a.n + kWriterRows - 1) / kWriterRows;
  const int64_t need = (ntiles + kWriterWaves - 1) / kWriterWaves;  // stripes with work for every wave
  // one block per CU (the R_g slice fills most of the LDS), in multiples of 8 when large
  int64_t stripes = (num_cus + NG - 1) / NG;
  if (stripes >= 8) stripes = (stripes / 8) * 8;
  if (stripes > need) stripes = need;
  if (stripes < 1) stripes = 1;
  a.nstripes = (int)stripes;
  // rope copy as 8-byte pieces: 16 columns per group, 8-byte aligned rows
  a.pe_vec = a.pe_s1 == 1 && a.R == 16 * NG && (a.pe_s0 % 4) == 0 &&
             (reinterpret_cast<uintptr_t>(a.k_pe) % 8) == 0 && (reinterpret_cast<uintptr_t>(a.rope) % 8) == 0;
  const dim3 grid((unsigned)(stripes * NG)), block(64 * kWriterWaves);
#define ROLAQ_WRITER(DD, NORM, LDS)                                                                         \
  if (D == DD && (a.gamma != nullptr) == NORM) {                                                           \
    const int lds = WriterGeo<DD>::LDS;                                                                    \
    const hipError_t e = hipFuncSetAttribute((const void*)writer_kernel<DD, NORM>,                         \
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds);             \
    if (e != hipSuccess) return e;                                                                         \
    hipLaunchKernelGGL((writer_kernel<DD, NORM>), grid, block, lds, stream, a);                            \
    return hipGetLastError();                                                                              \
  }
  ROLAQ_WRITER(512, false, LDS_BYTES)
  ROLAQ_WRITER(256, false, LDS_BYTES)
  ROLAQ_WRITER(512, true, LDS_NORM_BYTES)
  ROLAQ_WRITER(256, true, LDS_NORM_BYTES)
#undef ROLAQ_WRITER
  return hipErrorInvalidValue;
}
