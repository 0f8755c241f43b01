// Absorbed MLA decode attention over the packed INT2 cache (gfx950).
//
// Reference behaviour: packed_mla_decode_gf_fwd + _fwd_hp_window_stage1 +
// stage-2 merge of the OSCAR SGLang fork (call site
// deployment/patches/rolaq_sglang.patch:51-111); arithmetic of
// mla_quant/cache.py:1007-1073 + eager MLA attention.
//
// Work split: grid (B, max_splits + 1). Block (b, s) with s < nq = max(ns_b - 1, 1)
// handles a contiguous range of 32-token tiles of the INT2 positions
// [P, L_b - W); block s == nq handles the <= P + W BF16 window rows; larger s
// exit. A second kernel merges the nq + 1 partials by LSE.
//
// INT2 split, per wave (4 waves per block, tiles interleaved across waves):
//   scores  S^T[t, h] = sum_g scale_tg (sum_j q'_hj v_tj - 4 Q'_hg) - scale_tg zero_tg Qsum_hg
//           on bf16 MFMA 16x16x32 with M = 16 tokens, N = 16 heads, K = latent.
//           v_tj = 4 + c_tj 2^(e-5) is the code masked into a bf16 mantissa and
//           q'_hj = q_hj 2^(5-e) the matching exact rescale of the query.
//   output  O[h, f] += sum_t p'_g[h,t] v_t[f] with p'_g = p * scale_tg, M = heads,
//           N = 16 features, K = 32 tokens. The A operand is the softmax tile in
//           the score accumulator's own lane layout; the B operand is built by a
//           byte perm of two tokens' code words plus the same mantissa trick.
//           p'_g enters as a bf16 hi + lo pair (two MFMAs), so the output is
//           FP32-accurate. A ones-column MFMA accumulates SP_g = sum_t p'_g exactly
//           as the output MFMA sees it, so o = (O - 4 SP_g) 2^(5-e) - sum_t p'_g zero_tg.
#include <type_traits>

#include "rolaq_common.h"
#include "rolaq_args.h"

namespace rolaq {


struct SeqCtx {
  const int32_t* idx;
  int L;
  int shift;
};

__device__ __forceinline__ int64_t slot_of(const SeqCtx& c, int pos) {
  pos = min(max(pos, 0), c.L - 1);
  const int64_t page = c.idx[pos >> c.shift];
  return (page << c.shift) + (pos & ((1 << c.shift) - 1));
}

__device__ __forceinline__ int ring_row(int64_t req, int pos, int P, int W) {
  const int inner = pos < P ? pos : P + max(pos - P, 0) % max(W, 1);
  return int(1 + req * (P + W) + inner);
}

template <int N>
__device__ __forceinline__ void load_words(const uint8_t* p, uint32_t (&w)[N]) {
  static_assert(N % 2 == 0, "");
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p + 4 * i);
      w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      const u32x2 v = *reinterpret_cast<const u32x2*>(p + 4 * i);
      w[i] = v.x; w[i + 1] = v.y;
    }
  }
}

// ---------------------------------------------------------------------------
// Window split: attention over the BF16 sink/recent rows of one sequence.
// The <= MAXW rows (hp_c ring rows + rope) are staged into LDS with 16-byte
// loads, then thread t = (head h = t & 15 (+16 hb), chunk c = t >> 4) forms
// partial dots over D/16 latent + R/16 rope dims; waves reduce through LDS.
// Writes the normalised partial and natural-log LSE at split slot.
// ---------------------------------------------------------------------------
constexpr int kMaxWindow = 32;

template <int D, int R>
constexpr int window_rows_bytes() { return kMaxWindow * (D + R) * 2; }
constexpr int window_part_floats() { return (4 * 16 + 16) * kMaxWindow + 16; }

template <int D, int R, int NHB>
__device__ void window_split(const DecodeArgs& a, int b, int h0, int slot_split, const SeqCtx& sc,
                             int64_t req, float* smem, uint8_t* rows_mem) {
  constexpr int MAXW = kMaxWindow;
  constexpr int FC = D / 16, RC = R / 16;
  constexpr int ROWE = D + R;  // staged row: latent | rope (bf16 elements)
  const int t = threadIdx.x, h16 = t & 15, c = t >> 4, lane = t & 63, wave = t >> 6;
  const int L = sc.L, P = a.P, W = a.W;
  // window positions in increasing order: [0, min(P, L)) U [max(L - W, P), L)
  const int n_sink = min(P, L);
  const int rec_lo = max(L - W, n_sink);
  const int nw = n_sink + (L - rec_lo);
  uint16_t* rows = reinterpret_cast<uint16_t*>(rows_mem);             // [MAXW][ROWE]
  float* sc_part = smem;                                              // [4 waves][16][MAXW]
  float* prob = sc_part + 4 * 16 * MAXW;                              // [16][MAXW] + 16
  // stage rows: D/8 + R/8 16-byte chunks per row
  constexpr int CPR = (D + R) / 8;
  for (int k = t; k < nw * CPR; k += 256) {
    const int i = k / CPR, ch = k % CPR;
    const int pos = i < n_sink ? i : rec_lo + (i - n_sink);
    const uint16_t* src = ch < D / 8 ? a.hp + (int64_t)ring_row(req, pos, P, W) * D + 8 * ch
                                     : a.rope + slot_of(sc, pos) * R + 8 * (ch - D / 8);
    *reinterpret_cast<u32x4*>(rows + i * ROWE + 8 * ch) = *reinterpret_cast<const u32x4*>(src);
  }
  __syncthreads();
  for (int hb = 0; hb < NHB; ++hb) {
    const int h = h0 + 16 * hb + h16;
    const bool hv = h < a.H;
    const uint16_t* qh = a.q + b * a.q_sb + (int64_t)min(h, a.H - 1) * a.q_sh;
    float qv[FC], qr[RC];
#pragma unroll
    for (int i = 0; i < FC; i += 8) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qh + c * FC + i);
      qv[i] = bf16_lo(v.x); qv[i + 1] = bf16_hi(v.x); qv[i + 2] = bf16_lo(v.y); qv[i + 3] = bf16_hi(v.y);
      qv[i + 4] = bf16_lo(v.z); qv[i + 5] = bf16_hi(v.z); qv[i + 6] = bf16_lo(v.w); qv[i + 7] = bf16_hi(v.w);
    }
#pragma unroll
    for (int i = 0; i < RC; ++i) qr[i] = bf16_to_float(qh[D + c * RC + i]);
    if (!hv) {
#pragma unroll
      for (int i = 0; i < FC; ++i) qv[i] = 0.f;
#pragma unroll
      for (int i = 0; i < RC; ++i) qr[i] = 0.f;
    }
    for (int i = 0; i < nw; ++i) {
      const uint16_t* row = rows + i * ROWE;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < FC; ++k) acc = fmaf(qv[k], bf16_to_float(row[c * FC + k]), acc);
#pragma unroll
      for (int k = 0; k < RC; ++k) acc = fmaf(qr[k], bf16_to_float(row[D + c * RC + k]), acc);
      acc = wave_sum_over_groups(acc);  // chunks c, c^1, c^2, c^3 of this wave
      if (lane < 16) sc_part[(wave * 16 + h16) * MAXW + i] = acc;
    }
    __syncthreads();
    if (c == 0) {
      float m = -3.0e38f, l = 0.f;
      for (int i = 0; i < nw; ++i) {
        const float s = (sc_part[h16 * MAXW + i] + sc_part[(16 + h16) * MAXW + i] +
                         sc_part[(32 + h16) * MAXW + i] + sc_part[(48 + h16) * MAXW + i]) *
                        a.sm_scale * kLog2e;
        prob[h16 * MAXW + i] = s;
        m = fmaxf(m, s);
      }
      for (int i = 0; i < nw; ++i) {
        const float p = __builtin_amdgcn_exp2f(prob[h16 * MAXW + i] - m);
        prob[h16 * MAXW + i] = p;
        l += p;
      }
      const int64_t li = ((int64_t)b * a.H + h) * a.S1 + slot_split;
      if (hv) a.lse[li] = nw ? (m + __log2f(l)) * kLn2 : kNeutralLse;
      prob[16 * MAXW + h16] = nw ? 1.f / l : 0.f;
    }
    __syncthreads();
    const float inv = prob[16 * MAXW + h16];
    float o[FC];
#pragma unroll
    for (int k = 0; k < FC; ++k) o[k] = 0.f;
    for (int i = 0; i < nw; ++i) {
      const uint16_t* row = rows + i * ROWE;
      const float p = prob[h16 * MAXW + i];
#pragma unroll
      for (int k = 0; k < FC; ++k) o[k] = fmaf(p, bf16_to_float(row[c * FC + k]), o[k]);
    }
    if (hv) {
      float* dst = a.logits + (((int64_t)b * a.H + h) * a.S1 + slot_split) * D + c * FC;
#pragma unroll
      for (int k = 0; k < FC; k += 4) *reinterpret_cast<f32x4*>(dst + k) = f32x4{o[k] * inv, o[k + 1] * inv, o[k + 2] * inv, o[k + 3] * inv};
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Stage 1: one block per (split, sequence).
//
// Each wave walks its 32-token tiles with a one-tile software pipeline: the
// raw 16-byte chunks of tile i+1 (codes, rope, params) are loaded into
// registers while tile i is computed from the wave's LDS buffer, then written
// to that buffer. With PAGED (page size a multiple of 32) a tile occupies 32
// consecutive slots, so every lane's load offset is a per-lane constant plus
// one uniform page base.
// ---------------------------------------------------------------------------
template <int D, int R>
struct Geo {
  static constexpr int NG = D / 128;      // quantization groups
  static constexpr int KR = R / 32;       // rope K-blocks
  static constexpr int NB = D / 16;       // output N-blocks (16 features each)
  static constexpr int SW = 4 * NG;       // bytes of one superword (word s of every group)
  static constexpr int ROWB = D / 4;      // packed bytes per token
  static constexpr int PB = 8 * NG;       // param bytes per token
  static constexpr int RBYTES = 2 * R;    // rope bytes per token
  static constexpr int CCH = ROWB / 16;   // 16-byte chunks per row (8 / 4)
  static constexpr int RCH = RBYTES / 16;
  static constexpr int PCH = PB / 16;
  static constexpr int CL = 32 * CCH / 64;  // DMA loads (1 KB each) per tile
  static constexpr int RL = 32 * RCH / 64;
  static constexpr int PL = (32 * PCH + 63) / 64;
  static constexpr int OFF_R = 32 * ROWB;
  static constexpr int OFF_P = OFF_R + 32 * RBYTES;
  static constexpr int TILE_LDS = OFF_P + 64 * 16 * PL;
  // chunk c of token t sits at 16-byte slot t*CCH + (c ^ (t % CCH)): rows read
  // by 16 lanes at once then spread over the LDS banks
  __device__ static constexpr int cslot(int t, int c) { return t * CCH + (c ^ (t & (CCH - 1))); }
  __device__ static constexpr int rslot(int t, int c) { return t * RCH + (c ^ (t & (RCH - 1))); }
};

// One 16-byte direct global->LDS load per lane (global_load_lds_dwordx4). The
// LDS destination is wave-uniform: lane i lands at dst + 16 i.
__device__ __forceinline__ void lds_dma16(const uint8_t* src, uint8_t* dst) {
  typedef __attribute__((address_space(3))) void lds_t;
  __builtin_amdgcn_global_load_lds(src, (lds_t*)dst, 16, 0, 0);
}

__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t b) {
  uint32_t d;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(x), "s"(m), "v"(b));
  return d;
}

// unpack_word with one v_and_or_b32 per dword
__device__ __forceinline__ void unpack_word_fast(uint32_t w, uint32_t d[8], uint32_t base) {
  d[0] = and_or(w, 0x00030003u, base);
  d[1] = and_or(w, 0x000C000Cu, base);
  d[2] = and_or(w, 0x00300030u, base);
  const uint32_t w6 = w >> 6;
  d[3] = and_or(w6, 0x00030003u, base);
  d[4] = and_or(w6, 0x000C000Cu, base);
  d[5] = and_or(w6, 0x00300030u, base);
  const uint32_t w12 = w >> 12;
  d[6] = and_or(w12, 0x00030003u, base);
  d[7] = and_or(w12, 0x000C000Cu, base);
}

// State of one wave's INT2 split (everything the tile loop updates or reads).
template <int D, int R, int NHB>
struct WaveState {
  static constexpr int NG = D / 128, KR = R / 32, NB = D / 16;
  f32x4 O[NHB][NB];
  f32x4 SP[NHB][NG];
  float m_run[NHB], l_run[NHB], zp[NHB][NG];
  float q4[NHB][NG], qsum[NHB][NG];
  u32x4 qr[NHB][KR];
  const u32x4 (*s_qs)[4 * NG][64];
  u32x4 ones;
  uint32_t perm_sel, vbase;
  int lane, gq, la, lo, hi;
  float scale_log2;
};

// One 32-token tile from the wave's LDS buffer tl; FULL tiles lie inside [lo, hi).
template <int D, int R, int NHB, bool full>
__device__ __forceinline__ void tile_compute(WaveState<D, R, NHB>& st, int tile, const uint8_t* tl) {
  using G = Geo<D, R>;
  constexpr int NG = G::NG, KR = G::KR, NB = G::NB, SW = G::SW, PB = G::PB;
  constexpr int TILE = 32;
  auto& O = st.O;
  auto& SP = st.SP;
  auto& m_run = st.m_run;
  auto& l_run = st.l_run;
  auto& zp = st.zp;
  const auto& q4 = st.q4;
  const auto& qsum = st.qsum;
  const auto& qr = st.qr;
  const auto s_qs = st.s_qs;
  const u32x4 ones = st.ones;
  const uint32_t perm_sel = st.perm_sel, vbase = st.vbase;
  const int lane = st.lane, gq = st.gq, la = st.la, lo = st.lo, hi = st.hi;
  const float scale_log2 = st.scale_log2;
    const int p0 = tile * TILE;
    // -- scores: S^T[token, head] -----------------------------------------------
    float s[2][NHB][4];
    uint32_t cw[2][2 * NG];  // codes of token 16mb + la, superwords 2gq, 2gq+1
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int t = 16 * mb + la;
      if constexpr (NG == 4) {
        const u32x4 v0 = *reinterpret_cast<const u32x4*>(tl + 16 * G::cslot(t, 2 * gq));
        const u32x4 v1 = *reinterpret_cast<const u32x4*>(tl + 16 * G::cslot(t, 2 * gq + 1));
        cw[mb][0] = v0.x; cw[mb][1] = v0.y; cw[mb][2] = v0.z; cw[mb][3] = v0.w;
        cw[mb][4] = v1.x; cw[mb][5] = v1.y; cw[mb][6] = v1.z; cw[mb][7] = v1.w;
      } else {
        const u32x4 v0 = *reinterpret_cast<const u32x4*>(tl + 16 * G::cslot(t, gq));
        cw[mb][0] = v0.x; cw[mb][1] = v0.y; cw[mb][2] = v0.z; cw[mb][3] = v0.w;
      }
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kr = 0; kr < KR; ++kr) {
          const u32x4 ro = *reinterpret_cast<const u32x4*>(tl + G::OFF_R + 16 * G::rslot(t, 4 * kr + gq));
          acc = mfma16x16x32(ro, qr[hb][kr], acc);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) s[mb][hb][j] = acc[j];
      }
    }
    // (scale, zero) of groups 2gp, 2gp+1 for this lane's C-layout token 16mb + 4gq + j
    auto param2 = [&](int mb, int j, int gp) -> f32x4 {
      f32x4 v = *reinterpret_cast<const f32x4*>(tl + G::OFF_P + (16 * mb + 4 * gq + j) * PB + 16 * gp);
      if constexpr (!full) {
        // masked positions may hold rows that were never written: use 0
        const int pos = p0 + 16 * mb + 4 * gq + j;
        if (pos < lo || pos >= hi) v = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      return v;
    };
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      // a compiler-level fence per group: the loads below are not merged with
      // (or hoisted above) those of other groups, which bounds register use
      asm volatile("" ::: "memory");
      f32x4 pv[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) pv[mb][j] = param2(mb, j, g / 2);
      float scl[2][4], szr[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float sv = (g & 1) ? pv[mb][j].z : pv[mb][j].x;
          const float zv = (g & 1) ? pv[mb][j].w : pv[mb][j].y;
          scl[mb][j] = sv;
          szr[mb][j] = sv * zv;
        }
      u32x4 kop[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        uint32_t d0[8], d1[8];
        unpack_word_fast(cw[mb][g], d0, vbase);        // superword 2gq
        unpack_word_fast(cw[mb][NG + g], d1, vbase);   // superword 2gq + 1
        kop[mb][0] = u32x4{d0[0], d0[1], d0[2], d0[3]};
        kop[mb][1] = u32x4{d0[4], d0[5], d0[6], d0[7]};
        kop[mb][2] = u32x4{d1[0], d1[1], d1[2], d1[3]};
        kop[mb][3] = u32x4{d1[4], d1[5], d1[6], d1[7]};
      }
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
        const float init = -q4[hb][g];
        f32x4 acc[2] = {{init, init, init, init}, {init, init, init, init}};
#pragma unroll
        for (int kbl = 0; kbl < 4; ++kbl) {
          const u32x4 qv = s_qs[hb][4 * g + kbl][lane];
          acc[0] = mfma16x16x32(kop[0][kbl], qv, acc[0]);
          acc[1] = mfma16x16x32(kop[1][kbl], qv, acc[1]);
        }
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            s[mb][hb][j] = fmaf(scl[mb][j], acc[mb][j], fmaf(-szr[mb][j], qsum[hb][g], s[mb][hb][j]));
      }
      __builtin_amdgcn_sched_barrier(0);  // keep each group's LDS reads within the group
    }

    // -- online softmax (log2 domain, lazy rescale) ------------------------------
    float p[2][NHB][4];
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb) {
      float mt = -1.0e30f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v = s[mb][hb][j] * scale_log2;
          if constexpr (!full) {
            const int pos = p0 + 16 * mb + 4 * gq + j;
            if (pos < lo || pos >= hi) v = -1.0e30f;
          }
          s[mb][hb][j] = v;
          mt = fmaxf(mt, v);
        }
      mt = wave_max_over_groups(mt);
      // keep exp2 arguments <= 8: rescale only when a head's max grows past that
      if (__any(mt > m_run[hb] + 8.0f)) {
        const float m_new = fmaxf(m_run[hb], mt);
        const float alpha = __builtin_amdgcn_exp2f(m_run[hb] - m_new);
        l_run[hb] *= alpha;
#pragma unroll
        for (int g = 0; g < NG; ++g) zp[hb][g] *= alpha;
        float ao[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ao[j] = __shfl(alpha, 4 * gq + j);
        // rare: one accumulator tile at a time keeps the register footprint small
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
          for (int j = 0; j < 4; ++j) O[hb][nb][j] *= ao[j];
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
#pragma unroll
          for (int j = 0; j < 4; ++j) SP[hb][g][j] *= ao[j];
          __builtin_amdgcn_sched_barrier(0);
        }
        m_run[hb] = m_new;
      }
      float ls = 0.f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = __builtin_amdgcn_exp2f(s[mb][hb][j] - m_run[hb]);
          p[mb][hb][j] = e;
          ls += e;
        }
      l_run[hb] += ls;
    }
    __builtin_amdgcn_sched_barrier(0);

    // -- output: O += P'_g V_g per group -------------------------------------------
    uint32_t co[8][NG];  // tokens tau(i): word of every group in superword la/2
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = (i < 4 ? 4 * gq + i : 16 + 4 * gq + (i - 4));
      if constexpr (NG == 4) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(tl + 16 * G::cslot(t, la >> 1));
        co[i][0] = v.x; co[i][1] = v.y; co[i][2] = v.z; co[i][3] = v.w;
      } else {
        const u32x2 v = *reinterpret_cast<const u32x2*>(tl + 16 * G::cslot(t, la >> 2) + 8 * ((la >> 1) & 1));
        co[i][0] = v.x; co[i][1] = v.y;
      }
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      asm volatile("" ::: "memory");
      f32x4 pv[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) pv[mb][j] = param2(mb, j, g / 2);
      float scl[2][4], zr[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          scl[mb][j] = (g & 1) ? pv[mb][j].z : pv[mb][j].x;
          zr[mb][j] = (g & 1) ? pv[mb][j].w : pv[mb][j].y;
        }
      // p'_g = p * scale as a bf16 hi + lo pair: the two output MFMAs see
      // hi + lo = p'_g to ~2^-17, so the contraction is FP32-accurate.
      u32x4 Ph[NHB], Pl[NHB];
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
        float pg[8];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int j = 0; j < 4; ++j) pg[4 * mb + j] = p[mb][hb][j] * scl[mb][j];
        uint32_t hv[4], lv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          hv[r] = pack_bf16(pg[2 * r], pg[2 * r + 1]);
          lv[r] = pack_bf16(pg[2 * r] - bf16_lo(hv[r]), pg[2 * r + 1] - bf16_hi(hv[r]));
        }
        Ph[hb] = u32x4{hv[0], hv[1], hv[2], hv[3]};
        Pl[hb] = u32x4{lv[0], lv[1], lv[2], lv[3]};
        float z = zp[hb][g];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int j = 0; j < 4; ++j) z = fmaf(pg[4 * mb + j], zr[mb][j], z);
        zp[hb][g] = z;
      }
      uint32_t dr[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t x = __builtin_amdgcn_perm(co[2 * r + 1][g], co[2 * r][g], perm_sel);
        unpack_word_fast(x, dr[r], vbase);
      }
#pragma unroll
      for (int nbl = 0; nbl < 8; ++nbl) {
        const u32x4 bv = {dr[0][nbl], dr[1][nbl], dr[2][nbl], dr[3][nbl]};
#pragma unroll
        for (int hb = 0; hb < NHB; ++hb) {
          O[hb][8 * g + nbl] = mfma16x16x32(Ph[hb], bv, O[hb][8 * g + nbl]);
          O[hb][8 * g + nbl] = mfma16x16x32(Pl[hb], bv, O[hb][8 * g + nbl]);
        }
      }
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
        SP[hb][g] = mfma16x16x32(Ph[hb], ones, SP[hb][g]);
        SP[hb][g] = mfma16x16x32(Pl[hb], ones, SP[hb][g]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
}

template <int D, int R, int NHB, bool PAGED>
__global__ __launch_bounds__(256, 1) void decode_stage1(DecodeArgs a) {
  using G = Geo<D, R>;
  constexpr int NG = G::NG, KR = G::KR, NB = G::NB, SW = G::SW, ROWB = G::ROWB, PB = G::PB;
  constexpr int TILE = 32;
  static_assert(R % 32 == 0 && D % 256 == 0, "unsupported shape");

  // Three tile-ring buffers as separate LDS objects (so the compiler's wait
  // insertion can tell a read of one from the DMA in flight to another); after
  // the loop the first holds the merge buffer, and the window split uses the
  // first two for its partial sums and staged rows.
  constexpr int RING = 4 * G::TILE_LDS;  // 4 waves
  static_assert(16 * D * 4 <= RING, "merge buffer does not fit in one ring buffer");
  __shared__ __attribute__((aligned(16))) uint8_t s_r0[RING];
  __shared__ __attribute__((aligned(16))) uint8_t s_r1[RING];
  __shared__ __attribute__((aligned(16))) uint8_t s_r2[RING];
  __shared__ float s_ml[4][NHB * 16][2];
  // score-MFMA B operands of the query (one copy per block): [hb][K-block][lane]
  __shared__ __attribute__((aligned(16))) u32x4 s_qs[NHB][4 * NG][64];
  // blockIdx.x = (sequence, head group of 16 NHB heads); split-major grid: the
  // real splits of every sequence dispatch before the surplus (empty) ones
  const int nhg = (a.H + 16 * NHB - 1) / (16 * NHB);
  const int b = blockIdx.x / nhg, h0 = 16 * NHB * (blockIdx.x % nhg), split = blockIdx.y;
  const int ns = a.num_kv_splits[b];
  const int nq = min(max(ns - 1, 1), a.S1 - 1);
  if (split > nq) return;

  const int32_t start = a.kv_indptr[b];
  SeqCtx sc;
  sc.idx = a.kv_indices + start;
  sc.shift = a.page_shift;
  sc.L = a.seq_lens ? int(a.seq_lens[b]) : int(a.kv_indptr[b + 1] - start);
  const int64_t req = a.req_idx[b];

  if (split == nq) {
    window_split<D, R, NHB>(a, b, h0, split, sc, req, reinterpret_cast<float*>(s_r0), s_r1);
    return;
  }

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int gq = lane >> 4, la = lane & 15;
  const int L = sc.L;
  const int lo = min(a.P, L), hi = max(L - a.W, lo);
  const int t_first = lo / TILE;
  const int ntiles = hi > lo ? (hi + TILE - 1) / TILE - t_first : 0;
  const int per = (ntiles + nq - 1) / nq;
  const int my_begin = t_first + min(split * per, ntiles);
  const int my_end = t_first + min((split + 1) * per, ntiles);

  // ---- query operands -----------------------------------------------------------
  // s_qs[hb][4g+kbl]: B operand of the score MFMA, lane (gq, la) = head la+16hb,
  // element pair r of K-block kbl <-> in-group features 16s+k and 16s+k+8 with
  // s = 2gq + kbl/2, k = 4(kbl%2) + r, scaled by 2^(5-e_k). Wave hb%4 stores
  // head block hb; every wave keeps the per-head sums it needs.
  WaveState<D, R, NHB> st;
  auto& qr = st.qr;
  auto& q4 = st.q4;
  auto& qsum = st.qsum;
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    const int h = h0 + 16 * hb + la;
    const bool hv = h < a.H;
    const uint16_t* qh = a.q + b * a.q_sb + (int64_t)min(h, a.H - 1) * a.q_sh;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float s_sum = 0.f, s_w = 0.f;
#pragma unroll
      for (int kbl = 0; kbl < 4; ++kbl) {
        const int s = 2 * gq + kbl / 2;
        const int f0 = 128 * g + 16 * s + 4 * (kbl % 2);
        const u32x2 lo4 = *reinterpret_cast<const u32x2*>(qh + f0);
        const u32x2 hi4 = *reinterpret_cast<const u32x2*>(qh + f0 + 8);
        uint32_t outv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t wl = (r < 2 ? lo4.x : lo4.y), wh = (r < 2 ? hi4.x : hi4.y);
          const float vl = hv ? ((r & 1) ? bf16_hi(wl) : bf16_lo(wl)) : 0.f;
          const float vh = hv ? ((r & 1) ? bf16_hi(wh) : bf16_lo(wh)) : 0.f;
          const float wk = pair_weight(4 * (kbl % 2) + r);
          s_sum += vl + vh;
          s_w += (vl + vh) * wk;
          outv[r] = pack_bf16(vl * wk, vh * wk);
        }
        if (wave == (hb & 3)) s_qs[hb][4 * g + kbl][lane] = u32x4{outv[0], outv[1], outv[2], outv[3]};
      }
      qsum[hb][g] = wave_sum_over_groups(s_sum);
      q4[hb][g] = 4.f * wave_sum_over_groups(s_w);
    }
#pragma unroll
    for (int kr = 0; kr < KR; ++kr) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qh + D + 32 * kr + 8 * gq);
      qr[hb][kr] = hv ? v : u32x4{0, 0, 0, 0};
    }
  }
  __syncthreads();
  const uint32_t one = la == 0 ? 0x3F803F80u : 0u;
  st.ones = u32x4{one, one, one, one};
  st.perm_sel = (la & 1) ? 0x07060302u : 0x05040100u;
  st.vbase = 0x40804080u;
  st.s_qs = s_qs;
  st.lane = lane;
  st.gq = gq;
  st.la = la;
  st.lo = lo;
  st.hi = hi;
  st.scale_log2 = a.sm_scale * kLog2e;

  auto& O = st.O;
  auto& SP = st.SP;
  auto& m_run = st.m_run;
  auto& l_run = st.l_run;
  auto& zp = st.zp;
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) O[hb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < NG; ++g) { SP[hb][g] = f32x4{0.f, 0.f, 0.f, 0.f}; zp[hb][g] = 0.f; }
    m_run[hb] = -1.0e30f;
    l_run[hb] = 0.f;
  }

  // ---- tile pipeline ----------------------------------------------------------
  // Three LDS tile buffers per wave, filled by direct global->LDS loads two
  // tiles ahead; the slot lookup for a tile runs one further tile ahead.
  constexpr int NBUF = 3;
  static_assert(window_rows_bytes<D, R>() <= RING && window_part_floats() * 4 <= RING, "window scratch");
  uint8_t* const tb0 = s_r0 + wave * G::TILE_LDS;
  uint8_t* const tb1 = s_r1 + wave * G::TILE_LDS;
  uint8_t* const tb2 = s_r2 + wave * G::TILE_LDS;
  // what this lane moves for every tile: 16-byte slot q of a 1 KB DMA block.
  // PAGED: byte offsets from the tile's first slot; else token index + chunk.
  int c_tok[G::CL], c_off[G::CL], r_tok[G::RL], r_off[G::RL];
#pragma unroll
  for (int k = 0; k < G::CL; ++k) {
    const int q = 64 * k + lane, t = q / G::CCH, sl = q % G::CCH;
    c_tok[k] = t;
    c_off[k] = 16 * (sl ^ (t & (G::CCH - 1)));  // inverse of cslot
  }
#pragma unroll
  for (int k = 0; k < G::RL; ++k) {
    const int q = 64 * k + lane, t = q / G::RCH, sl = q % G::RCH;
    r_tok[k] = t;
    r_off[k] = 16 * (sl ^ (t & (G::RCH - 1)));
  }
  const bool p_live = lane < 32 * G::PCH;
  const int p_tok = p_live ? lane / G::PCH : 0, p_off = p_live ? 16 * (lane % G::PCH) : 0;

  // slot lookup for one tile: PAGED -> one page base; else per-lane token slots
  struct Idx {
    int base;
    int cs[PAGED ? 1 : G::CL], rs[PAGED ? 1 : G::RL], ps;
  };
  auto lookup = [&](int tile, Idx& x) {
    const int p0 = tile * TILE;
    if constexpr (PAGED) {
      x.base = int(slot_of(sc, p0));
    } else {
#pragma unroll
      for (int k = 0; k < G::CL; ++k) x.cs[k] = int(slot_of(sc, p0 + c_tok[k]));
#pragma unroll
      for (int k = 0; k < G::RL; ++k) x.rs[k] = int(slot_of(sc, p0 + r_tok[k]));
      x.ps = int(slot_of(sc, p0 + p_tok));
    }
  };
  auto dma = [&](const Idx& x, uint8_t* buf) {
    if constexpr (PAGED) {
      const uint8_t* cb = a.codes + (int64_t)x.base * ROWB;
      const uint8_t* rb = reinterpret_cast<const uint8_t*>(a.rope) + (int64_t)x.base * G::RBYTES;
      const uint8_t* pb = reinterpret_cast<const uint8_t*>(a.params) + (int64_t)x.base * PB;
#pragma unroll
      for (int k = 0; k < G::CL; ++k)
        lds_dma16(cb + (c_tok[k] * ROWB + c_off[k]), buf + 1024 * k);
#pragma unroll
      for (int k = 0; k < G::RL; ++k)
        lds_dma16(rb + (r_tok[k] * G::RBYTES + r_off[k]), buf + G::OFF_R + 1024 * k);
      lds_dma16(pb + (p_tok * PB + p_off), buf + G::OFF_P);
    } else {
#pragma unroll
      for (int k = 0; k < G::CL; ++k)
        lds_dma16(a.codes + (int64_t)x.cs[k] * ROWB + c_off[k], buf + 1024 * k);
#pragma unroll
      for (int k = 0; k < G::RL; ++k)
        lds_dma16(reinterpret_cast<const uint8_t*>(a.rope) + (int64_t)x.rs[k] * G::RBYTES + r_off[k],
                  buf + G::OFF_R + 1024 * k);
      lds_dma16(reinterpret_cast<const uint8_t*>(a.params) + (int64_t)x.ps * PB + p_off, buf + G::OFF_P);
    }
  };

  auto compute = [&](int tile, const uint8_t* tl) {
    const int p0 = tile * TILE;
    if ((p0 >= lo) && (p0 + TILE <= hi))
      tile_compute<D, R, NHB, true>(st, tile, tl);
    else
      tile_compute<D, R, NHB, false>(st, tile, tl);
  };

  // tiles of this wave: my_begin + wave + 4k
  const int t0 = my_begin + wave;
  const int nmine = t0 < my_end ? (my_end - t0 + 3) / 4 : 0;
  Idx ix0, ix1, ix2;
  if (nmine > 0) { lookup(t0, ix0); dma(ix0, tb0); }
  if (nmine > 1) { lookup(t0 + 4, ix1); dma(ix1, tb1); }
  if (nmine > 2) lookup(t0 + 8, ix2);
  // step k computes tile k from ring buffer k % 3, after starting the DMA of
  // tile k + 2 (its slots were looked up during step k - 1) and the lookup of k + 3
  for (int k = 0; k < nmine; k += NBUF) {
    if (k + 2 < nmine) dma(ix2, tb2);
    if (k + 3 < nmine) lookup(t0 + 4 * (k + 3), ix0);
    compute(t0 + 4 * k, tb0);
    if (k + 1 >= nmine) break;
    if (k + 3 < nmine) dma(ix0, tb0);
    if (k + 4 < nmine) lookup(t0 + 4 * (k + 4), ix1);
    compute(t0 + 4 * (k + 1), tb1);
    if (k + 2 >= nmine) break;
    if (k + 4 < nmine) dma(ix1, tb1);
    if (k + 5 < nmine) lookup(t0 + 4 * (k + 5), ix2);
    compute(t0 + 4 * (k + 2), tb2);
  }

  // ---- finalize this wave: unnormalised o, m, l ------------------------------
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    l_run[hb] = wave_sum_over_groups(l_run[hb]);
#pragma unroll
    for (int g = 0; g < NG; ++g) zp[hb][g] = wave_sum_over_groups(zp[hb][g]);
    if (gq == 0) {
      s_ml[wave][16 * hb + la][0] = m_run[hb];
      s_ml[wave][16 * hb + la][1] = l_run[hb];
    }
  }
  __syncthreads();  // every wave is done with its tile buffers: s_r0 becomes the merge buffer
  float* s_obuf = reinterpret_cast<float*>(s_r0);
  float fac[NHB][4];
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int h = 16 * hb + 4 * gq + j;
      float M = -1.0e30f;
#pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, s_ml[w][h][0]);
      float Ls = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) Ls += __builtin_amdgcn_exp2f(s_ml[w][h][0] - M) * s_ml[w][h][1];
      fac[hb][j] = Ls > 0.f ? __builtin_amdgcn_exp2f(s_ml[wave][h][0] - M) / Ls : 0.f;
    }
  // one head block at a time: the four waves' partials are summed in a fixed
  // order (deterministic) in s_obuf, then written out
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    for (int w = 0; w < 4; ++w) {
      if (wave == w) {
        float spo[NG][4], zpo[NG][4];
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            spo[g][j] = __shfl(SP[hb][g][j], 16 * gq);
            zpo[g][j] = __shfl(zp[hb][g], 4 * gq + j);
          }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int g = nb / 8, nbl = nb % 8;
          const int f = 128 * g + 16 * (la >> 1) + 8 * (la & 1) + nbl;
          const float wgt = pair_weight(nbl);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float v = ((O[hb][nb][j] - 4.f * spo[g][j]) * wgt - zpo[g][j]) * fac[hb][j];
            float* dst = &s_obuf[(4 * gq + j) * D + f];
            *dst = (w == 0) ? v : *dst + v;
          }
        }
      }
      __syncthreads();
    }
    // write the head block's normalised partial
    const int hmax = min(16, a.H - h0 - 16 * hb);
    for (int e = tid; e < hmax * D; e += 256) {
      const int h = e / D, f = e % D;
      a.logits[(((int64_t)b * a.H + h0 + 16 * hb + h) * a.S1 + split) * D + f] = s_obuf[h * D + f];
    }
    __syncthreads();
  }
  if (lane < 16 && wave < NHB) {
    const int h = 16 * wave + lane;
    if (h0 + h < a.H) {
      float M = -1.0e30f;
      for (int w = 0; w < 4; ++w) M = fmaxf(M, s_ml[w][h][0]);
      float Ls = 0.f;
      for (int w = 0; w < 4; ++w) Ls += __builtin_amdgcn_exp2f(s_ml[w][h][0] - M) * s_ml[w][h][1];
      a.lse[((int64_t)b * a.H + h0 + h) * a.S1 + split] = Ls > 0.f ? (M + __log2f(Ls)) * kLn2 : kNeutralLse;
    }
  }
}

// ---------------------------------------------------------------------------
// Stage 2: LSE merge of the nq + 1 partials -> bf16 output.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(128) void decode_stage2(const float* __restrict__ logits,
                                                     const float* __restrict__ lse,
                                                     const int32_t* __restrict__ num_kv_splits,
                                                     int H, int S1, uint16_t* out, int64_t o_sb,
                                                     int64_t o_sh) {
  constexpr int FPT = D / 128;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int nq = min(max(num_kv_splits[b] - 1, 1), S1 - 1);
  const int64_t row = ((int64_t)b * H + h) * S1;
  float M = -3.0e38f;
  for (int s = 0; s <= nq; ++s) M = fmaxf(M, lse[row + s]);
  float acc[FPT], den = 0.f;
#pragma unroll
  for (int i = 0; i < FPT; ++i) acc[i] = 0.f;
  for (int s = 0; s <= nq; ++s) {
    const float w = __builtin_amdgcn_exp2f((lse[row + s] - M) * kLog2e);
    den += w;
    const float* src = logits + (row + s) * D + threadIdx.x * FPT;
#pragma unroll
    for (int i = 0; i < FPT; ++i) acc[i] = fmaf(w, src[i], acc[i]);
  }
  const float inv = 1.f / den;
  uint16_t* dst = out + b * o_sb + h * o_sh + threadIdx.x * FPT;
#pragma unroll
  for (int i = 0; i < FPT; ++i) dst[i] = float_to_bf16(acc[i] * inv);
}

}  // namespace rolaq

// ---------------------------------------------------------------------------
// Host launchers (called from api.cpp).
// ---------------------------------------------------------------------------
hipError_t rolaq_launch_decode(const rolaq::DecodeArgs& a, int D, int R, int max_splits,
                               uint16_t* out, int64_t o_sb, int64_t o_sh, hipStream_t stream) {
  using namespace rolaq;
  // one block per (sequence, 16 heads, split)
  const dim3 grid(a.B * ((a.H + 15) / 16), max_splits + 1), block(256);
#define ROLAQ_DEC(DD, RR, NH)                                                         \
  if (D == DD && R == RR) {                                                           \
    if (a.page_shift >= 5)                                                            \
      hipLaunchKernelGGL((decode_stage1<DD, RR, NH, true>), grid, block, 0, stream, a);  \
    else                                                                              \
      hipLaunchKernelGGL((decode_stage1<DD, RR, NH, false>), grid, block, 0, stream, a); \
    hipLaunchKernelGGL((decode_stage2<DD>), dim3(a.B * a.H), dim3(128), 0, stream,     \
                       a.logits, a.lse, a.num_kv_splits, a.H, a.S1, out, o_sb, o_sh); \
    return hipGetLastError();                                                         \
  }
  ROLAQ_DEC(512, 64, 1)
  ROLAQ_DEC(256, 32, 1)
#undef ROLAQ_DEC
  return hipErrorInvalidValue;
}
