// Absorbed MLA decode attention over the packed INT2 cache (gfx950).
//
// Reference behaviour: packed_mla_decode_gf_fwd + _fwd_hp_window_stage1 +
// stage-2 merge of the OSCAR SGLang fork (call site
// deployment/patches/rolaq_sglang.patch:51-111); arithmetic of
// mla_quant/cache.py:1007-1073 + eager MLA attention.
//
// Work split: grid (max_splits + 1, B). Block (s, b) with s < nq = max(ns_b - 1, 1)
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
// Thread t: head h = t & 15 (+16 hb), chunk c = t >> 4 of D/16 latent and R/16
// rope dims. Writes the normalised partial and natural-log LSE at split slot.
// ---------------------------------------------------------------------------
template <int D, int R, int NHB>
__device__ void window_split(const DecodeArgs& a, int b, int slot_split, const SeqCtx& sc,
                             int64_t req, float* smem) {
  constexpr int MAXW = 64;
  constexpr int FC = D / 16, RC = R / 16;
  const int t = threadIdx.x, h16 = t & 15, c = t >> 4, lane = t & 63, wave = t >> 6;
  const int L = sc.L, P = a.P, W = a.W;
  // window positions in increasing order: [0, min(P, L)) U [max(L - W, P), L)
  const int n_sink = min(P, L);
  const int rec_lo = max(L - W, n_sink);
  const int nw = n_sink + (L - rec_lo);
  float* sc_part = smem;               // [4 waves][16 heads][MAXW]
  float* prob = smem + 4 * 16 * MAXW;  // [16 heads][MAXW]
  for (int hb = 0; hb < NHB; ++hb) {
    const int h = 16 * hb + h16;
    const bool hv = h < a.H;
    const uint16_t* qh = a.q + b * a.q_sb + (int64_t)min(h, a.H - 1) * a.q_sh;
    float qv[FC], qr[RC];
#pragma unroll
    for (int i = 0; i < FC; ++i) qv[i] = hv ? bf16_to_float(qh[c * FC + i]) : 0.f;
#pragma unroll
    for (int i = 0; i < RC; ++i) qr[i] = hv ? bf16_to_float(qh[D + c * RC + i]) : 0.f;
    for (int i = 0; i < nw; ++i) {
      const int pos = i < n_sink ? i : rec_lo + (i - n_sink);
      const uint16_t* row = a.hp + (int64_t)ring_row(req, pos, P, W) * D;
      const uint16_t* rp = a.rope + slot_of(sc, pos) * R;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < FC; ++k) acc = fmaf(qv[k], bf16_to_float(row[c * FC + k]), acc);
#pragma unroll
      for (int k = 0; k < RC; ++k) acc = fmaf(qr[k], bf16_to_float(rp[c * RC + k]), acc);
      acc = wave_sum_over_groups(acc);  // chunks c, c^1, c^2, c^3 of this wave
      if (lane < 16) sc_part[(wave * 16 + h16) * MAXW + i] = acc;
    }
    __syncthreads();
    float m = -3.0e38f, l = 0.f;
    if (c == 0) {
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
      const int pos = i < n_sink ? i : rec_lo + (i - n_sink);
      const uint16_t* row = a.hp + (int64_t)ring_row(req, pos, P, W) * D;
      const float p = prob[h16 * MAXW + i];
#pragma unroll
      for (int k = 0; k < FC; ++k) o[k] = fmaf(p, bf16_to_float(row[c * FC + k]), o[k]);
    }
    if (hv) {
      float* dst = a.logits + (((int64_t)b * a.H + h) * a.S1 + slot_split) * D + c * FC;
#pragma unroll
      for (int k = 0; k < FC; ++k) dst[k] = o[k] * inv;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Stage 1: one block per (split, sequence).
// ---------------------------------------------------------------------------
template <int D, int R, int NHB>
__global__ __launch_bounds__(256, 1) void decode_stage1(DecodeArgs a) {
  constexpr int NG = D / 128;     // quantization groups
  constexpr int KR = R / 32;      // rope K-blocks
  constexpr int NB = D / 16;      // output N-blocks (16 features each)
  constexpr int SW = 4 * NG;      // bytes of one superword (word s of every group)
  constexpr int ROWB = D / 4;     // packed bytes per token
  constexpr int PB = 8 * NG;      // param bytes per token
  constexpr int TILE = 32;
  static_assert(R % 32 == 0 && D % 128 == 0, "unsupported shape");

  constexpr int WIN_FLOATS = (4 * 16 + 16) * 64 + 16;  // window_split scratch
  constexpr int OBUF = NHB * 16 * D > WIN_FLOATS ? NHB * 16 * D : WIN_FLOATS;
  __shared__ __attribute__((aligned(16))) float s_obuf[OBUF];
  // tile params, per wave and buffer, transposed: [group][scale|zero][token]
  __shared__ __attribute__((aligned(16))) float s_par[4][2][NG][2][TILE];
  // score-MFMA B operands of the query (one copy per block): [hb][K-block][lane]
  __shared__ __attribute__((aligned(16))) u32x4 s_qs[NHB][4 * NG][64];
  __shared__ float s_ml[4][NHB * 16][2];

  const int split = blockIdx.x, b = blockIdx.y;
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
    window_split<D, R, NHB>(a, b, split, sc, req, s_obuf);
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

  // ---- query operands -------------------------------------------------------
  // s_qs[hb][4g+kbl]: B operand of the score MFMA, lane (gq, la) = head la+16hb,
  // element pair r of K-block kbl <-> in-group features 16s+k and 16s+k+8 with
  // s = 2gq + kbl/2, k = 4(kbl%2) + r, scaled by 2^(5-e_k). Wave hb%4 builds
  // head block hb; every wave derives the per-head sums it needs.
  u32x4 qr[NHB][KR];
  float q4[NHB][NG], qsum[NHB][NG];
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    const int h = 16 * hb + la;
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
  const u32x4 ones = {one, one, one, one};
  const uint32_t perm_sel = (la & 1) ? 0x07060302u : 0x05040100u;

  f32x4 O[NHB][NB];
  f32x4 SP[NHB][NG];
  float m_run[NHB], l_run[NHB], zp[NHB][NG];
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) O[hb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < NG; ++g) { SP[hb][g] = f32x4{0.f, 0.f, 0.f, 0.f}; zp[hb][g] = 0.f; }
    m_run[hb] = -1.0e30f;
    l_run[hb] = 0.f;
  }
  const float scale_log2 = a.sm_scale * kLog2e;
  const bool paged = a.page_shift >= 5;  // a 32-token tile never straddles a page

  int buf = 0;
  for (int tile = my_begin + wave; tile < my_end; tile += 4, buf ^= 1) {
    const int p0 = tile * TILE;
    int64_t base = 0;
    if (paged) base = slot_of(sc, p0);
    auto slot_at = [&](int t) -> int64_t { return paged ? base + t : slot_of(sc, p0 + t); };

    // -- loads ---------------------------------------------------------------
    uint32_t cs[2][2 * NG];   // score rows: token 16mb + la, superwords 2gq, 2gq+1
    u32x4 ro[2][KR];          // rope rows of the same tokens
    uint32_t co[8][NG];       // output tokens tau(i): word of every group in superword la/2
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int64_t s = slot_at(16 * mb + la);
      load_words(a.codes + s * ROWB + 2 * SW * gq, cs[mb]);
#pragma unroll
      for (int kr = 0; kr < KR; ++kr)
        ro[mb][kr] = *reinterpret_cast<const u32x4*>(a.rope + s * R + 32 * kr + 8 * gq);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = (i < 4 ? 4 * gq + i : 16 + 4 * gq + (i - 4));
      const int64_t s = slot_at(t);
      load_words(a.codes + s * ROWB + SW * (la >> 1), co[i]);
    }
    // params of the tile -> this wave's LDS buffer, transposed to [g][field][token]
    float (*par)[2][TILE] = s_par[wave][buf];
    if (lane < 16 * NG) {
      // positions outside [lo, hi) get zero params so that masked tokens (p = 0)
      // contribute exact zeros even if their slot was never written
      const int tok = (lane * 16) / PB, g0 = ((lane * 16) % PB) / 8;
      const int pos = p0 + tok;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (pos >= lo && pos < hi) {
        const int64_t s = slot_at(tok);
        v = *reinterpret_cast<const f32x4*>(a.params + s * 2 * NG + 2 * g0);
      }
      par[g0][0][tok] = v.x;
      par[g0][1][tok] = v.y;
      par[g0 + 1][0][tok] = v.z;
      par[g0 + 1][1][tok] = v.w;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // -- scores --------------------------------------------------------------
    float s[2][NHB][4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kr = 0; kr < KR; ++kr) acc = mfma16x16x32(ro[mb][kr], qr[hb][kr], acc);
#pragma unroll
        for (int j = 0; j < 4; ++j) s[mb][hb][j] = acc[j];
      }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      u32x4 kop[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        uint32_t d0[8], d1[8];
        unpack_word(cs[mb][g], d0);        // superword 2gq
        unpack_word(cs[mb][NG + g], d1);   // superword 2gq + 1
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
        for (int mb = 0; mb < 2; ++mb) {
          const f32x4 scl = *reinterpret_cast<const f32x4*>(&par[g][0][16 * mb + 4 * gq]);
          const f32x4 zer = *reinterpret_cast<const f32x4*>(&par[g][1][16 * mb + 4 * gq]);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            s[mb][hb][j] = fmaf(scl[j], acc[mb][j], fmaf(-scl[j] * zer[j], qsum[hb][g], s[mb][hb][j]));
        }
      }
    }

    // -- online softmax (log2 domain) ----------------------------------------
    const bool full = (p0 >= lo) && (p0 + TILE <= hi);
    float p[2][NHB][4];
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb) {
      float mt = -1.0e30f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v = s[mb][hb][j] * scale_log2;
          if (!full) {
            const int pos = p0 + 16 * mb + 4 * gq + j;
            if (pos < lo || pos >= hi) v = -1.0e30f;
          }
          s[mb][hb][j] = v;
          mt = fmaxf(mt, v);
        }
      mt = wave_max_over_groups(mt);
      const float m_new = fmaxf(m_run[hb], mt);
      if (__any(m_new > m_run[hb])) {
        const float alpha = __builtin_amdgcn_exp2f(m_run[hb] - m_new);
        l_run[hb] *= alpha;
#pragma unroll
        for (int g = 0; g < NG; ++g) zp[hb][g] *= alpha;
        float ao[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ao[j] = __shfl(alpha, 4 * gq + j);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int j = 0; j < 4; ++j) O[hb][nb][j] *= ao[j];
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int j = 0; j < 4; ++j) SP[hb][g][j] *= ao[j];
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

    // -- output: O += P'_g V_g per group --------------------------------------
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      f32x4 scl[2], zr[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        scl[mb] = *reinterpret_cast<const f32x4*>(&par[g][0][16 * mb + 4 * gq]);
        zr[mb] = *reinterpret_cast<const f32x4*>(&par[g][1][16 * mb + 4 * gq]);
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
        unpack_word(x, dr[r]);
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
    }
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
  __syncthreads();
  float fac[NHB][4];
  float Mh[NHB][4], Lh[NHB][4];
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
      Mh[hb][j] = M;
      Lh[hb][j] = Ls;
      fac[hb][j] = Ls > 0.f ? __builtin_amdgcn_exp2f(s_ml[wave][h][0] - M) / Ls : 0.f;
    }
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
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
            const int h = 16 * hb + 4 * gq + j;
            const float v = ((O[hb][nb][j] - 4.f * spo[g][j]) * wgt - zpo[g][j]) * fac[hb][j];
            float* dst = &s_obuf[h * D + f];
            *dst = (w == 0) ? v : *dst + v;
          }
        }
      }
    }
    __syncthreads();
  }
  // ---- write the split's normalised partial + LSE -----------------------------
  for (int e = tid; e < a.H * D; e += 256) {
    const int h = e / D, f = e % D;
    a.logits[(((int64_t)b * a.H + h) * a.S1 + split) * D + f] = s_obuf[h * D + f];
  }
  if (lane < 16 && wave < NHB) {
    // heads 16*wave + lane: recompute M, L from s_ml
    const int h = 16 * wave + lane;
    if (h < a.H) {
      float M = -1.0e30f;
      for (int w = 0; w < 4; ++w) M = fmaxf(M, s_ml[w][h][0]);
      float Ls = 0.f;
      for (int w = 0; w < 4; ++w) Ls += __builtin_amdgcn_exp2f(s_ml[w][h][0] - M) * s_ml[w][h][1];
      a.lse[((int64_t)b * a.H + h) * a.S1 + split] = Ls > 0.f ? (M + __log2f(Ls)) * kLn2 : kNeutralLse;
    }
  }
  (void)Mh; (void)Lh;
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
  const dim3 grid(max_splits + 1, a.B), block(256);
  const int nhb = (a.H + 15) / 16;
#define ROLAQ_DEC(DD, RR, NH)                                                         \
  if (D == DD && R == RR && nhb == NH) {                                              \
    hipLaunchKernelGGL((decode_stage1<DD, RR, NH>), grid, block, 0, stream, a);       \
    hipLaunchKernelGGL((decode_stage2<DD>), dim3(a.B * a.H), dim3(128), 0, stream,     \
                       a.logits, a.lse, a.num_kv_splits, a.H, a.S1, out, o_sb, o_sh); \
    return hipGetLastError();                                                         \
  }
  ROLAQ_DEC(512, 64, 1)
  ROLAQ_DEC(256, 32, 1)
  ROLAQ_DEC(256, 32, 3)
#undef ROLAQ_DEC
  return hipErrorInvalidValue;
}
