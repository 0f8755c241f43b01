// Absorbed MLA decode attention over the packed INT2 cache (gfx950).
//
// Reference behaviour: packed_mla_decode_gf_fwd + _fwd_hp_window_stage1 +
// stage-2 merge of the OSCAR SGLang fork (call site
// deployment/patches/rolaq_sglang.patch:51-111); arithmetic of
// mla_quant/cache.py:1007-1073 + eager MLA attention.
//
// Work split: grid (B * ceil(H / 16), max_splits + 1). Block (b, head group,
// s) with s < nq = max(ns_b - 1, 1) handles a contiguous range of 32-token
// tiles of the INT2 positions [P, L_b - W) for 16 heads; block s == nq handles
// the <= P + W BF16 window rows; larger s exit. A second kernel merges the
// nq + 1 partials by LSE.
//
// INT2 split arithmetic (per 32-token tile):
//   scores  S^T[t, h] = rope_th + 2^(1-kq_h) sum_g scale_tg (A_tgh - zero_tg Qsum_hg 2^(kq_h-1)),
//           A_tgh = sum_j (c_tj / 2) q'_hj on the fp4 x fp8 MFMA 16x16x128 with
//           M = 16 tokens, N = 16 heads, K = one quantization group: the code c
//           masked into an e2m1 nibble (0b00cc = c / 2) and q'_h = q_h 2^kq_h as
//           two e4m3 pieces (exact to 2^-10 of the head's largest |q|). The rope
//           term is a bf16 MFMA 16x16x32.
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

// Cache slot of position pos (clamped into [0, L)): page table entry * page + offset.
__device__ __forceinline__ int64_t slot_of(const SeqCtx& c, int pos) {
  pos = min(max(pos, 0), c.L - 1);
  const int64_t page = c.idx[pos >> c.shift];
  return (page << c.shift) + (pos & ((1 << c.shift) - 1));
}

__device__ __forceinline__ int ring_row(int64_t req, int pos, int P, int W) {
  const int inner = pos < P ? pos : P + max(pos - P, 0) % max(W, 1);
  return int(1 + req * (P + W) + inner);
}

__device__ __forceinline__ u32x4 lds128(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ f32x4 lds128f(const uint8_t* p) { return *reinterpret_cast<const f32x4*>(p); }

// ---------------------------------------------------------------------------
// Window split: attention over the BF16 sink/recent rows of one sequence.
// The <= MAXW rows (hp_c ring rows + rope) are staged into LDS with 16-byte
// loads, then thread t < 256 = (head h = t & 15, chunk c = t >> 4) forms
// partial dots over D/16 latent + R/16 rope dims; waves reduce through LDS.
// Writes the normalised partial and natural-log LSE at split slot.
// Every thread of the block reaches every barrier.
// ---------------------------------------------------------------------------
constexpr int kMaxWindow = 32;
template <int D, int R>
constexpr int window_half_rows_bytes() { return kMaxWindow / 2 * (D + R) * 2; }

template <int D, int R>
__device__ void window_split(const DecodeArgs& a, int b, int h0, int slot_split, const SeqCtx& sc,
                             int64_t req, float* sc_part, float* prob, uint8_t* rows_lo, uint8_t* rows_hi) {
  constexpr int MAXW = kMaxWindow;
  constexpr int FC = D / 16, RC = R / 16;
  constexpr int ROWE = D + R;  // staged row: latent | rope (bf16 elements)
  const int t = threadIdx.x, h16 = t & 15, c = t >> 4, lane = t & 63, wave = t >> 6;
  const bool act = t < 256;
  const int L = sc.L, P = a.P, W = a.W;
  // window positions in increasing order: [0, min(P, L)) U [max(L - W, P), L)
  const int n_sink = min(P, L);
  const int rec_lo = max(L - W, n_sink);
  const int nw = n_sink + (L - rec_lo);
  // staged rows [MAXW][ROWE]: rows 0-15 in rows_lo, 16-31 in rows_hi
  auto row_at = [&](int i) {
    return reinterpret_cast<uint16_t*>(i < MAXW / 2 ? rows_lo : rows_hi) + (i & (MAXW / 2 - 1)) * ROWE;
  };
  // sc_part: [4 waves][16][MAXW]; prob: [16][MAXW] + 16
  // stage rows: D/8 + R/8 16-byte chunks per row
  constexpr int CPR = (D + R) / 8;
  for (int k = t; k < nw * CPR; k += blockDim.x) {
    const int i = k / CPR, ch = k % CPR;
    const int pos = i < n_sink ? i : rec_lo + (i - n_sink);
    const uint16_t* src = ch < D / 8 ? a.hp + (int64_t)ring_row(req, pos, P, W) * D + 8 * ch
                                     : a.rope + slot_of(sc, pos) * R + 8 * (ch - D / 8);
    *reinterpret_cast<u32x4*>(row_at(i) + 8 * ch) = *reinterpret_cast<const u32x4*>(src);
  }
  __syncthreads();
  const int h = h0 + h16;
  const bool hv = h < a.H;
  if (act) {
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
    static_assert(FC % 8 == 0 && (RC == 4 || RC == 2), "window chunking");
    for (int i = 0; i < nw; ++i) {
      const uint16_t* row = row_at(i);
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < FC; k += 8) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(row + c * FC + k);
        acc = fmaf(qv[k], bf16_lo(v.x), acc); acc = fmaf(qv[k + 1], bf16_hi(v.x), acc);
        acc = fmaf(qv[k + 2], bf16_lo(v.y), acc); acc = fmaf(qv[k + 3], bf16_hi(v.y), acc);
        acc = fmaf(qv[k + 4], bf16_lo(v.z), acc); acc = fmaf(qv[k + 5], bf16_hi(v.z), acc);
        acc = fmaf(qv[k + 6], bf16_lo(v.w), acc); acc = fmaf(qv[k + 7], bf16_hi(v.w), acc);
      }
      if constexpr (RC == 4) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(row + D + c * RC);
        acc = fmaf(qr[0], bf16_lo(v.x), acc); acc = fmaf(qr[1], bf16_hi(v.x), acc);
        acc = fmaf(qr[2], bf16_lo(v.y), acc); acc = fmaf(qr[3], bf16_hi(v.y), acc);
      } else {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(row + D + c * RC);
        acc = fmaf(qr[0], bf16_lo(v), acc); acc = fmaf(qr[1], bf16_hi(v), acc);
      }
      acc = wave_sum_over_groups(acc);  // chunks c, c^1, c^2, c^3 of this wave
      if (lane < 16) sc_part[(wave * 16 + h16) * MAXW + i] = acc;
    }
  }
  __syncthreads();
  if (t < 16) {
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
  if (act) {
    const float inv = prob[16 * MAXW + h16];
    float o[FC];
#pragma unroll
    for (int k = 0; k < FC; ++k) o[k] = 0.f;
    for (int i = 0; i < nw; ++i) {
      const uint16_t* row = row_at(i);
      const float p = prob[h16 * MAXW + i];
#pragma unroll
      for (int k = 0; k < FC; k += 8) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(row + c * FC + k);
        o[k] = fmaf(p, bf16_lo(v.x), o[k]); o[k + 1] = fmaf(p, bf16_hi(v.x), o[k + 1]);
        o[k + 2] = fmaf(p, bf16_lo(v.y), o[k + 2]); o[k + 3] = fmaf(p, bf16_hi(v.y), o[k + 3]);
        o[k + 4] = fmaf(p, bf16_lo(v.z), o[k + 4]); o[k + 5] = fmaf(p, bf16_hi(v.z), o[k + 5]);
        o[k + 6] = fmaf(p, bf16_lo(v.w), o[k + 6]); o[k + 7] = fmaf(p, bf16_hi(v.w), o[k + 7]);
      }
    }
    if (hv) {
      float* dst = a.logits + (((int64_t)b * a.H + h) * a.S1 + slot_split) * D + c * FC;
#pragma unroll
      for (int k = 0; k < FC; k += 4) *reinterpret_cast<f32x4*>(dst + k) = f32x4{o[k] * inv, o[k + 1] * inv, o[k + 2] * inv, o[k + 3] * inv};
    }
  }
}

// ---------------------------------------------------------------------------
// LDS image of one 32-token tile: codes (32 x D/4 B), rope (32 x 2R B), params
// (32 x 8 NG B). Code and rope rows are stored as 16-byte chunks with chunk c
// of token t at slot t*CH + (c ^ (t % CH)): sixteen lanes reading one chunk
// column of sixteen tokens then spread over the LDS banks.
// ---------------------------------------------------------------------------
template <int D, int R>
struct Geo {
  static constexpr int NG = D / 128;      // quantization groups
  static constexpr int KR = R / 32;       // rope K-blocks
  static constexpr int ROWB = D / 4;      // packed bytes per token
  static constexpr int PB = 8 * NG;       // param bytes per token
  static constexpr int RBYTES = 2 * R;    // rope bytes per token
  static constexpr int CCH = ROWB / 16;   // 16-byte chunks per row (8 / 4)
  static constexpr int RCH = RBYTES / 16;
  static constexpr int OFF_R = 32 * ROWB;
  static constexpr int OFF_P = OFF_R + 32 * RBYTES;
  static constexpr int TILE_LDS = OFF_P + 32 * PB;
  __device__ static constexpr int cslot(int t, int c) { return t * CCH + (c ^ (t & (CCH - 1))); }
  __device__ static constexpr int rslot(int t, int c) { return t * RCH + (c ^ (t & (RCH - 1))); }
};

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

// One 16-byte direct global->LDS load per lane (global_load_lds_dwordx4). The
// LDS destination is wave-uniform: lane i lands at dst + 16 i. Issued as
// inline asm, so the compiler adds no waits for it (it would otherwise wait
// for every such load at the first LDS read after it): the caller orders reads
// of the destination after the load with its own counted vmcnt wait. Nothing
// else in these kernels uses m0.
__device__ __forceinline__ void lds_dma16(const uint8_t* src, uint8_t* dst) {
  typedef __attribute__((address_space(3))) uint8_t lds8;
  const uint32_t lds_addr = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds8*)dst)));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory");
}

// s_waitcnt immediates (gfx9 encoding): vmcnt <= n only / lgkmcnt == 0 only.
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
constexpr int kLgkmcnt0 = 0xF | (0x3 << 14) | (0x7 << 4);

// Workgroup barrier that waits for this wave's LDS operations only (not for
// its global->LDS loads in flight); the empty asm statements keep the compiler
// from moving memory operations across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Page-table entries a wave needs for its share of one tile's direct loads:
// with pages of >= 32 tokens the tile's one page, else one entry per load
// instruction and lane. They are loaded a step before use, so the wait for
// them never waits for the tile loads issued in between.
template <int CLW, int RLW, bool PAGED>
struct TilePages {
  int pg;  // PAGED
  int cs[PAGED ? 1 : CLW], rs[PAGED ? 1 : RLW], ps;
};

constexpr int kXcds = 8;                 // accelerator dies (own L2 each) of the MI355X
constexpr int kPairs = 2;                // wave pairs per block
constexpr int kThreads = 128 * kPairs;   // 4 waves; two blocks share a CU
constexpr float kNoRef = -1.0e30f;       // "no score yet" / masked score (log2 units)
constexpr float kRefSlack = 64.f;        // max exp2 argument before a split is redone
constexpr float kFastShare = 0.65f;      // extra tile share of a first-round split (measured)

// ---------------------------------------------------------------------------
// Stage 1 INT2 splits. The block's 8 waves form 4 pairs; pair pr takes tiles
// my_begin + pr + 4k. For each tile, wave wh of a pair
//   phase 1: computes the scores of tokens 16wh..16wh+15 over the whole latent
//            and rope and leaves them in LDS for its partner;
//   phase 2: after the block barrier, takes the softmax of all 32 tokens (the
//            same values in both waves) and accumulates the output of its own
//            half of the quantization groups.
// Each wave keeps only its half of the output accumulators, so a wave fits in
// 256 registers and two waves share a SIMD.
//
// Tiles reach LDS by direct global->LDS loads, three buffers per pair; both
// waves of a pair load half a tile each. The barrier of step k follows a
// vmcnt(0) wait, so after it tile k+1 is complete for both waves, and every
// wave is done with the buffer of tile k-1, which then receives tile k+2.
//
// The softmax uses a fixed reference per head: the max of the pair's first
// tile. Later scores may exceed it by up to kRefSlack (exp2 <= 2^64 stays
// finite in every accumulator); a split where any score goes further is
// recomputed with the true max, so the tile loop carries no rescaling.
// ---------------------------------------------------------------------------
template <int D, int R, bool PAGED>
__global__ __launch_bounds__(kThreads, 2) void decode_stage1(DecodeArgs a) {
  using G = Geo<D, R>;
  constexpr int NG = G::NG, KR = G::KR, ROWB = G::ROWB, PB = G::PB, CCH = G::CCH, RCH = G::RCH;
  constexpr int GW = NG / 2;                  // output groups per wave
  constexpr int CLW = CCH / 4, RLW = RCH / 4; // direct loads per wave and tile (codes, rope)
  constexpr int PCT = PB / 16;                // 16-byte param chunks per token
  constexpr int TILE = 32;
  constexpr int RING = kPairs * G::TILE_LDS;
  static_assert(R % 32 == 0 && D % 256 == 0, "unsupported shape");
  static_assert(8 * D * 4 <= RING, "merge buffer (8 heads) does not fit in one ring buffer");
  static_assert(window_half_rows_bytes<D, R>() <= RING && 4 * 16 * kMaxWindow * 4 <= RING &&
                (16 * kMaxWindow + 16) * 4 <= NG * 4 * 64 * 16, "window scratch");
  using Pages = TilePages<CLW, RLW, PAGED>;

  // Three tile buffers as separate LDS objects, so the compiler's wait
  // insertion can tell reads of one from direct loads in flight to another.
  __shared__ __attribute__((aligned(16))) uint8_t s_r0[RING];
  __shared__ __attribute__((aligned(16))) uint8_t s_r1[RING];
  __shared__ __attribute__((aligned(16))) uint8_t s_r2[RING];
  // score-MFMA B operands of the query (fp8 e4m3): [group][piece][half][lane]
  __shared__ __attribute__((aligned(16))) u32x4 s_qs[NG][2][2][64];
  __shared__ __attribute__((aligned(16))) u32x4 s_qr[KR][64];  // rope B operands (bf16)
  __shared__ f32x2 s_qq[NG][16];           // per group and head: Qsum / 2, MFMA scale exponent (bits)
  __shared__ float s_ml[kPairs][16][3];    // per pair and head: reference max, sum of each wave
  __shared__ float s_mt[kPairs][2][16];    // per pair, wave and head: largest score seen

  const int nhg = (a.H + 15) / 16;
  // Head groups of one (sequence, split) read the same cache rows. With more
  // than one, the blocks are renumbered so that the nhg blocks of a (sequence,
  // split) get consecutive dispatch slots of one XCD (the dispatcher deals
  // linear block ids to the 8 XCDs round-robin): the second and later read the
  // rows from that XCD's L2 instead of HBM.
  int lin = blockIdx.x + gridDim.x * blockIdx.y;
  const int nblk = gridDim.x * gridDim.y;
  if (nhg > 1 && nblk % kXcds == 0) lin = (lin % kXcds) * (nblk / kXcds) + lin / kXcds;
  const int hg = lin % nhg, rest = lin / nhg;
  const int split = nhg > 1 ? rest % gridDim.y : blockIdx.y;
  const int b = nhg > 1 ? rest / gridDim.y : blockIdx.x / nhg;
  const int h0 = 16 * (nhg > 1 ? hg : blockIdx.x % nhg);
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
    window_split<D, R>(a, b, h0, split, sc, req, reinterpret_cast<float*>(s_r2),
                       reinterpret_cast<float*>(&s_qs[0][0][0]), s_r0, s_r1);
    return;
  }

  const int tid = threadIdx.x, lane = tid & 63;
  // the wave index is uniform: tile indices, LDS bases and page lookups then
  // live in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pr = wave >> 1, wh = wave & 1;
  const int gq = lane >> 4, la = lane & 15;
  const int L = sc.L;
  const int lo = min(a.P, L), hi = max(L - a.W, lo);
  const int t_first = lo / TILE;
  const int ntiles = hi > lo ? (hi + TILE - 1) / TILE - t_first : 0;
  // Tile shares: the first fsp splits (their blocks go out in the first
  // dispatch round) weigh 1 + kFastShare, the others 1 (measured at cfg2:
  // stage 1 51.9 -> 49.0 us; the blocks of the second round otherwise end
  // ~10 us after those of the first).
  // Without a first round to favour: equal shares of ceil(ntiles / nq) tiles
  // (surplus splits, if any, at the end and empty).
  const int fsp = min(a.fast_splits, nq);
  const int per = (ntiles + nq - 1) / nq;
  auto bound = [&](int sp) {
    if (fsp == 0 || fsp == nq) return min(sp * per, ntiles);
    if (sp >= nq) return ntiles;
    const float tot = fsp * (1.0f + kFastShare) + (nq - fsp);
    const float acc = sp <= fsp ? sp * (1.0f + kFastShare) : fsp * (1.0f + kFastShare) + (sp - fsp);
    return min(ntiles, (int)(ntiles * acc / tot + 0.5f));
  };
  const int my_begin = t_first + bound(split);
  const int my_end = t_first + bound(split + 1);
  // pair pr computes tiles tile0 + kPairs * k, k < nmine; the block runs kmax steps
  const int kmax = (my_end - my_begin + kPairs - 1) / kPairs;
  const int tile0 = my_begin + pr;
  const int nmine = tile0 < my_end ? (my_end - tile0 + kPairs - 1) / kPairs : 0;

  // ---- this wave's share of a tile's direct loads ------------------------------
  // load k of kind X moves chunk q = 64 (XLW wh + k) + lane to LDS slot q.
  int c_tok[CLW], c_off[CLW], r_tok[RLW], r_off[RLW];
#pragma unroll
  for (int k = 0; k < CLW; ++k) {
    const int q = 64 * (CLW * wh + k) + lane, t = q / CCH, sl = q % CCH;
    c_tok[k] = t;
    c_off[k] = 16 * (sl ^ (t & (CCH - 1))) + (PAGED ? t * ROWB : 0);
  }
#pragma unroll
  for (int k = 0; k < RLW; ++k) {
    const int q = 64 * (RLW * wh + k) + lane, t = q / RCH, sl = q % RCH;
    r_tok[k] = t;
    r_off[k] = 16 * (sl ^ (t & (RCH - 1))) + (PAGED ? t * G::RBYTES : 0);
  }
  // params: 2 PB chunks per tile, PB per wave (lanes < PB), not swizzled
  const bool p_live = lane < PB;
  const int p_tok = p_live ? (PB * wh + lane) / PCT : 0;
  const int p_off = p_live ? 16 * ((PB * wh + lane) % PCT) + (PAGED ? p_tok * PB : 0) : 0;

  // positions are clamped into [0, L) as slot_of does; a tile never starts past L
  const int pmask = (1 << sc.shift) - 1;
  auto entry = [&](int pos) { return sc.idx[min(pos, L - 1) >> sc.shift]; };
  auto slot = [&](int page, int pos) { return ((int64_t)page << sc.shift) + (min(pos, L - 1) & pmask); };
  // PAGED: lane i holds the page of the pair's tile at step kb + i, so a step's
  // page comes from a register (v_readlane) instead of a load and its wait
  int pg_lane = 0;
  auto lookup = [&](int step, Pages& x) {
    const int tile = tile0 + kPairs * step;
    const int p0 = tile * TILE;
    if constexpr (PAGED) {
      if ((step & 63) == 0) {
        const int t = tile + kPairs * lane;
        pg_lane = t < my_end ? entry(t * TILE) : 0;
      }
      x.pg = __builtin_amdgcn_readlane(pg_lane, step & 63);
    } else {
#pragma unroll
      for (int k = 0; k < CLW; ++k) x.cs[k] = entry(p0 + c_tok[k]);
#pragma unroll
      for (int k = 0; k < RLW; ++k) x.rs[k] = entry(p0 + r_tok[k]);
      x.ps = entry(p0 + p_tok);
    }
  };
  auto dma = [&](int tile, const Pages& x, uint8_t* buf) {
    const int p0 = tile * TILE;
    const uint8_t* rope8 = reinterpret_cast<const uint8_t*>(a.rope);
    const uint8_t* par8 = reinterpret_cast<const uint8_t*>(a.params);
    if constexpr (PAGED) {
      const int64_t base = slot(x.pg, p0);
      const uint8_t* cb = a.codes + base * ROWB;
      const uint8_t* rb = rope8 + base * G::RBYTES;
      const uint8_t* pb = par8 + base * PB;
#pragma unroll
      for (int k = 0; k < CLW; ++k) lds_dma16(cb + c_off[k], buf + 1024 * (CLW * wh + k));
#pragma unroll
      for (int k = 0; k < RLW; ++k) lds_dma16(rb + r_off[k], buf + G::OFF_R + 1024 * (RLW * wh + k));
      if (p_live) lds_dma16(pb + p_off, buf + G::OFF_P + 16 * PB * wh);
    } else {
#pragma unroll
      for (int k = 0; k < CLW; ++k)
        lds_dma16(a.codes + slot(x.cs[k], p0 + c_tok[k]) * ROWB + c_off[k], buf + 1024 * (CLW * wh + k));
#pragma unroll
      for (int k = 0; k < RLW; ++k)
        lds_dma16(rope8 + slot(x.rs[k], p0 + r_tok[k]) * G::RBYTES + r_off[k], buf + G::OFF_R + 1024 * (RLW * wh + k));
      if (p_live) lds_dma16(par8 + slot(x.ps, p0 + p_tok) * PB + p_off, buf + G::OFF_P + 16 * PB * wh);
    }
  };

  uint8_t* const tb0 = s_r0 + pr * G::TILE_LDS;
  uint8_t* const tb1 = s_r1 + pr * G::TILE_LDS;
  uint8_t* const tb2 = s_r2 + pr * G::TILE_LDS;
  // ---- query operands (wave w prepares groups w, w + 4, .. and rope K-block w) ---
  // Phase 1 forms the latent scores on MFMA with the codes as fp4 A operands
  // (0b00cc is c/2 in e2m1: a mask, no unpacking) and the query as fp8 e4m3 B
  // operands: q of head la and group g scaled by 2^kq (its largest |q| lands in
  // [128, 256)) and split into two e4m3 pieces q1 + q2; the MFMA's block scale
  // 2^-kq undoes the scaling. A bf16 value minus its nearest e4m3 has at most 4
  // significant bits, so the pair is exact for every element down to 2^-10 of
  // the group's maximum (below, off by < 2^-10 of it).
  // A lane (token, gq) holds the codes of features 32gq .. 32gq+31 of a group:
  // dword d nibble n = feature 32gq + 16(d>>1) + 2n + (d&1) (words 2gq, 2gq+1
  // split into even and odd codes). With the fp4 A layout this puts feature
  //   f(G', j) = 32 G + 16 (G'&1) + 2 (j&7) + ((j>>3)&1),  G = (G'>>1) + 2 (j>>4)
  // at K = 32 G' + j, byte j of B lane (head, G'): bytes j, j + 8 (j & 8 == 0)
  // hold the adjacent features 32 G + 16 (G'&1) + 2 (j&7) + {0, 1}, so lane
  // (head la, gq) reads its 32 features as two contiguous 16-feature chunks.
  // The query's global loads go out first, before the page lookups: they then
  // complete together with the lookups instead of queueing behind the first
  // tiles' direct loads (the memory counter drains in order).
  constexpr int QG = (NG + 2 * kPairs - 1) / (2 * kPairs);  // groups per wave
  const int hq = h0 + la;
  const bool hv = hq < a.H;
  const uint16_t* qh = a.q + b * a.q_sb + (int64_t)min(hq, a.H - 1) * a.q_sh;
  u32x4 qrv = {0u, 0u, 0u, 0u};
  if (wave < KR) qrv = *reinterpret_cast<const u32x4*>(qh + D + 32 * wave + 8 * gq);
  u32x4 qv[QG][4];  // chunk h (features 32((gq>>1) + 2h) + 16(gq&1) ..+15) in qv[gi][2h], [2h+1]
#pragma unroll
  for (int gi = 0; gi < QG; ++gi) {
    const int g = wave + 2 * kPairs * gi;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f = 32 * ((gq >> 1) + 2 * (i >> 1)) + 16 * (gq & 1) + 8 * (i & 1);
      qv[gi][i] = g < NG ? *reinterpret_cast<const u32x4*>(qh + 128 * g + f) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  // the first two tiles' loads fly while the query operands are prepared. The
  // wait for the page lookups (which also covers the query loads) comes before
  // the direct loads on every path: a wait for the query placed after them
  // would also wait for the tiles.
  Pages ix0, ix1, ix2;
  if (nmine > 0) lookup(0, ix0);
  if (nmine > 1) lookup(1, ix1);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  if (nmine > 0) dma(tile0, ix0, tb0);
  if (nmine > 1) dma(tile0 + kPairs, ix1, tb1);

  if (wave < KR) s_qr[wave][lane] = hv ? qrv : u32x4{0, 0, 0, 0};
#pragma unroll
  for (int gi = 0; gi < QG; ++gi) {
    const int g = wave + 2 * kPairs * gi;
    if (g >= NG) break;
    float mx = 0.f, sm = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!hv) qv[gi][i] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16_lo(qv[gi][i][e]), hi = bf16_hi(qv[gi][i][e]);
        mx = fmaxf(mx, fmaxf(fabsf(lo), fabsf(hi)));
        sm += lo + hi;
      }
    }
    mx = wave_max_over_groups(mx);  // over the group's 128 features of head la
    sm = wave_sum_over_groups(sm);
    int e = 0;
    if (mx > 0.f) frexpf(mx, &e);  // mx in [2^(e-1), 2^e)
    const int kq = mx > 0.f ? 8 - e : 0;
    const float qscale = ldexpf(1.f, kq);
    uint32_t w1[8], w2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w1[i] = w2[i] = 0u;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int k = 0; k < 8; ++k) {  // features 2k, 2k+1 of chunk h -> bytes j = 16h + k and j + 8
        const uint32_t qw = qv[gi][2 * h + (k >> 2)][k & 3];
        const float x0 = bf16_lo(qw) * qscale, x1 = bf16_hi(qw) * qscale;
        const uint32_t p1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
        const float r0 = x0 - __builtin_amdgcn_cvt_f32_fp8((int)p1, 0);
        const float r1 = x1 - __builtin_amdgcn_cvt_f32_fp8((int)p1, 1);
        const uint32_t p2 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r0, r1, 0, false);
        const int j = 16 * h + k;
        w1[j >> 2] |= (p1 & 0xffu) << (8 * (j & 3));
        w1[(j + 8) >> 2] |= ((p1 >> 8) & 0xffu) << (8 * (j & 3));
        w2[j >> 2] |= (p2 & 0xffu) << (8 * (j & 3));
        w2[(j + 8) >> 2] |= ((p2 >> 8) & 0xffu) << (8 * (j & 3));
      }
    s_qs[g][0][0][lane] = u32x4{w1[0], w1[1], w1[2], w1[3]};
    s_qs[g][0][1][lane] = u32x4{w1[4], w1[5], w1[6], w1[7]};
    s_qs[g][1][0][lane] = u32x4{w2[0], w2[1], w2[2], w2[3]};
    s_qs[g][1][1][lane] = u32x4{w2[4], w2[5], w2[6], w2[7]};
    // latent score = 2 sum_g scale (A_g - zero Qsum_g / 2), A_g = sum (c / 2) q
    if (gq == 0) s_qq[g][la] = f32x2{0.5f * sm, __int_as_float(127 - kq)};
  }
  lds_barrier();
  const uint32_t one = la == 0 ? 0x3F803F80u : 0u;
  const u32x4 ones = {one, one, one, one};
  const uint32_t perm_sel = (la & 1) ? 0x07060302u : 0x05040100u;
  const uint32_t vbase = 0x40804080u;
  const float scale_log2 = a.sm_scale * kLog2e;

  // ---- per-wave accumulators ---------------------------------------------------
  f32x4 O[GW][8];   // output, groups GW wh + gg, N-block nbl: head 4gq + j, column la
  f32x4 SP[GW];     // sum of p' per head (column 0)
  float zp[GW];     // sum of p' * zero per head la (partial over this lane's tokens)
  float l_lane;     // sum of p per head la (partial)
  float m_ref = kNoRef, m_seen = kNoRef;

  // phase 1: scores of tokens 16wh + (0..15), left for the partner in this
  // wave's own (now consumed) rope rows of the tile buffer
  // pre: the pair's reference is known (every tile but the first of the first
  // pass), so this wave turns its own 16 tokens' scores into probabilities
  // here -- each softmax term is computed once per pair -- and leaves those
  auto phase1 = [&](int tile, uint8_t* tl, bool pre) {
    const int p0 = tile * TILE;
    const int tA = 16 * wh + la;  // A-operand token of this lane
    // All of the query's B operands are read up front: read next to its MFMA,
    // each read's latency would stall the chain, and a buffer refilled while an
    // MFMA still reads it costs wait states.
    u32x4 qrp[KR];
    u32x8 qop[NG][2];  // [group][piece]
#pragma unroll
    for (int kr = 0; kr < KR; ++kr) qrp[kr] = s_qr[kr][lane];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) {
        const u32x4 lo4 = s_qs[g][pc][0][lane], hi4 = s_qs[g][pc][1][lane];
        qop[g][pc] = u32x8{lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
      }
    uint32_t cw[2 * NG];          // words s = 2gq (cw[g]) and 2gq+1 (cw[NG+g]) of token tA
    if constexpr (NG == 4) {
      const u32x4 v0 = lds128(tl + 16 * G::cslot(tA, 2 * gq));
      const u32x4 v1 = lds128(tl + 16 * G::cslot(tA, 2 * gq + 1));
      cw[0] = v0.x; cw[1] = v0.y; cw[2] = v0.z; cw[3] = v0.w;
      cw[4] = v1.x; cw[5] = v1.y; cw[6] = v1.z; cw[7] = v1.w;
    } else {
      const u32x4 v0 = lds128(tl + 16 * G::cslot(tA, gq));
      cw[0] = v0.x; cw[1] = v0.y; cw[2] = v0.z; cw[3] = v0.w;
    }
    u32x4 ropa[KR];
    f32x2 qqv[NG];  // Qsum / 2, MFMA scale exponent of head la per group
#pragma unroll
    for (int kr = 0; kr < KR; ++kr) ropa[kr] = lds128(tl + G::OFF_R + 16 * G::rslot(tA, 4 * kr + gq));
#pragma unroll
    for (int g = 0; g < NG; ++g) qqv[g] = s_qq[g][la];
    f32x4 accr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kr = 0; kr < KR; ++kr) accr = mfma16x16x32(ropa[kr], qrp[kr], accr);
    float s[4] = {0.f, 0.f, 0.f, 0.f};  // latent part, halved
    // C-layout tokens of this lane: 16wh + 4gq + j
    f32x4 pv[NG / 2][4];
#pragma unroll
    for (int gp = 0; gp < NG / 2; ++gp)
#pragma unroll
      for (int j = 0; j < 4; ++j) pv[gp][j] = lds128f(tl + G::OFF_P + (16 * wh + 4 * gq + j) * PB + 16 * gp);
    // all groups' MFMAs (independent chains of two), then the accumulation
    f32x4 acc[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      // codes as fp4: even codes of a word in one dword, odd codes in the next
      const u32x4 a4 = {cw[g] & 0x33333333u, (cw[g] >> 2) & 0x33333333u, cw[NG + g] & 0x33333333u,
                        (cw[NG + g] >> 2) & 0x33333333u};
      const int sb = __float_as_int(qqv[g].y);  // 127 - kq of (head la, group g)
      acc[g] = mfma_f4_f8(a4, qop[g][0], f32x4{0.f, 0.f, 0.f, 0.f}, sb);
      acc[g] = mfma_f4_f8(a4, qop[g][1], acc[g], sb);
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const f32x2 qq = qqv[g];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float scl = (g & 1) ? pv[g >> 1][j].z : pv[g >> 1][j].x;
        const float zr = (g & 1) ? pv[g >> 1][j].w : pv[g >> 1][j].y;
        s[j] = fmaf(scl, fmaf(-zr, qq.x, acc[g][j]), s[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = fmaf(2.f, s[j], accr[j]);
    const int pb = p0 + 16 * wh + 4 * gq;
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = (pb + j >= lo && pb + j < hi) ? s[j] * scale_log2 : kNoRef;
    if (pre) {
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        m_seen = fmaxf(m_seen, s[j]);
        s[j] = __builtin_amdgcn_exp2f(s[j] - m_ref);  // masked: 2^(-1e30) = 0
        ls += s[j];
      }
      l_lane += ls;  // this wave's own tokens only
    }
    *reinterpret_cast<f32x4*>(tl + G::OFF_R + 16 * G::RBYTES * wh + 16 * lane) = f32x4{s[0], s[1], s[2], s[3]};
    // params of masked tokens (rows that may never have been written) are
    // zeroed for phase 2, so they contribute exactly 0 whatever they held
    if (lane < PB) {
      const int t = 16 * wh + lane / PCT, pos = p0 + t;
      if (pos < lo || pos >= hi)
        *reinterpret_cast<f32x4*>(tl + G::OFF_P + t * PB + 16 * (lane % PCT)) = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  // phase 2: softmax of the tile and the output of groups GW wh .. GW wh + GW - 1
  auto phase2 = [&](const uint8_t* tl, bool first) {
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(tl + G::OFF_R + 16 * lane);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(tl + G::OFF_R + 16 * G::RBYTES + 16 * lane);
    // tokens tau(gq, i): probabilities, or (first tile of the first pass)
    // scores, from which both waves take the reference and the probabilities
    float p[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    if (first) {
      const float lm = fmaxf(fmaxf(fmaxf(p[0], p[1]), fmaxf(p[2], p[3])), fmaxf(fmaxf(p[4], p[5]), fmaxf(p[6], p[7])));
      m_seen = fmaxf(m_seen, lm);
      m_ref = wave_max_over_groups(lm);
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = __builtin_amdgcn_exp2f(p[i] - m_ref);
      // the sum counts this wave's own tokens (the partner counts the others)
      l_lane += wh == 0 ? (p[0] + p[1]) + (p[2] + p[3]) : (p[4] + p[5]) + (p[6] + p[7]);
    }
    // tokens tau(gq, i) = 4gq + i (i < 4), 16 + 4gq + i - 4 (i >= 4)
    float scl[GW][8], zr[GW][8];
    uint32_t co[8][GW];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = i < 4 ? 4 * gq + i : 16 + 4 * gq + (i - 4);
      if constexpr (GW == 2) {
        const f32x4 v = lds128f(tl + G::OFF_P + t * PB + 16 * wh);
        scl[0][i] = v.x; zr[0][i] = v.y; scl[1][i] = v.z; zr[1][i] = v.w;
        const u32x2 c = *reinterpret_cast<const u32x2*>(tl + 16 * G::cslot(t, la >> 1) + 8 * wh);
        co[i][0] = c.x; co[i][1] = c.y;
      } else {
        const f32x2 v = *reinterpret_cast<const f32x2*>(tl + G::OFF_P + t * PB + 8 * wh);
        scl[0][i] = v.x; zr[0][i] = v.y;
        co[i][0] = *reinterpret_cast<const uint32_t*>(tl + 16 * G::cslot(t, la >> 2) + 8 * ((la >> 1) & 1) + 4 * wh);
      }
    }
#pragma unroll
    for (int gg = 0; gg < GW; ++gg) {
      // p'_g = p * scale as a bf16 hi + lo pair: the two output MFMAs see
      // hi + lo = p'_g to ~2^-17, so the contraction is FP32-accurate.
      float pg[8];
      float z = zp[gg];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pg[i] = p[i] * scl[gg][i];
        z = fmaf(pg[i], zr[gg][i], z);
      }
      zp[gg] = z;
      uint32_t hv[4], lv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        hv[r] = pack_bf16(pg[2 * r], pg[2 * r + 1]);
        lv[r] = pack_bf16(pg[2 * r] - bf16_lo(hv[r]), pg[2 * r + 1] - bf16_hi(hv[r]));
      }
      const u32x4 Ph = {hv[0], hv[1], hv[2], hv[3]}, Pl = {lv[0], lv[1], lv[2], lv[3]};
      uint32_t dr[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        unpack_word_fast(__builtin_amdgcn_perm(co[2 * r + 1][gg], co[2 * r][gg], perm_sel), dr[r], vbase);
#pragma unroll
      for (int nbl = 0; nbl < 8; ++nbl) {
        const u32x4 bv = {dr[0][nbl], dr[1][nbl], dr[2][nbl], dr[3][nbl]};
        O[gg][nbl] = mfma16x16x32(Ph, bv, O[gg][nbl]);
        O[gg][nbl] = mfma16x16x32(Pl, bv, O[gg][nbl]);
      }
      SP[gg] = mfma16x16x32(Ph, ones, SP[gg]);
      SP[gg] = mfma16x16x32(Pl, ones, SP[gg]);
    }
  };

  // ---- tile loop ---------------------------------------------------------------

  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int gg = 0; gg < GW; ++gg) {
#pragma unroll
      for (int nbl = 0; nbl < 8; ++nbl) O[gg][nbl] = f32x4{0.f, 0.f, 0.f, 0.f};
      SP[gg] = f32x4{0.f, 0.f, 0.f, 0.f};
      zp[gg] = 0.f;
    }
    l_lane = 0.f;
    m_seen = kNoRef;
    if (pass > 0) {
      if (nmine > 0) { lookup(0, ix0); dma(tile0, ix0, tb0); }
      if (nmine > 1) { lookup(1, ix1); dma(tile0 + kPairs, ix1, tb1); }
    }
    if (nmine > 2) lookup(2, ix2);
    // Step k computes the pair's tile k from buffer k % 3. Each wave loads the
    // rows of its own 16 tokens, waits for them itself (the loads issued after
    // those of tile k are the page lookups of tile k + 2 and the loads of tile
    // k + 1, at least kDmaW memory ops, so vmcnt <= kDmaW completes tile k), and
    // reads its partner's rows only after the barrier that follows the
    // partner's own wait. After the barrier it looks up the pages of tile k + 3
    // and loads tile k + 2 into buffer (k + 2) % 3, which both waves finished
    // reading before that barrier.
    constexpr int kDmaW = CLW + RLW + 1;
#define ROLAQ_STEP(KK, CUR, NXT, IXN, IXL)                                         \
    {                                                                              \
      const int kk = (KK);                                                         \
      const bool act = kk < nmine;                                                 \
      if (kk + 1 < nmine)                                                          \
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kDmaW));                              \
      else                                                                         \
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));                                  \
      if (act) phase1(tile0 + kPairs * kk, CUR, pass > 0 || kk > 0);              \
      lds_barrier();                                                               \
      if (kk + 3 < nmine) lookup(kk + 3, IXL);                                     \
      if (kk + 2 < nmine) dma(tile0 + kPairs * (kk + 2), IXN, NXT);                \
      if (act) phase2(CUR, pass == 0 && kk == 0);                                  \
    }
    for (int k = 0; k < kmax; k += 3) {
      ROLAQ_STEP(k, tb0, tb2, ix2, ix0)
      if (k + 1 >= kmax) break;
      ROLAQ_STEP(k + 1, tb1, tb0, ix0, ix1)
      if (k + 2 >= kmax) break;
      ROLAQ_STEP(k + 2, tb2, tb1, ix1, ix2)
    }
#undef ROLAQ_STEP
    // a score above the reference by more than the slack: redo with the true max
    const float m_true = wave_max_over_groups(m_seen);
    if (gq == 0) s_mt[pr][wh][la] = m_true;
    const int redo = __syncthreads_or(pass == 0 && m_true > m_ref + kRefSlack);
    if (!redo) break;
    m_ref = fmaxf(s_mt[pr][0][la], s_mt[pr][1][la]);  // the pair's largest score
  }

  // ---- merge the pairs: unnormalised o, m, l --------------------------------
  const float l_sum = wave_sum_over_groups(l_lane);
#pragma unroll
  for (int gg = 0; gg < GW; ++gg) zp[gg] = wave_sum_over_groups(zp[gg]);
  if (gq == 0) {
    if (wh == 0) s_ml[pr][la][0] = m_ref;
    s_ml[pr][la][1 + wh] = l_sum;
  }
  __syncthreads();  // every wave is done with its tile buffers
  float fac[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int h = 4 * gq + j;
    float M = kNoRef;
#pragma unroll
    for (int w = 0; w < kPairs; ++w) M = fmaxf(M, s_ml[w][h][0]);
    float Ls = 0.f;
#pragma unroll
    for (int w = 0; w < kPairs; ++w) Ls += __builtin_amdgcn_exp2f(s_ml[w][h][0] - M) * (s_ml[w][h][1] + s_ml[w][h][2]);
    fac[j] = Ls > 0.f ? __builtin_amdgcn_exp2f(s_ml[pr][h][0] - M) / Ls : 0.f;
  }
  // this wave's partial o = ((O - 4 SP) 2^(5-e) - ZP) * fac for its groups, in place
#pragma unroll
  for (int gg = 0; gg < GW; ++gg) {
    float spo[4], zpo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      spo[j] = __shfl(SP[gg][j], 16 * gq);
      zpo[j] = __shfl(zp[gg], 4 * gq + j);
    }
#pragma unroll
    for (int nbl = 0; nbl < 8; ++nbl) {
      const float wgt = pair_weight(nbl);
#pragma unroll
      for (int j = 0; j < 4; ++j) O[gg][nbl][j] = ((O[gg][nbl][j] - 4.f * spo[j]) * wgt - zpo[j]) * fac[j];
    }
  }
  // pairs 1 .. kPairs-1 hand their partials to pair 0 through LDS in the
  // accumulator layout (plain stores and loads, no read-modify-write chains);
  // pair 0 adds them in a fixed order (p0 + p1 + p2 + ..). Wave wh of pair pr
  // uses partial slot 2 (pr - 1) + wh: two per ring buffer when they fit.
  constexpr int PBUF = GW * 8 * 64 * 16;                   // bytes of one wave's partial
  constexpr int PER_RING = 2 * PBUF <= RING ? 2 : 1;
  static_assert(PBUF <= RING && 2 * (kPairs - 1) <= 3 * PER_RING, "partial buffers");
  auto pslot = [&](int q) {
    uint8_t* ring = (q / PER_RING) == 0 ? s_r0 : (q / PER_RING) == 1 ? s_r1 : s_r2;
    return reinterpret_cast<f32x4*>(ring + (q % PER_RING) * PBUF);
  };
  auto slot4 = [&](int gg, int nbl) { return (gg * 8 + nbl) * 64 + lane; };
  if (pr > 0) {
    f32x4* xb = pslot(2 * (pr - 1) + wh);
#pragma unroll
    for (int gg = 0; gg < GW; ++gg)
#pragma unroll
      for (int nbl = 0; nbl < 8; ++nbl) xb[slot4(gg, nbl)] = O[gg][nbl];
  }
  __syncthreads();
  if (pr == 0) {
#pragma unroll
    for (int p = 1; p < kPairs; ++p) {
      const f32x4* xb = pslot(2 * (p - 1) + wh);
#pragma unroll
      for (int gg = 0; gg < GW; ++gg)
#pragma unroll
        for (int nbl = 0; nbl < 8; ++nbl) O[gg][nbl] += xb[slot4(gg, nbl)];
    }
  }
  __syncthreads();  // partials consumed: s_r2 / s_r0 take heads 0-7 / 8-15
  auto obuf = [&](int h) { return reinterpret_cast<float*>(h < 8 ? s_r2 : s_r0) + (h & 7) * D; };
  if (pr == 0) {
#pragma unroll
    for (int gg = 0; gg < GW; ++gg) {
      const int g = GW * wh + gg;
#pragma unroll
      for (int nbl = 0; nbl < 8; ++nbl) {
        const int f = 128 * g + 16 * (la >> 1) + 8 * (la & 1) + nbl;
#pragma unroll
        for (int j = 0; j < 4; ++j) obuf(4 * gq + j)[f] = O[gg][nbl][j];
      }
    }
  }
  __syncthreads();
  const int hmax = min(16, a.H - h0);
  for (int e = 4 * tid; e < hmax * D; e += 4 * kThreads) {
    const int h = e / D, f = e % D;
    *reinterpret_cast<f32x4*>(&a.logits[(((int64_t)b * a.H + h0 + h) * a.S1 + split) * D + f]) =
        *reinterpret_cast<const f32x4*>(obuf(h) + f);
  }
  if (tid < hmax) {
    const int h = tid;
    float M = kNoRef;
    for (int w = 0; w < kPairs; ++w) M = fmaxf(M, s_ml[w][h][0]);
    float Ls = 0.f;
    for (int w = 0; w < kPairs; ++w) Ls += __builtin_amdgcn_exp2f(s_ml[w][h][0] - M) * (s_ml[w][h][1] + s_ml[w][h][2]);
    a.lse[((int64_t)b * a.H + h0 + h) * a.S1 + split] = Ls > 0.f ? (M + __log2f(Ls)) * kLn2 : kNeutralLse;
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
  // unrolled so that the loads of several splits are in flight together
  float M = -3.0e38f;
#pragma unroll 8
  for (int s = 0; s <= nq; ++s) M = fmaxf(M, lse[row + s]);
  float acc[FPT], den = 0.f;
#pragma unroll
  for (int i = 0; i < FPT; ++i) acc[i] = 0.f;
#pragma unroll 8
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
                               uint16_t* out, int64_t o_sb, int64_t o_sh, int stages,
                               hipStream_t stream) {
  using namespace rolaq;
  // stage 1: one block per (sequence, 16 heads, split); stage 2: one per (sequence, head)
  const dim3 grid(a.B * ((a.H + 15) / 16), max_splits + 1), block(kThreads);
#define ROLAQ_DEC(DD, RR)                                                                \
  if (D == DD && R == RR) {                                                              \
    if (stages & kStagePartials) {                                                       \
      if (a.page_shift >= 5)                                                             \
        hipLaunchKernelGGL((decode_stage1<DD, RR, true>), grid, block, 0, stream, a);    \
      else                                                                               \
        hipLaunchKernelGGL((decode_stage1<DD, RR, false>), grid, block, 0, stream, a);   \
    }                                                                                    \
    if (stages & kStageMerge)                                                            \
      hipLaunchKernelGGL((decode_stage2<DD>), dim3(a.B * a.H), dim3(128), 0, stream,      \
                         a.logits, a.lse, a.num_kv_splits, a.H, a.S1, out, o_sb, o_sh);  \
    return hipGetLastError();                                                            \
  }
  ROLAQ_DEC(512, 64)
  ROLAQ_DEC(256, 32)
#undef ROLAQ_DEC
  return hipErrorInvalidValue;
}
