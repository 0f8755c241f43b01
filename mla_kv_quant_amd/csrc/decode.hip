// Absorbed MLA decode attention over the packed INT2 cache (gfx950).
//
// Reference behaviour: packed_mla_decode_gf_fwd + _fwd_hp_window_stage1 +
// stage-2 merge of the OSCAR SGLang fork (call site
// deployment/patches/rolaq_sglang.patch:51-111). The cache rows it attends
// over are the reference's stored rows: an INT2 row is
// bf16((code - zero) * scale) in FP32 (mla_quant/oscar.py:144, rounded to the
// model dtype by mla_quant/quantizer.py:120), a window row (first P / last W
// positions) is the BF16 rotated latent (mla_quant/cache.py:1007-1073).
//
// Work split: grid (B * head blocks, max_splits + 1). Block (b, head block,
// split s < nq = max(ns_b - 1, 1)) takes units [U s / nq, U (s+1) / nq) of the
// sequence (bounds rounded up), where unit 0 is the window tile (the <= P + W
// BF16 rows, when there are any) and the others are the 32-token tiles of the
// INT2 positions [P, L - W). Split nq, the reference's window split, carries
// the neutral partial (its rows are folded into split 0); larger s exit.
//
// Each of the 4 waves (one per SIMD) walks its own units (every 4th) with its
// own softmax state, holding the query of HG head groups in registers. Per
// 32-token tile:
//   expansion  a lane owns one (token, quantization group): the four levels
//              bf16((k - zero) * scale), k = 0..3, carried as fp16 (the same
//              numbers: a bf16 value is exact in fp16 between 2^-17 and
//              65504), form a byte table, and two byte permutes per four
//              codes pick the lanes' values, which ARE the reference's stored
//              row (no approximation);
//   scores     S^T[token, head] = K Q^T on fp16 MFMA 16x16x32 with the
//              expanded codes as the A operand in registers and the latent
//              query converted to fp16 once (exact products, FP32
//              accumulate); rope on bf16 MFMA into the same accumulators;
//   softmax    FP32 in the log2 domain against a per-wave reference per head
//              (the first tile's maximum + 8); a tile whose maximum passes it
//              by more than 15 moves it to that maximum + 8 and scales O and
//              the sum by the difference, so every probability is at most
//              2^15;
//   output     O[head, f] += P V on fp16 MFMA (P rounded to fp16: relative
//              error 2^-12 per probability) with V read transposed out of the
//              wave's LDS copy of the expanded tile (ds_read_b64_tr_b16).
// The output contraction of a tile runs inside the next tile's expansion
// (both touch the same LDS elements, old reads before new writes). Loads go
// straight to registers, one tile ahead; the four waves merge their (max,
// sum, O) through LDS into one partial per block.
//
// Range: the latent query, the stored INT2 levels and the window rows are
// carried in fp16, so magnitudes above 65504 become inf and the outputs of
// that request non-finite (never silently wrong); rope terms stay bf16.
#include "rolaq_common.h"
#include "rolaq_args.h"

#include <algorithm>
#include <type_traits>
#include <mutex>

namespace rolaq {

constexpr int kTile = 32;                  // tokens per tile (two 16-row M-blocks)
constexpr int kWaves = 4;                  // one per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kXcds = 8;                   // accelerator dies (own L2 each) of the MI355X
constexpr float kNoRef = -1.0e30f;         // masked score / "no score yet" (log2 units)
constexpr float kRefSlack = 15.f;          // max exp2 argument: a probability stays <= 2^15 (fp16)
constexpr float kRefHeadroom = 8.f;        // a reference sits this far above the maximum it was set from
// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kSchedValu = 0x002, kSchedMfma = 0x008, kSchedDsRead = 0x100, kSchedDsWrite = 0x200;
// s_waitcnt immediate (gfx9 encoding) waiting for lgkmcnt == 0 only
constexpr int kLgkmcnt0 = 0xF | (0x3 << 14) | (0x7 << 4);

template <int D, int R>
struct DGeo {
  static constexpr int NG = D / 128;       // quantization groups
  static constexpr int KL = D / 32;        // latent K-steps of the score MFMA
  static constexpr int KR = R / 32;        // rope K-steps
  static constexpr int CB = D / 16;        // packed code bytes of one lane per token
  static constexpr int CV = CB / 16;       // 16-byte code loads per lane and token
  static constexpr int WPL = CB / 4;       // packed words per lane and token
  static constexpr int ROWB = 2 * D;       // bytes of one expanded row in LDS
  static constexpr int WBUF = kTile * ROWB;  // expanded tile of one wave
  static constexpr int NB = D / 16;        // output N-blocks
  static constexpr int NL = 2 * (CV + 1 + KR);  // vector loads of one tile per lane
};

// ---------------------------------------------------------------------------
// Expanded-row layout in LDS. Lane (la, gq) of the score MFMA at K-step j
// holds 8 fp16 of token la: features feature(gq, j, i), i = 0..7, stored as the
// 16-byte logical chunk 4j + gq of the token's row, so a row's LDS element
// e = 32j + 8gq + i. Physical chunk = logical ^ sw(row): the 8 rows that a
// 16-byte store of 8 lanes touches, and the 4 rows x 2 chunks that a 16-lane
// transposed read touches, land in distinct 16-byte bank groups.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int sw(int row) { return ((row & 3) << 1) | ((row >> 2) & 1); }

// Lane group gq owns quantization group g_of(gq) and its packed words
// s0(gq) .. s0(gq) + WPL - 1 (32 bytes at D = 512, 16 at D = 256).
template <int D>
__device__ __forceinline__ int lane_group(int gq) { return gq * (D / 128) / 4; }
template <int D>
__device__ __forceinline__ int lane_word0(int gq) { return (gq * (D / 64)) % 8; }

// Inside an 8-feature chunk the expansion leaves features in the order
// pi = [0, 4, 1, 5, 2, 6, 3, 7]: dword d of a chunk = (feature d, feature d + 4).
// The query operand is permuted the same way.
__device__ __forceinline__ u32x4 pi_permute(u32x4 n) {
  return u32x4{__builtin_amdgcn_perm(n.z, n.x, 0x05040100u), __builtin_amdgcn_perm(n.z, n.x, 0x07060302u),
               __builtin_amdgcn_perm(n.w, n.y, 0x05040100u), __builtin_amdgcn_perm(n.w, n.y, 0x07060302u)};
}

// Byte tables of the four stored levels v_k = bf16((k - zero) * scale), as
// fp16: L = low bytes of v_0..v_3, H = high bytes. A masked token gets zeros.
struct Lut {
  uint32_t L, H;
};
__device__ __forceinline__ Lut make_lut(f32x2 sz, bool live) {
  const float s = sz.x, z = sz.y;
  const uint32_t A = bf16x2_to_f16x2(pack_bf16((0.0f - z) * s, (1.0f - z) * s));
  const uint32_t B = bf16x2_to_f16x2(pack_bf16((2.0f - z) * s, (3.0f - z) * s));
  Lut t;
  t.L = live ? __builtin_amdgcn_perm(B, A, 0x06040200u) : 0u;
  t.H = live ? __builtin_amdgcn_perm(B, A, 0x07050301u) : 0u;
  return t;
}

// One packed word (16 codes, code p at bits 2p) -> two 16-byte chunks of
// 16-bit values: c0 = features [0,4,1,5,2,6,3,7], c1 = 8 + the same. x_p
// selects, per byte, the codes p, p+4, p+8, p+12; a permute with the code
// bytes as selectors reads the tables; two more interleave low and high bytes
// into value pairs.
__device__ __forceinline__ void expand_word(uint32_t w, const Lut& t, u32x4& c0, u32x4& c1) {
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t x = (w >> (2 * p)) & 0x03030303u;
    lo[p] = __builtin_amdgcn_perm(t.H, t.L, x);
    hi[p] = __builtin_amdgcn_perm(t.L, t.H, x);
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    c0[p] = __builtin_amdgcn_perm(hi[p], lo[p], 0x05010400u);
    c1[p] = __builtin_amdgcn_perm(hi[p], lo[p], 0x07030602u);
  }
}

__device__ __forceinline__ void lds_store128(uint8_t* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x4 lds_load128(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// 64 bits of the output MFMA's B operand, read transposed out of the expanded
// rows (ds_read_b64_tr_b16: within each 16-lane group, lane 4s + e receives
// element e of the 8-byte chunks addressed by lanes s, s+4, s+8, s+12). Lane
// (gq, la) addresses row 16h + 4gq + (la >> 2) at elements 16nb + 4(la & 3),
// so it receives rows 16h + 4gq + 0..3 of element 16nb + la.
template <int ROWB>
__device__ __forceinline__ u32x2 read_vt(const uint8_t* buf, int gq, int la, int nb, int h) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int row = 16 * h + 4 * gq + (la >> 2);
  const int e = 16 * nb + 4 * (la & 3);
  const uint8_t* p = buf + row * ROWB + 16 * ((e >> 3) ^ sw(row)) + 2 * (e & 7);
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p)));
}

template <int D, int R>
struct TileRegs {
  u32x4 code[2][DGeo<D, R>::CV];  // packed words of the lane's group, M-blocks 0 / 1
  f32x2 prm[2];                   // (scale, zero) of the lane's group
  u32x4 rope[2][DGeo<D, R>::KR];  // rope A operands
};

// Partial with no keys: logits 0, LSE -1e4 (SGLang's empty-split convention).
__device__ void write_neutral(const DecodeArgs& a, int b, int h0, int nh, int split, int D) {
  for (int e = threadIdx.x; e < nh * D / 4; e += blockDim.x) {
    const int h = e / (D / 4), f = 4 * (e % (D / 4));
    *reinterpret_cast<f32x4*>(&a.logits[(((int64_t)b * a.H + h0 + h) * a.S1 + split) * D + f]) =
        f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if ((int)threadIdx.x < nh) a.lse[((int64_t)b * a.H + h0 + threadIdx.x) * a.S1 + split] = kNeutralLse;
}

// ---------------------------------------------------------------------------
// Stage 1. HG head groups of 16 per block (their query operands and output
// accumulators live in one wave); D = 512 uses HG = 1.
// ---------------------------------------------------------------------------
template <int D, int R, int HG>
__global__ __launch_bounds__(kThreads, 1) void decode_stage1(DecodeArgs a) {
  using G = DGeo<D, R>;
  constexpr int KL = G::KL, KR = G::KR, CB = G::CB, CV = G::CV, WPL = G::WPL, ROWB = G::ROWB, NB = G::NB;
  constexpr int NG = G::NG;
  static_assert(R % 32 == 0 && D % 256 == 0, "unsupported shape");
  static_assert(16 * D * 4 <= G::WBUF, "merge buffer of one wave (one head group at a time)");

  define_acc_macros();
  __shared__ __attribute__((aligned(16))) uint8_t s_buf[kWaves * G::WBUF];
  __shared__ float s_m[kWaves][HG][16];  // per wave: softmax reference of each head
  __shared__ float s_l[kWaves][HG][16];  // per wave: sum of exponentials of each head

  // Every argument the prologue reads, fetched in one batch of scalar loads
  // (left to itself the compiler issues each where it is first used: one
  // dependent round trip per use at kernel start).
  asm volatile("" ::"s"(a.q), "s"(a.q_sb), "s"(a.q_sh), "s"(a.codes), "s"(a.params), "s"(a.rope), "s"(a.hp),
               "s"(a.kv_indptr), "s"(a.kv_indices), "s"(a.page_shift), "s"(a.seq_lens), "s"(a.req_idx),
               "s"(a.num_kv_splits), "s"(a.split_cap), "s"(a.S1), "s"(a.max_reqs), "s"(a.H), "s"(a.P),
               "s"(a.W), "s"(a.sm_scale), "s"(gridDim.x), "s"(gridDim.y));

  // ---- which (sequence, head block, split) ------------------------------------
  const int nhb = ((a.H + 15) / 16 + HG - 1) / HG;
  // Head blocks of one (sequence, split) read the same rows: with more than one,
  // the blocks are renumbered so that they take consecutive dispatch slots of
  // one XCD (the dispatcher deals linear block ids to the 8 XCDs round-robin)
  // and the later ones read the rows from that XCD's L2.
  int lin = blockIdx.x + gridDim.x * blockIdx.y;
  const int nblk = gridDim.x * gridDim.y;
  if (nhb > 1 && nblk % kXcds == 0) lin = (lin % kXcds) * (nblk / kXcds) + lin / kXcds;
  const int hb = nhb > 1 ? lin % nhb : 0;
  const int split = nhb > 1 ? (lin / nhb) % (int)gridDim.y : (int)blockIdx.y;
  const int b = nhb > 1 ? (lin / nhb) / (int)gridDim.y : (int)blockIdx.x;
  const int h0 = 16 * HG * hb;
  const int nh = min(16 * HG, a.H - h0);  // heads of this block
  const int tid = threadIdx.x, lane = tid & 63, la = lane & 15, gq = lane >> 4;
  const int gl = lane_group<D>(gq), s0 = lane_word0<D>(gq);

  // The sequence's metadata: five loads issued together and waited for once
  // (the split test below would otherwise wait for its own load first), then
  // the query's loads, which the first tile needs only after two more round
  // trips (page lookups, tile data).
  const int ns_req = a.num_kv_splits[b];
  const int kv0 = a.kv_indptr[b], kv1 = a.kv_indptr[b + 1];
  const int64_t req = a.req_idx[b];
  const int64_t slv = (a.seq_lens ? a.seq_lens : a.req_idx)[b];  // no branch before the loads
  u32x4 qB[HG][KL], qR[HG][KR];
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
    const uint16_t* qh = a.q + b * a.q_sb + (int64_t)min(h0 + 16 * hg + la, a.H - 1) * a.q_sh;
#pragma unroll
    for (int j = 0; j < KL; ++j) qB[hg][j] = gload<u32x4>(qh + 128 * gl + 16 * (s0 + j / 2) + 8 * (j & 1));
#pragma unroll
    for (int kr = 0; kr < KR; ++kr) qR[hg][kr] = gload<u32x4>(qh + D + 32 * kr + 8 * gq);
  }
  asm volatile("" ::"v"(ns_req), "v"(kv0), "v"(kv1), "v"(req), "v"(slv));
  const int ns = min(ns_req, a.split_cap);
  const int L = a.seq_lens ? (int)slv : kv1 - kv0;
  const int nq = min(max(ns - 1, 1), a.S1 - 1);
  if (split > nq) return;
  if (split == nq) {
    if (a.neutral) write_neutral(a, b, h0, nh, split, D);
    return;
  }

  // a request without ring rows (index outside [0, max_reqs)) has no window:
  // the writer stored none for it, so every position is read from its codes
  const bool has_ring = req >= 0 && req < a.max_reqs;
  const int P = has_ring ? a.P : 0, W = has_ring ? a.W : 0;
  const int lo = min(P, L), hi = max(L - W, lo);          // INT2 positions [lo, hi)
  const int n_sink = lo, rec_lo = max(L - W, n_sink);
  const int nw = n_sink + (L - rec_lo);                    // window rows
  const int t_first = lo / kTile;
  const int ntiles = hi > lo ? (hi + kTile - 1) / kTile - t_first : 0;
  const int has_win = nw > 0 ? 1 : 0;
  const int U = ntiles + has_win;
  // ceil(U s / nq): unit 0 (the window) always goes to split 0 (32-bit
  // division whenever U (s + 1) + nq fits, as it does below 2^27 tokens)
  const uint64_t num_b = (uint64_t)U * split + nq - 1, num_e = (uint64_t)U * (split + 1) + nq - 1;
  const bool narrow = num_e < (1ull << 32);
  const int ub = narrow ? (int)((uint32_t)num_b / (uint32_t)nq) : (int)(num_b / nq);
  const int ue = narrow ? (int)((uint32_t)num_e / (uint32_t)nq) : (int)(num_e / nq);
  const bool win_block = has_win && ub == 0 && ue > 0;  // this block holds unit 0

  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool win_mine = win_block && wave == 0;
  // INT2 units of this wave: u0, u0 + 4, ... below ue
  int u0 = ub + wave;
  if (u0 < has_win) u0 += kWaves;
  const int n = u0 < ue ? (ue - u0 + kWaves - 1) / kWaves : 0;
  const int T0 = t_first + u0 - has_win;  // tile of INT2 unit i: T0 + 4i

  const int pmask = (1 << a.page_shift) - 1;
  uint8_t* const wbuf = s_buf + wave * G::WBUF;
  const float sl2 = a.sm_scale * kLog2e;

  // ---- per-wave softmax state and accumulators ----------------------------------
  f32x4 O[HG][NB];
  float m_ref[HG], l_lane[HG];

  // page of a position; an empty sequence reads its kv_indptr entry instead
  // (a valid address; its result is not used)
  auto page_of = [&](int pos) {
    return gload<int32_t>(L > 0 ? a.kv_indices + kv0 + (pos >> a.page_shift) : a.kv_indptr + b);
  };
  auto lookup = [&](int i, int32_t (&pg)[2]) {
    const int base = kTile * (T0 + kWaves * i);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) pg[mb] = page_of(min(base + 16 * mb + la, L - 1));
  };
  auto load = [&](int i, const int32_t (&pg)[2], TileRegs<D, R>& d) {
    const int base = kTile * (T0 + kWaves * i);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int pos = min(base + 16 * mb + la, L - 1);
      const uint32_t page = L > 0 ? (uint32_t)pg[mb] : 0u;  // empty sequence: slot 0's row, unused
      const uint64_t slot = ((uint64_t)page << a.page_shift) + (uint32_t)(pos & pmask);
#pragma unroll
      for (int v = 0; v < CV; ++v) d.code[mb][v] = gload<u32x4>(a.codes + slot * (D / 4) + CB * gq + 16 * v);
      d.prm[mb] = gload<f32x2>(a.params + slot * (2 * NG) + 2 * gl);
#pragma unroll
      for (int kr = 0; kr < KR; ++kr) d.rope[mb][kr] = gload<u32x4>(a.rope + slot * R + 32 * kr + 8 * gq);
    }
  };

  // The window tile's loads (wave 0 of the block holding unit 0), issued in
  // its prologue.
  auto win_pos = [&](int i) { return i < n_sink ? i : rec_lo + (i - n_sink); };
  u32x4 wc[2][KL], wr[2][KR];
  int32_t wpg[2];
  auto window_pages = [&]() {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) wpg[mb] = page_of(win_pos(min(16 * mb + la, nw - 1)));
  };
  auto window_rows = [&]() {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int pos = win_pos(min(16 * mb + la, nw - 1));
      const int inner = pos < P ? pos : P + (pos - P) % max(W, 1);
      const uint16_t* row = a.hp + (1 + req * (P + W) + inner) * D + 128 * gl + 16 * s0;
#pragma unroll
      for (int j = 0; j < KL; ++j) wc[mb][j] = gload<u32x4>(row + 16 * (j / 2) + 8 * (j & 1));
    }
  };
  auto window_rope = [&]() {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int pos = win_pos(min(16 * mb + la, nw - 1));
      const int64_t slot = ((int64_t)wpg[mb] << a.page_shift) + (pos & pmask);
#pragma unroll
      for (int kr = 0; kr < KR; ++kr) wr[mb][kr] = gload<u32x4>(a.rope + slot * R + 32 * kr + 8 * gq);
    }
  };
  TileRegs<D, R> dc, dn;  // the two tile register slots
  int32_t pgc[2], pgn[2];  // their pages
  const int nl = max(n - 1, 0);
  u32x4 Ph[HG];  // the pending tile's probabilities (fp16)

  // The output contraction of a tile runs during the next tile's expansion:
  // word step s of tile i + 1 first reads tile i's V^T for N-blocks 4s..4s+3
  // (LDS elements 64s..64s+63), then writes its own expanded chunks to those
  // same elements (LDS executes one wave's operations in order), so one buffer
  // per wave suffices and the reads' latency and the output MFMAs overlap the
  // expansion's VALU work. Ph holds the pending tile's probabilities; at
  // the start they are zero and the buffer holds zeros, so the first step's
  // contraction adds exactly 0.

  // Probabilities are 2^(score - reference) against a per-wave, per-head
  // reference: the first tile's maximum + 8. A tile whose scores pass the
  // reference by more than 15 (a probability would not fit fp16) moves the
  // reference of those heads to its maximum + 8 and scales O and the sum by
  // the difference, in place, before its probabilities are formed. The
  // pending tile's output is already in O (its MFMAs ran inside this tile's
  // steps). O is held transposed: lane (la, gq) holds head la, the head
  // whose scores and sum it holds, so its factor is its own.
  auto rescale = [&](const float (&mx)[HG], const uint64_t (&need)[HG]) {
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
      float f = 1.f;
      if (__builtin_expect(need[hg] != 0, 0)) {
        const float mt = wave_max_over_groups(mx[hg]);
        const float mn = mt > m_ref[hg] + kRefSlack ? mt + kRefHeadroom : m_ref[hg];
        f = __builtin_amdgcn_exp2f(m_ref[hg] - mn);  // 0 when nothing was summed yet
        l_lane[hg] *= f;
        m_ref[hg] = mn;
      }
      const float fj[4] = {f, f, f, f};
      static_assert(NB % 16 == 0, "rescale in groups of 16 N-blocks");
#pragma unroll
      for (int nb = 0; nb < NB; nb += 16)
        scale_acc16(*reinterpret_cast<f32x4(*)[16]>(&O[hg][nb]), fj, need[hg]);
    }
  };
  // the scores of one tile in log2 units, masked by the validity of token
  // 16 mb + 4 gq + r
  auto masked = [&](const f32x4 (&S)[2][HG], auto valid, float (&x)[HG][8]) {
#pragma unroll
    for (int hg = 0; hg < HG; ++hg)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          x[hg][4 * mb + r] = valid(16 * mb + 4 * gq + r) ? S[mb][hg][r] * sl2 : kNoRef;
  };
  // softmax of one tile's masked scores into Ph; the first tile of a wave sets
  // the reference (nothing is summed yet). One instance per tile, so that O
  // passes through one rescale on every path.
  // (rescaling: std::true_type, or std::false_type for a wave's first unit,
  // which never rescales, so that O is not touched on that path)
  auto softmax_impl = [&](const float (&x)[HG][8], bool first, auto rescaling) {
    float mx[HG];
    uint64_t need[HG];  // per head group: lanes past the slack
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
      mx[hg] = x[hg][0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mx[hg] = fmaxf(mx[hg], x[hg][i]);
      need[hg] = __builtin_amdgcn_ballot_w64(!first && mx[hg] > m_ref[hg] + kRefSlack);
    }
    if (__builtin_expect(first, 0)) {
#pragma unroll
      for (int hg = 0; hg < HG; ++hg) m_ref[hg] = wave_max_over_groups(mx[hg]) + kRefHeadroom;
    }
    if constexpr (decltype(rescaling)::value) rescale(mx, need);
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = __builtin_amdgcn_exp2f(x[hg][i] - m_ref[hg]);  // masked: 2^-1e30 = 0
#pragma unroll
      for (int d = 0; d < 4; ++d) Ph[hg][d] = pack_f16(p[2 * d], p[2 * d + 1]);
      // the sum of the fp16 probabilities the output MFMA uses
#pragma unroll
      for (int d = 0; d < 4; ++d) l_lane[hg] = sum_f16x2(Ph[hg][d], l_lane[hg]);
    }
  };
  auto softmax = [&](const float (&x)[HG][8], bool first) { softmax_impl(x, first, std::true_type{}); };
  // O^T[element, head] += V^T P^T: the V^T rows as the A operand, the
  // probabilities (P[head la][tokens 8 gq + i]) as the B operand, so lane
  // (la, gq) accumulates head la at elements 16 nb + 4 gq + j
  auto out_nb = [&](int nb, u32x2 v0, u32x2 v1) {
    const u32x4 vt = {v0.x, v0.y, v1.x, v1.y};
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) O[hg][nb] = mfma16x16x32_f16(vt, Ph[hg], O[hg][nb]);
  };
  // LDS addresses as a few per-lane bases plus immediate offsets. The swizzle
  // only touches the low 3 bits of a 16-byte chunk index, so
  //   store of K-step j, M-block mb:  wb[mb][j & 1] + 128 (j >> 1)
  //   V^T read of N-block nb, half h: rb[nb & 3] + 128 (nb >> 2) + 16 ROWB h
  // (read_vt's address, regrouped).
  uint8_t* wb[2][2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
      const int row = 16 * mb + la;
      wb[mb][jp] = wbuf + row * ROWB + 16 * ((4 * jp + gq) ^ sw(row));
    }
  const uint8_t* rb[4];
  {
    const int row = 4 * gq + (la >> 2), sig = (la & 3) >> 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) rb[q] = wbuf + row * ROWB + 16 * ((2 * q + sig) ^ sw(row)) + 8 * (la & 1);
  }
  auto vt_read = [&](int nb, int h) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const uint8_t* p = rb[nb & 3] + 128 * (nb >> 2) + 16 * ROWB * h;
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p)));
  };
  // the pending tile's output alone (after a wave's last tile)
  auto flush = [&]() {
    __builtin_amdgcn_s_waitcnt(kLgkmcnt0);  // the last tile's stores have landed
    asm volatile("" ::: "memory");
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) out_nb(nb, vt_read(nb, 0), vt_read(nb, 1));
  };

  // INT2 tile i: expand, score, write the rows (with the pending tile's
  // output interleaved), then its softmax becomes the pending one
  auto compute = [&](int i, const TileRegs<D, R>& d, bool first) {
    const int base = kTile * (T0 + kWaves * i);
    // rope scores first (their operands are then free), then the latent
    // K-steps; with one head group, even and odd K-steps accumulate apart (two
    // independent MFMA chains per M-block), summed before the softmax
    f32x4 S[2][HG], S2[2][HG];
    f32x4 (&So)[2][HG] = HG == 1 ? S2 : S;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int hg = 0; hg < HG; ++hg) {
        S[mb][hg] = f32x4{0.f, 0.f, 0.f, 0.f};
        S2[mb][hg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kr = 0; kr < KR; ++kr) S[mb][hg] = mfma16x16x32(d.rope[mb][kr], qR[hg][kr], S[mb][hg]);
      }
    Lut t[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int pos = base + 16 * mb + la;
      t[mb] = make_lut(d.prm[mb], pos >= lo && pos < hi);
    }
    // Word step s: the expansion of step s, the output MFMAs of step s on the
    // reads issued PFD steps earlier, the reads of step s + PFD, its score
    // MFMAs, then the stores of step s. Step s stores over the elements its
    // reads came from; the LDS runs a wave's instructions in order, so those
    // reads (issued earlier) have their data before the stores land, and the
    // only waits are the compiler's, for the read registers. The scheduling
    // groups interleave the output MFMAs with the expansion's VALU work, so
    // the matrix core runs while the VALU expands. Reads two steps ahead give
    // them a whole step of cover (one step with three head groups, whose
    // registers are full).
    constexpr int PFD = HG >= 3 ? 1 : 2;  // steps the transposed reads run ahead
    u32x2 vr[PFD + 1][4][2];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        vr[0][k][h] = vt_read(k, h);
        if (PFD > 1 && WPL > 1) vr[1][k][h] = vt_read(4 + k, h);
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < WPL; ++s) {
      u32x2 (&cur)[4][2] = vr[s % (PFD + 1)];
      u32x2 (&nxt)[4][2] = vr[(s + PFD) % (PFD + 1)];
      asm volatile("" ::: "memory");
      u32x4 c[2][2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) expand_word(d.code[mb][s / 4][s % 4], t[mb], c[mb][0], c[mb][1]);
#pragma unroll
      for (int k = 0; k < 4; ++k) out_nb(4 * s + k, cur[k][0], cur[k][1]);
      if (s + PFD < WPL) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int h = 0; h < 2; ++h) nxt[k][h] = vt_read(4 * (s + PFD) + k, h);
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        lds_store128(wb[mb][0] + 128 * s, c[mb][0]);  // K-step 2s
        lds_store128(wb[mb][1] + 128 * s, c[mb][1]);  // K-step 2s + 1
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int hg = 0; hg < HG; ++hg) {
          S[mb][hg] = mfma16x16x32_f16(c[mb][0], qB[hg][2 * s], S[mb][hg]);
          So[mb][hg] = mfma16x16x32_f16(c[mb][1], qB[hg][2 * s + 1], So[mb][hg]);
        }
      // issue order: (10 VALU, HG output MFMAs) x 4, the rest of the VALU,
      // the transposed reads of step s + PFD, then (HG score MFMAs, a store) x 4
      // (the reads go out ahead of the stores: the LDS runs a wave's
      // operations in order, so reads behind 4 KB of stores would wait for
      // them; their elements are not the ones this step stores)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        __builtin_amdgcn_sched_group_barrier(kSchedValu, 10, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, HG, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 64, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8, 0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, HG, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsWrite, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (HG == 1) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) S[mb][0] += S2[mb][0];
    }
    float x[HG][8];
    if (__builtin_expect(base >= lo && base + kTile <= hi, 1))  // an interior tile: every token is an INT2 one
      masked(S, [](int) { return true; }, x);
    else
      masked(S, [&](int tok) { return base + tok >= lo && base + tok < hi; }, x);
    softmax(x, first);
  };

  // window tile: rows 0 .. nw-1 are positions [0, n_sink) U [rec_lo, L), the
  // ring rows of hp_c (BF16, carried as fp16). Wave 0 alone loads them in the
  // score operand's layout, scores them and stores them into its buffer in the
  // expanded layout, where the next tile's steps contract them like an INT2
  // tile (it is always wave 0's first unit: no output is pending before it).
  auto window_tile = [&]() {
    f32x4 S[2][HG];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int i = 16 * mb + la;
#pragma unroll
      for (int hg = 0; hg < HG; ++hg) S[mb][hg] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint32_t keep = keep_mask(i < nw);  // bit masks, not selects: no branch per K-step
#pragma unroll
      for (int kr = 0; kr < KR; ++kr) {
        const u32x4 v = wr[mb][kr] & keep;
#pragma unroll
        for (int hg = 0; hg < HG; ++hg) S[mb][hg] = mfma16x16x32(v, qR[hg][kr], S[mb][hg]);
      }
#pragma unroll
      for (int j = 0; j < KL; ++j) {
        const u32x4 v = bf16x8_to_f16x8(pi_permute(wc[mb][j])) & keep;
        lds_store128(wb[mb][j & 1] + 128 * (j >> 1), v);  // K-step j of row 16 mb + la
#pragma unroll
        for (int hg = 0; hg < HG; ++hg) S[mb][hg] = mfma16x16x32_f16(v, qB[hg][j], S[mb][hg]);
      }
    }
    float x[HG][8];
    masked(S, [&](int tok) { return tok < nw; }, x);
    softmax(x, true);  // always the wave's first unit
  };

  // ---- prologue: the first tiles' pages (the query is in flight already), -----
  // the buffer, state and query set-up while they travel, then the first
  // tile's loads. Every wave issues the same loads up to there (a wave with no
  // tile reads a clamped position's page and row and ignores them): the
  // compiler's counted waits after a join take the path with the fewest loads
  // in flight, so a conditional load would make the common code wait for
  // later loads too. The wave that computes the window tile (wave 0 of the
  // block holding unit 0) has a prologue of its own: the window's ring rows go
  // out with the page lookups, its rope rows ahead of the first tile's loads,
  // and the window tile is computed before the paths join, where the loads
  // in flight are the same (the first tile's) on both.
  auto setup = [&]() {
    // this wave's buffer starts as zeros (see the pending-output rule below),
    // the softmax state, and the query operands (their loads went out with
    // the metadata, ahead of the page lookups)
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) O[hg][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
      m_ref[hg] = kNoRef;
      l_lane[hg] = 0.f;
      Ph[hg] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int k = 0; k < G::WBUF / 1024; ++k) lds_store128(wbuf + 1024 * k + 16 * lane, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
      const bool hv = h0 + 16 * hg + la < a.H;
#pragma unroll
      for (int j = 0; j < KL; ++j) qB[hg][j] = bf16x8_to_f16x8(pi_permute(qB[hg][j])) & keep_mask(hv);
#pragma unroll
      for (int kr = 0; kr < KR; ++kr) qR[hg][kr] &= keep_mask(hv);
    }
    // (kept here: left alone, the compiler sinks the conversion to its first
    // use, past the loads that follow, where it would wait for them)
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
      for (int j = 0; j < KL; ++j) asm volatile("" : "+v"(qB[hg][j])::"memory");
#pragma unroll
      for (int kr = 0; kr < KR; ++kr) asm volatile("" : "+v"(qR[hg][kr])::"memory");
    }
  };
  bool first = true;
  if (win_mine) {
    lookup(0, pgc);
    lookup(min(1, nl), pgn);
    window_pages();
    window_rows();
    __builtin_amdgcn_sched_barrier(0);
    setup();
    __builtin_amdgcn_sched_barrier(0);
    window_rope();
    load(0, pgc, dn);
    __builtin_amdgcn_sched_barrier(0);
    window_tile();
    first = false;
  } else {
    lookup(0, pgc);
    lookup(min(1, nl), pgn);
    __builtin_amdgcn_sched_barrier(0);
    setup();
    __builtin_amdgcn_sched_barrier(0);
    load(0, pgc, dn);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- the wave's units ------------------------------------------------------------
  // Tile pipeline: two register slots (dn, dc) take turns, unrolled by two so
  // that no tile is copied between them: tile i + 1's data is loaded into one
  // slot while tile i is computed from the other, and the pages are looked up
  // a tile before that (the first tile is already in flight from the
  // prologue). Four independent waves per CU keep enough bytes in flight with
  // one tile of prefetch each. The scheduling barriers keep the issue order,
  // so the compiler's counted waits release tile i while tile i + 1's loads
  // are in flight.
  int i = 0;
  for (; i + 1 < n; i += 2) {
    // tile i is in dn: load tile i + 1 into dc, compute tile i
    pgc[0] = pgn[0];
    pgc[1] = pgn[1];
    __builtin_amdgcn_sched_barrier(0);
    load(i + 1, pgc, dc);
    __builtin_amdgcn_sched_barrier(0);
    lookup(min(i + 2, nl), pgn);
    __builtin_amdgcn_sched_barrier(0);
    compute(i, dn, first);
    first = false;
    // tile i + 1 is in dc: load tile i + 2 into dn, compute tile i + 1
    pgc[0] = pgn[0];
    pgc[1] = pgn[1];
    __builtin_amdgcn_sched_barrier(0);
    load(min(i + 2, nl), pgc, dn);
    __builtin_amdgcn_sched_barrier(0);
    lookup(min(i + 3, nl), pgn);
    __builtin_amdgcn_sched_barrier(0);
    compute(i + 1, dc, false);
  }
  if (i < n) compute(i, dn, first);  // the last tile (odd count), already in dn
  flush();

  // ---- merge the four waves: one partial per block ------------------------------
  float l_sum[HG];
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
    l_sum[hg] = wave_sum_over_groups(l_lane[hg]);
    if (gq == 0) {
      s_m[wave][hg][la] = m_ref[hg];
      s_l[wave][hg][la] = l_sum[hg];
    }
  }
  // Each wave stores its raw O^T (weighted in the sum below) into its own
  // buffer as head rows of D elements in LDS element order, 16-byte chunk c
  // of row h at chunk c ^ s(c) ^ h, s(c) = bits 4, 6, 5 of c moved to bits
  // 0, 1, 2 (only the low 4 bits change, so a chunk stays in its row): the
  // 16 lanes of one lane group (rows 0..15, one c) write 16 distinct bank
  // groups, and the 16 threads of one head in the sum read 16 distinct ones.
  // No barrier before the stores: each wave's buffer is its own until the
  // sum, and its own reads of it are done.
  auto mchunk = [](int c, int h) { return c ^ (((c >> 4) & 1) | ((c >> 5) & 2) | ((c >> 3) & 4)) ^ h; };
  float* const mbuf = reinterpret_cast<float*>(wbuf);
  // thread (h, tt) of the sum: head h, octets (K-step j, lane group gq') with
  // j = tt % KL, gq' = (16 / KL) k + tt / KL; consecutive tt write consecutive
  // features (an octet of LDS elements is 8 consecutive features in pi order)
  const int mh = tid >> 4, tt = tid & 15;
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      *reinterpret_cast<f32x4*>(mbuf + la * D + 4 * mchunk(4 * nb + gq, la)) = O[hg][nb];
    __syncthreads();
    float M = kNoRef, Ls = 0.f, wt[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][hg][mh]);
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      wt[w] = __builtin_amdgcn_exp2f(s_m[w][hg][mh] - M);
      Ls += wt[w] * s_l[w][hg][mh];
    }
    const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wt[w] *= inv;
    const int hh = 16 * hg + mh;
    // every read first (all independent), then the weighted sums
    f32x4 part[KL / 4][kWaves][2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < KL / 4; ++k) {
      const int j = tt % KL, gqo = (16 / KL) * k + tt / KL, oct = 4 * j + gqo;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float* src = reinterpret_cast<const float*>(s_buf + w * G::WBUF) + mh * D;
        part[k][w][0] = *reinterpret_cast<const f32x4*>(src + 4 * mchunk(2 * oct, mh));
        part[k][w][1] = *reinterpret_cast<const f32x4*>(src + 4 * mchunk(2 * oct + 1, mh));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x4 lo4[KL / 4], hi4[KL / 4];
#pragma unroll
    for (int k = 0; k < KL / 4; ++k) {
      lo4[k] = part[k][0][0] * wt[0];
      hi4[k] = part[k][0][1] * wt[0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) {
        lo4[k] += part[k][w][0] * wt[w];
        hi4[k] += part[k][w][1] * wt[w];
      }
    }
    if (hh < nh) {
      float* const row = a.logits + (((int64_t)b * a.H + h0 + hh) * a.S1 + split) * D;
#pragma unroll
      for (int k = 0; k < KL / 4; ++k) {
        const int j = tt % KL, gqo = (16 / KL) * k + tt / KL;
        const int f0 = 128 * lane_group<D>(gqo) + 16 * (lane_word0<D>(gqo) + j / 2) + 8 * (j & 1);
        // elements [0..7] of an octet hold features [0, 4, 1, 5, 2, 6, 3, 7]
        *reinterpret_cast<f32x4*>(row + f0) = f32x4{lo4[k][0], lo4[k][2], hi4[k][0], hi4[k][2]};
        *reinterpret_cast<f32x4*>(row + f0 + 4) = f32x4{lo4[k][1], lo4[k][3], hi4[k][1], hi4[k][3]};
      }
      if (tt == 0)
        a.lse[((int64_t)b * a.H + h0 + hh) * a.S1 + split] = Ls > 0.f ? (M + __log2f(Ls)) * kLn2 : kNeutralLse;
    }
    if (hg + 1 < HG) __syncthreads();  // before the next head group reuses the buffers
  }
}

// ---------------------------------------------------------------------------
// Stage 2: LSE merge of the partials -> bf16 output: the nq quantized splits'
// partials and, when stage 1 wrote it (neutral = 1), the window split's
// neutral one. The LSEs and partials of up to kBatch splits are loaded
// together (one round trip after the split count), then merged online.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(128) void decode_stage2(const float* __restrict__ logits,
                                                     const float* __restrict__ lse,
                                                     const int32_t* __restrict__ num_kv_splits,
                                                     int split_cap, int neutral, int H, int S1, uint16_t* out,
                                                     int64_t o_sb, int64_t o_sh) {
  constexpr int FPT = D / 128;
  constexpr int kBatch = 16;
  typedef float fv __attribute__((ext_vector_type(FPT)));
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int nq = min(max(min(num_kv_splits[b], split_cap) - 1, 1), S1 - 1);
  const int np = nq + neutral;  // partials to merge (1 <= np <= S1)
  const int64_t row = ((int64_t)b * H + h) * S1;
  float M = -3.0e38f, den = 0.f;
  fv acc = {};
  for (int s0 = 0; s0 < np; s0 += kBatch) {
    float ls[kBatch];
    fv v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int s = min(s0 + i, np - 1);
      ls[i] = lse[row + s];
      v[i] = *reinterpret_cast<const fv*>(logits + (row + s) * D + threadIdx.x * FPT);
    }
    float mb = M;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) mb = s0 + i < np ? fmaxf(mb, ls[i]) : mb;
    const float c = __builtin_amdgcn_exp2f((M - mb) * kLog2e);  // 0 on the first batch
    den *= c;
    acc *= c;
    M = mb;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const float w = s0 + i < np ? __builtin_amdgcn_exp2f((ls[i] - M) * kLog2e) : 0.f;
      den += w;
      acc += w * v[i];
    }
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
static int rolaq_decode_head_groups(int D, int H) {
  const int nhg = (H + 15) / 16;
  return D == 512 ? 1 : (nhg < 3 ? nhg : 3);
}

int rolaq_decode_head_blocks(int D, int H) {
  const int HG = rolaq_decode_head_groups(D, H);
  return ((H + 15) / 16 + HG - 1) / HG;
}

hipError_t rolaq_launch_decode(const rolaq::DecodeArgs& a, int D, int R, int max_splits,
                               uint16_t* out, int64_t o_sb, int64_t o_sh, int stages,
                               hipStream_t stream) {
  using namespace rolaq;
  const int HG = rolaq_decode_head_groups(D, a.H);
  const int nhb = ((a.H + 15) / 16 + HG - 1) / HG;
  // split rows 0 .. nq, nq = min(max(min(ns, cap) - 1, 1), max_splits): the
  // quantized splits, then (neutral = 1) the window split's neutral partial
  const int nq_max = std::max(std::min(a.split_cap - 1, max_splits), 1);
  const int rows = nq_max + (a.neutral ? 1 : 0);
  const dim3 grid(a.B * nhb, rows), block(kThreads);
#define ROLAQ_S1(DD, RR, GG) \
  if (D == DD && R == RR && HG == GG) hipLaunchKernelGGL((decode_stage1<DD, RR, GG>), grid, block, 0, stream, a);
  if (stages & kStagePartials) {
    ROLAQ_S1(512, 64, 1)
    else ROLAQ_S1(256, 32, 1)
    else ROLAQ_S1(256, 32, 2)
    else ROLAQ_S1(256, 32, 3)
    else return hipErrorInvalidValue;
  }
#undef ROLAQ_S1
  if (stages & kStageMerge) {
    if (D == 512)
      hipLaunchKernelGGL((decode_stage2<512>), dim3(a.B * a.H), dim3(128), 0, stream, a.logits, a.lse,
                         a.num_kv_splits, a.split_cap, a.neutral, a.H, a.S1, out, o_sb, o_sh);
    else if (D == 256)
      hipLaunchKernelGGL((decode_stage2<256>), dim3(a.B * a.H), dim3(128), 0, stream, a.logits, a.lse,
                         a.num_kv_splits, a.split_cap, a.neutral, a.H, a.S1, out, o_sb, o_sh);
    else
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Workspace of the allocation-free decode entry point: the split partials
// and their LSE live in this file-scope array, one copy per GPU, held until
// the process ends. The kernels take its device address, which host code
// obtains once per device with hipGetSymbolAddress (the array's name is not a
// device address in host code).
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

hipError_t rolaq_noalloc_scratch(void** ptr) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* per_device[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!per_device[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // with device dev current
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    per_device[dev] = p;
  }
  *ptr = per_device[dev];
  return hipSuccess;
}
