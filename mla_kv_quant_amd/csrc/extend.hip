// Absorbed MLA extend (chunked-prefill) attention over the packed INT2 cache.
//
// Reference behaviour: the packed pool's extend path of the patched SGLang
// (deployment/patches/rolaq_sglang.patch:208-235 builds q = [q_nope_out | q_pe]
// in the rotated frame and hands the chunk's own k = [k_nope | k_pe] and the
// pool to the MLA attention); prefix rows are the cache's rows (INT2 codes
// dequantized as (code - zero) * scale and rounded to bf16, the HF cache's
// stored form, mla_quant/cache.py:1030-1039), except the first P and the last
// W positions of the extended sequence, which are the BF16 window rows; the
// chunk's rows enter as the given BF16 keys; attention is causal.
//
// Layout of the work: a block takes BM consecutive (token, head) query rows of
// one sequence (all heads share the keys: MQA) and walks the keys in tiles of
// 32. Each tile is built in LDS by 256 threads of the block -- key rows
// [latent | rope] -- while the previous tile is being consumed,
// double-buffered. Per wave and tile:
//   S^T[32 keys, RW rows] = K . Q^T   on MFMA 16x16x32 (Q held in registers)
//   softmax in the log2 domain against a fixed per-row reference (the row's
//   maximum over the first tile); a block whose scores exceed it by more than
//   2^64 somewhere is redone with the true maxima, so O is never rescaled
//   O[RW rows, D] += P . V           on MFMA 16x16x32, the keys of each lane
//                                     taken in the order the score MFMA left them,
//                                     P split into bf16 hi + lo (FP32-level accuracy).
#include "rolaq_common.h"
#include "rolaq_args.h"

namespace rolaq {

constexpr int kExtKeys = 32;          // keys per tile
constexpr float kExtSlack = 64.0f;    // log2 headroom of a score over the softmax reference
constexpr float kExtMasked = -1.0e30f;

template <int D, int R>
struct ExtGeo {
  static constexpr int DR = D + R;
  static constexpr int KSQ = DR / 32;               // K-steps of the score MFMA
  static constexpr int NBR = 1;                     // 16-row blocks per wave
  static constexpr int RW = 16 * NBR;               // query rows per wave
  // D = 256: 8 waves, two per SIMD (one wave's softmax and tile build overlap
  // the other's MFMAs; 16 rows per wave keep it within 256 registers);
  // D = 512: 4 waves, one per SIMD (the 32 output blocks need the registers)
  static constexpr int WAVES = D == 256 ? 8 : 4;
  static constexpr int BM = WAVES * RW;             // query rows per block
  static constexpr int ND = D / 16;                 // output column blocks
  static constexpr int KSTR = 2 * DR + 32;          // bytes per key row in LDS (padding measured: +32 B fastest)
  static constexpr int KBYTES = kExtKeys * KSTR;
  static constexpr int BUF = KBYTES;                // one tile: key rows only
  static constexpr int OPT = D / 256;               // latent octets per loader thread
};

__device__ __forceinline__ float max_over_rows(float v) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float add_over_rows(float v) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Where the rows of one key tile come from, per loader thread: key quad
// kq (keys 4 kq .. 4 kq + 3 of the tile) and latent octets OPT * o .. .
template <int D, int R>
struct TileRaw {
  static constexpr int OPT = ExtGeo<D, R>::OPT;
  u32x4 lat[4][OPT];  // bf16 rows
  uint32_t code[4];   // packed codes of the thread's octets (INT2 rows)
  u32x4 rope[4];      // rope octet o (threads o < R / 8)
  f32x2 prm[4];       // (scale, zero) of the INT2 rows' group
  uint32_t mode;      // 2 bits per key: 0 zero, 1 bf16, 2 int2
};

// Pages of the prefix keys of a tile (page-table lookups), one tile ahead of
// the data loads; the values are first used by the next tile's load_tile, so
// no instruction of this tile waits on them (0 for keys without a page).
template <int D, int R>
__device__ __forceinline__ void lookup_tile(const ExtendArgs& a, int32_t pg[4], int k0, int kq, int64_t prefix,
                                            int64_t kv0, int kend) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int kp = k0 + 4 * kq + k;
    pg[k] = (kp < kend && kp < prefix) ? gload<int32_t>(a.kv_indices + kv0 + (kp >> a.page_shift)) : 0;
  }
}

// INT2 = true: every key of the tile is an INT2 prefix row (the tile lies in
// [P, min(prefix, L - W))), so no per-key source selection is needed.
template <int D, int R, bool INT2>
__device__ __forceinline__ void load_tile(const ExtendArgs& a, TileRaw<D, R>& t, const int32_t pg[4], int k0,
                                          int kq, int o, int64_t qo0, int64_t prefix, int64_t L, int64_t req,
                                          int kend) {
  constexpr int NG = D / 128, OPT = ExtGeo<D, R>::OPT;
  const int dlo = 8 * OPT * o;  // first latent column of this thread
  const int g = dlo / 128;
  if constexpr (INT2) {
    const uint32_t coff = dlo / 4;  // elements dlo .. of the packed row start at byte dlo / 4
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int kp = k0 + 4 * kq + k;
      const uint32_t slot = ((uint32_t)pg[k] << a.page_shift) + (kp & ((1 << a.page_shift) - 1));
      const uint64_t sl = slot;  // 64-bit offsets: a pool may exceed 4 GB per array
      if constexpr (OPT == 2) t.code[k] = gload<uint32_t>(a.codes + sl * (D / 4) + coff);
      else t.code[k] = gload<uint16_t>(a.codes + sl * (D / 4) + coff);
      t.prm[k] = gload<f32x2>(a.params + sl * (2 * NG) + 2 * g);
      t.rope[k] = o < R / 8 ? gload<u32x4>(a.rope + sl * R + 8 * o) : u32x4{0u, 0u, 0u, 0u};
    }
    t.mode = 0xAAu;
    return;
  }
  // where each key's bytes are (all addresses first: the pages were loaded an
  // iteration ago, and no load below may wait behind another)
  const uint16_t* lat[4];
  const uint16_t* rope[4];
  const uint8_t* code[4];
  const float* prm[4];
  uint32_t mode = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int kp = k0 + 4 * kq + k;
    const int64_t slot = (int64_t)pg[k] * (1 << a.page_shift) + (kp & ((1 << a.page_shift) - 1));
    lat[k] = nullptr;
    rope[k] = nullptr;
    code[k] = nullptr;
    prm[k] = nullptr;
    if (kp >= kend) continue;
    if (kp >= prefix) {  // a row of the chunk itself: the given BF16 key
      lat[k] = a.kc + (qo0 + kp - prefix) * a.kc_st + dlo;
      rope[k] = a.kc + (qo0 + kp - prefix) * a.kc_st + D + 8 * o;
      mode |= 1u << (2 * k);
    } else if (kp < a.P || kp >= L - a.W) {  // BF16 window row
      const int inner = kp < a.P ? kp : a.P + (kp - a.P) % (a.W > 0 ? a.W : 1);
      lat[k] = a.hp + (1 + req * (a.P + a.W) + inner) * D + dlo;
      rope[k] = a.rope + slot * R + 8 * o;
      mode |= 1u << (2 * k);
    } else {  // INT2 row
      code[k] = a.codes + slot * (D / 4) + dlo / 4;
      prm[k] = a.params + slot * 2 * NG + 2 * g;
      rope[k] = a.rope + slot * R + 8 * o;
      mode |= 2u << (2 * k);
    }
  }
  t.mode = mode;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t m = (mode >> (2 * k)) & 3u;
#pragma unroll
    for (int j = 0; j < OPT; ++j) t.lat[k][j] = m == 1u ? gload<u32x4>(lat[k] + 8 * j) : u32x4{0u, 0u, 0u, 0u};
    if constexpr (OPT == 2) t.code[k] = m == 2u ? gload<uint32_t>(code[k]) : 0u;
    else t.code[k] = m == 2u ? uint32_t(gload<uint16_t>(code[k])) : 0u;
    t.prm[k] = m == 2u ? gload<f32x2>(prm[k]) : f32x2{0.f, 0.f};
    t.rope[k] = (m != 0u && o < R / 8) ? gload<u32x4>(rope[k]) : u32x4{0u, 0u, 0u, 0u};
  }
}

// Dequantize (INT2 rows) and store one tile's key rows [key][latent | rope]
// (bf16). The output MFMA reads the latent transposed out of the same rows.
template <int D, int R, bool INT2>
__device__ __forceinline__ void store_tile(const TileRaw<D, R>& t, uint8_t* buf, int kq, int o) {
  using G = ExtGeo<D, R>;
  constexpr int OPT = G::OPT;
  uint8_t* kb = buf;
#pragma unroll
  for (int j = 0; j < OPT; ++j) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t m = (t.mode >> (2 * k)) & 3u;
      u32x4 v;
      if (INT2 || m == 2u) {
        // (code - zero) * scale, rounded to bf16 as the reference's QDQ rows are
        const uint32_t bits = OPT == 2 ? (t.code[k] >> (16 * j)) : t.code[k];
        const float sc = t.prm[k].x, z = t.prm[k].y;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (float((bits >> (2 * e)) & 3u) - z) * sc;
        v = u32x4{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])};
      } else {
        v = t.lat[k][j];
      }
      *reinterpret_cast<u32x4*>(kb + (4 * kq + k) * G::KSTR + 16 * (OPT * o + j)) = v;
    }
  }
  if (o < R / 8) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      *reinterpret_cast<u32x4*>(kb + (4 * kq + k) * G::KSTR + 2 * D + 16 * o) = t.rope[k];
  }
}

// 64 bits of the output MFMA's B operand, read transposed out of the key rows
// (ds_read_b64_tr_b16: within each 16-lane group, lane 4s + e receives element
// e of the chunks addressed by lanes s, s + 4, s + 8, s + 12). Lane (gq, la)
// addresses key row tau(gq, 4h + (la >> 2)) at latent columns 16 nd + 4 (la & 3),
// so it receives rows tau(gq, 4h + 0..3) of column 16 nd + la: K-index
// 8 gq + 4h + k of B is key tau(gq, 4h + k), the order P is held in.
__device__ __forceinline__ u32x2 read_v_tr(const uint8_t* kb, int kstr, int gq, int la, int nd, int h) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const int key = 16 * h + 4 * gq + (la >> 2);
  const uint8_t* p = kb + key * kstr + 2 * (16 * nd + 4 * (la & 3));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

template <int D, int R>
__global__ __launch_bounds__((64 * ExtGeo<D, R>::WAVES), 1) void extend_kernel(ExtendArgs a) {
  using G = ExtGeo<D, R>;
  constexpr int KSQ = G::KSQ, NBR = G::NBR, RW = G::RW, BM = G::BM, ND = G::ND;
  extern __shared__ __attribute__((aligned(16))) uint8_t s_buf[];

  const int b = blockIdx.x;
  const int64_t qo0 = a.qo_indptr[b];
  const int64_t Tq = a.qo_indptr[b + 1] - qo0;
  // heavier blocks (later tokens) first
  const int64_t r0 = (int64_t)(gridDim.y - 1 - blockIdx.y) * BM;
  const int64_t nrows = Tq * a.H;
  if (r0 >= nrows) return;
  const int64_t prefix = a.prefix_lens[b];
  const int64_t L = prefix + Tq;
  const int64_t req = a.req_idx[b];
  // a request without ring rows (index outside [0, max_reqs)) has no BF16
  // window: the writer stored none for it, so its prefix is read from the codes
  if (req < 0 || req >= a.max_reqs) a.P = a.W = 0;
  const int64_t kv0 = a.kv_indptr[b];
  // last query token of the block -> keys 0 .. prefix + t_last
  const int64_t t_last = min(nrows - 1, r0 + BM - 1) / a.H;
  const int kend = (int)(prefix + t_last + 1);
  const int ntiles = (kend + kExtKeys - 1) / kExtKeys;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gq = lane >> 4, la = lane & 15;
  // loader role: the first 256 threads build the tiles (key quad kq, octet o)
  const int kq = (tid >> 5) & 7, o = tid & 31;
  const bool ldr = tid < 256;

  // ---- query rows of this wave: Q^T fragments and positions -----------------
  u32x4 qf[NBR][KSQ];
  int64_t qpos[NBR];
#pragma unroll
  for (int nb = 0; nb < NBR; ++nb) {
    const int64_t r = r0 + RW * wave + 16 * nb + la;
    const bool ok = r < nrows;
    const int64_t t = ok ? r / a.H : 0, h = ok ? r % a.H : 0;
    qpos[nb] = ok ? prefix + t : -1;
    const uint16_t* qr = a.q + (qo0 + t) * a.q_st + h * a.q_sh + 8 * gq;
#pragma unroll
    for (int ks = 0; ks < KSQ; ++ks)
      qf[nb][ks] = ok ? *reinterpret_cast<const u32x4*>(qr + 32 * ks) : u32x4{0u, 0u, 0u, 0u};
  }

  const float c2 = a.sm_scale * kLog2e;
  int qp[NBR];  // causal limit of each lane's rows (-1: no row)
#pragma unroll
  for (int nb = 0; nb < NBR; ++nb) qp[nb] = (int)qpos[nb];

  // a tile of INT2 prefix rows only ([P, min(prefix, L - W))): loads without per-key selection
  const int64_t int2_end = min(prefix, L - (int64_t)a.W);
  auto int2_tile = [&](int t0) { return t0 >= a.P && (int64_t)t0 + kExtKeys <= int2_end; };

  f32x4 acc_o[NBR][ND];
  float m_ref[NBR], m_lane[NBR], l_run[NBR];
  bool redo = false;
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int nb = 0; nb < NBR; ++nb) {
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) acc_o[nb][nd] = f32x4{0.f, 0.f, 0.f, 0.f};
      m_lane[nb] = kExtMasked;
      l_run[nb] = 0.f;
    }

    TileRaw<D, R> raw;
    int32_t sl[4];
    if (ldr) {
      lookup_tile<D, R>(a, sl, 0, kq, prefix, kv0, kend);
      load_tile<D, R, false>(a, raw, sl, 0, kq, o, qo0, prefix, L, req, kend);
      lookup_tile<D, R>(a, sl, kExtKeys, kq, prefix, kv0, kend);
      store_tile<D, R, false>(raw, s_buf, kq, o);
    }
    __syncthreads();

    for (int it = 0; it < ntiles; ++it) {
      const uint8_t* kb = s_buf + (it & 1) * G::BUF;
      const int k0 = it * kExtKeys;
      // loads of the next tile first: they have this tile's compute to land
      // (its pages were looked up an iteration ago)
      if (ldr && it + 1 < ntiles) {
        if (int2_tile(k0 + kExtKeys)) load_tile<D, R, true>(a, raw, sl, k0 + kExtKeys, kq, o, qo0, prefix, L, req, kend);
        else load_tile<D, R, false>(a, raw, sl, k0 + kExtKeys, kq, o, qo0, prefix, L, req, kend);
        lookup_tile<D, R>(a, sl, k0 + 2 * kExtKeys, kq, prefix, kv0, kend);
      }

      // ---- scores S^T[key, row] --------------------------------------------
      f32x4 s[2][NBR];
#pragma unroll
      for (int mk = 0; mk < 2; ++mk)
#pragma unroll
        for (int nb = 0; nb < NBR; ++nb) s[mk][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSQ; ++ks) {
#pragma unroll
        for (int mk = 0; mk < 2; ++mk) {
          const u32x4 kf = *reinterpret_cast<const u32x4*>(kb + (16 * mk + la) * G::KSTR + 64 * ks + 16 * gq);
#pragma unroll
          for (int nb = 0; nb < NBR; ++nb) s[mk][nb] = mfma16x16x32(kf, qf[nb][ks], s[mk][nb]);
        }
      }

      // ---- softmax against the fixed reference (row = 16 nb + la; keys 16 mk + 4 gq + i)
#pragma unroll
      for (int nb = 0; nb < NBR; ++nb) {
        float mx = m_lane[nb];
#pragma unroll
        for (int mk = 0; mk < 2; ++mk)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kp = k0 + 16 * mk + 4 * gq + i;
            const float v = kp <= qp[nb] ? s[mk][nb][i] * c2 : kExtMasked;
            s[mk][nb][i] = v;
            mx = fmaxf(mx, v);
          }
        m_lane[nb] = mx;
      }
      // the reference of the first pass: each row's maximum over the first tile
      // (key 0 is visible to every row, so it is finite)
      if (it == 0 && pass == 0) {
#pragma unroll
        for (int nb = 0; nb < NBR; ++nb) m_ref[nb] = max_over_rows(m_lane[nb]);
      }
      u32x4 pf[NBR], pl[NBR];
#pragma unroll
      for (int nb = 0; nb < NBR; ++nb) {
        float p[2][4];
#pragma unroll
        for (int mk = 0; mk < 2; ++mk)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[mk][i] = __builtin_amdgcn_exp2f(s[mk][nb][i] - m_ref[nb]);  // masked: 2^-1e30 = 0
            l_run[nb] += p[mk][i];
          }
        // P as bf16 hi + lo: the output keeps FP32-level accuracy in P
        pf[nb] = u32x4{pack_bf16(p[0][0], p[0][1]), pack_bf16(p[0][2], p[0][3]), pack_bf16(p[1][0], p[1][1]),
                       pack_bf16(p[1][2], p[1][3])};
        float r[2][4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w = pf[nb][e];
          r[e >> 1][2 * (e & 1)] = p[e >> 1][2 * (e & 1)] - bf16_lo(w);
          r[e >> 1][2 * (e & 1) + 1] = p[e >> 1][2 * (e & 1) + 1] - bf16_hi(w);
        }
        pl[nb] = u32x4{pack_bf16(r[0][0], r[0][1]), pack_bf16(r[0][2], r[0][3]), pack_bf16(r[1][0], r[1][1]),
                       pack_bf16(r[1][2], r[1][3])};
      }

      // ---- O[row, d] += P . V ------------------------------------------------
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        const u32x2 v0 = read_v_tr(kb, G::KSTR, gq, la, nd, 0), v1 = read_v_tr(kb, G::KSTR, gq, la, nd, 1);
        const u32x4 vf = {v0.x, v0.y, v1.x, v1.y};
#pragma unroll
        for (int nb = 0; nb < NBR; ++nb) {
          acc_o[nb][nd] = mfma16x16x32(pf[nb], vf, acc_o[nb][nd]);
          acc_o[nb][nd] = mfma16x16x32(pl[nb], vf, acc_o[nb][nd]);
        }
      }

      // ---- next tile into the other buffer (last read before the previous barrier)
      if (ldr && it + 1 < ntiles) {
        if (int2_tile(k0 + kExtKeys)) store_tile<D, R, true>(raw, s_buf + ((it + 1) & 1) * G::BUF, kq, o);
        else store_tile<D, R, false>(raw, s_buf + ((it + 1) & 1) * G::BUF, kq, o);
      }
      __syncthreads();
    }

    // a score above the reference by more than the slack (2^64 bounds every P
    // and keeps the sums finite): redo the block with each row's true maximum
    bool over = false;
#pragma unroll
    for (int nb = 0; nb < NBR; ++nb) {
      const float mt = max_over_rows(m_lane[nb]);
      over |= mt > m_ref[nb] + kExtSlack;
      m_ref[nb] = mt;
    }
    redo = __syncthreads_or(pass == 0 && over);
    if (!redo) break;
  }

  // ---- normalise and store -----------------------------------------------------
#pragma unroll
  for (int nb = 0; nb < NBR; ++nb) {
    const float l = add_over_rows(l_run[nb]);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ii = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (4 * gq + i), __float_as_int(inv)));
      const int64_t r = r0 + RW * wave + 16 * nb + 4 * gq + i;
      if (r >= nrows) continue;
      const int64_t t = r / a.H, h = r % a.H;
      uint16_t* dst = a.out + (qo0 + t) * a.o_st + h * a.o_sh + la;
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) dst[16 * nd] = float_to_bf16(acc_o[nb][nd][i] * ii);
    }
  }
}

}  // namespace rolaq

hipError_t rolaq_launch_extend(const rolaq::ExtendArgs& a, int D, int R, int max_q_len, hipStream_t stream) {
  using namespace rolaq;
#define ROLAQ_EXT(DD, RR)                                                                               \
  if (D == DD && R == RR) {                                                                             \
    using G = ExtGeo<DD, RR>;                                                                           \
    const int64_t rows = (int64_t)max_q_len * a.H;                                                      \
    const dim3 grid((unsigned)a.B, (unsigned)((rows + G::BM - 1) / G::BM));                             \
    const int lds = 2 * G::BUF;                                                                         \
    const hipError_t e = hipFuncSetAttribute((const void*)extend_kernel<DD, RR>,                        \
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds);          \
    if (e != hipSuccess) return e;                                                                      \
    hipLaunchKernelGGL((extend_kernel<DD, RR>), grid, dim3(64 * G::WAVES), lds, stream, a);             \
    return hipGetLastError();                                                                           \
  }
  ROLAQ_EXT(256, 32)
  ROLAQ_EXT(512, 64)
#undef ROLAQ_EXT
  return hipErrorInvalidValue;
}
