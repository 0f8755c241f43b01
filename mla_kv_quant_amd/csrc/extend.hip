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
// Layout of the work: two launches.
//   gather  every key row of the extended sequences -- [latent | rope], INT2
//           rows dequantized and rounded to bf16 once -- into the caller's
//           workspace as fp16 (the same numbers: a bf16 value is exact in fp16
//           between 2^-17 and 65504), sequence b at rows koff_b .. koff_b +
//           prefix_b + q_b - 1 (koff_b = sum over b' < b of prefix_b' + q_b');
//           HBM-bound, read once per call instead of once per query block.
//   attend  a block takes BM consecutive (token, head) query rows of one
//           sequence (all heads share the keys: MQA) and walks its keys in
//           tiles of 64, each copied from the workspace into LDS by the whole
//           block while the previous tile is consumed (double-buffered, one
//           barrier per tile). Per wave and tile:
//   S^T[64 keys, RW rows] = K . Q^T   on fp16 MFMA 16x16x32 (Q converted to fp16
//                                     once, held in registers: exact products);
//   the causal mask only on tiles that reach past the block's first query position
//   softmax in the log2 domain against a per-row reference (the row's maximum
//   over the first tile + 8); a tile whose scores pass it by more than 15
//   moves it to the tile's maximum + 8 and scales O and the row sum by the
//   difference in place (scale_acc16), so every probability fits fp16
//   O[RW rows, D] += P . V           on fp16 MFMA 16x16x32 per 32-key half, the keys of
//                                     each lane taken in the order the score MFMA left
//                                     them, P rounded to fp16 (relative error 2^-12).
// A sequence whose key rows do not fit the workspace (the caller's key_rows
// was short of the true sum) gets NaN outputs.
#include "rolaq_common.h"
#include "rolaq_args.h"

namespace rolaq {

constexpr int kExtKeys = 64;          // keys per tile
constexpr int kExtMK = kExtKeys / 16;  // 16-key blocks per tile
constexpr int kExtKH = kExtKeys / 32;  // 32-key halves (K-steps of the output MFMA)
constexpr float kExtSlack = 15.0f;    // max exp2 argument: a probability stays <= 2^15 (fp16)
constexpr float kExtHeadroom = 8.0f;  // a reference sits this far above the maximum it was set from
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
  // tiles per barrier: D = 256 keeps a ring of four tiles in LDS and meets at
  // a barrier every second tile (fewer points where all eight waves align);
  // D = 512's tiles allow two buffers, one barrier per tile
  static constexpr int TPB = D == 256 ? 2 : 1;
  static constexpr int NBUF = 2 * TPB;
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

// Workspace row of key 0 of sequence b.
__device__ __forceinline__ int64_t key_offset(const ExtendArgs& a, int b) {
  int64_t off = 0;
  for (int i = 0; i < b; ++i) off += a.prefix_lens[i] + (a.qo_indptr[i + 1] - a.qo_indptr[i]);
  return off;
}

// Key rows of sequence blockIdx.x as fp16 (one thread per 16-byte chunk, rows
// strided over blockIdx.y): chunk rows from k_chunk, prefix rows from the BF16
// window (t < P or t >= L - W of the extended length L) or the INT2 row
// ((code - zero) * scale rounded to bf16), rope from rope_buf.
template <int D, int R>
__global__ __launch_bounds__(256) void extend_gather_kernel(ExtendArgs a) {
  constexpr int DR = D + R, CPR = DR / 8, NG = D / 128;
  const int b = blockIdx.x;
  const int64_t qo0 = a.qo_indptr[b];
  const int64_t Tq = a.qo_indptr[b + 1] - qo0;
  const int64_t prefix = a.prefix_lens[b];
  const int64_t L = prefix + Tq;
  const int64_t req = a.req_idx[b];
  const bool ring = req >= 0 && req < a.max_reqs;
  const int P = ring ? a.P : 0, W = ring ? a.W : 0;
  const int64_t koff = key_offset(a, b);
  const int64_t kv0 = a.kv_indptr[b];
  const int pmask = (1 << a.page_shift) - 1;
  const int64_t n = min(L, a.ws_rows - koff) * CPR;
  for (int64_t e = (int64_t)blockIdx.y * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.y * blockDim.x) {
    const int64_t t = e / CPR;
    const int c = (int)(e - t * CPR);
    u32x4 v;
    if (t >= prefix) {
      v = bf16x8_to_f16x8(gload<u32x4>(a.kc + (qo0 + t - prefix) * a.kc_st + 8 * c));
    } else {
      const int64_t slot = ((int64_t)a.kv_indices[kv0 + (t >> a.page_shift)] << a.page_shift) + (t & pmask);
      if (c >= D / 8) {
        v = bf16x8_to_f16x8(gload<u32x4>(a.rope + slot * R + 8 * (c - D / 8)));
      } else if (t < P || t >= L - W) {
        const int64_t inner = t < P ? t : P + (t - P) % (W > 0 ? W : 1);
        v = bf16x8_to_f16x8(gload<u32x4>(a.hp + (1 + req * (P + W) + inner) * D + 8 * c));
      } else {
        // elements 8c .. 8c + 7 sit in bytes 2c, 2c + 1 of the packed row
        const uint32_t bits = gload<uint16_t>(a.codes + slot * (D / 4) + 2 * c);
        const f32x2 sz = gload<f32x2>(a.params + slot * (2 * NG) + 2 * (c / 16));
        float f[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] = (float((bits >> (2 * k)) & 3u) - sz.y) * sz.x;
        v = bf16x8_to_f16x8(
            u32x4{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])});
      }
    }
    *reinterpret_cast<u32x4*>(a.ws + (koff + t) * DR + 8 * c) = v;
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
  define_acc_macros();
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
  const int64_t koff = key_offset(a, b);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gq = lane >> 4, la = lane & 15;
  if (koff + L > a.ws_rows) {
    // the sequence's key rows did not fit the workspace: its outputs are NaN
    for (int64_t e = tid; e < (int64_t)BM * D; e += 64 * G::WAVES) {
      const int64_t r = r0 + e / D;
      if (r < nrows) a.out[(qo0 + r / a.H) * a.o_st + (r % a.H) * a.o_sh + e % D] = 0x7FC0;
    }
    return;
  }
  // last query token of the block -> keys 0 .. prefix + t_last
  const int64_t t_last = min(nrows - 1, r0 + BM - 1) / a.H;
  const int kend = (int)(prefix + t_last + 1);
  const int ntiles = (kend + kExtKeys - 1) / kExtKeys;

  // tile copy: thread tid moves 16-byte chunks tid, tid + NT, ... of the tile's
  // key rows (keys past the block's last key are zeros)
  constexpr int DR = D + R, CPR = DR / 8, CH = kExtKeys * CPR, NT = 64 * G::WAVES, NCH = (CH + NT - 1) / NT;
  u32x4 raw[NCH];
  auto load_keys = [&](int k0) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ci = tid + NT * j;
      const int key = ci / CPR, c = ci - key * CPR;
      const int64_t kp = k0 + key;
      raw[j] = (ci < CH && kp < kend) ? gload<u32x4>(a.ws + (koff + kp) * DR + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_keys = [&](uint8_t* buf) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ci = tid + NT * j;
      const int key = ci / CPR, c = ci - key * CPR;
      if (ci < CH) *reinterpret_cast<u32x4*>(buf + key * G::KSTR + 16 * c) = raw[j];
    }
  };

  // ---- query rows of this wave: Q^T fragments (fp16) and positions ------------
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
      qf[nb][ks] = ok ? bf16x8_to_f16x8(*reinterpret_cast<const u32x4*>(qr + 32 * ks)) : u32x4{0u, 0u, 0u, 0u};
  }

  const float c2 = a.sm_scale * kLog2e;
  const int qfirst = (int)(prefix + r0 / a.H);  // causal limit of the block's first row
  int qp[NBR];  // causal limit of each lane's rows (-1: no row)
#pragma unroll
  for (int nb = 0; nb < NBR; ++nb) qp[nb] = (int)qpos[nb];

  f32x4 acc_o[NBR][ND];
  float m_ref[NBR], l_run[NBR];
#pragma unroll
  for (int nb = 0; nb < NBR; ++nb) {
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) acc_o[nb][nd] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_ref[nb] = kExtMasked;
    l_run[nb] = 0.f;
  }

  constexpr int TPB = G::TPB, NBUF = G::NBUF;
#pragma unroll
  for (int t = 0; t < TPB; ++t) {
    if (t < ntiles) {
      load_keys(t * kExtKeys);
      store_keys(s_buf + t * G::BUF);
    }
  }
  __syncthreads();

  // Tile it is read from buffer it % NBUF; tile it + TPB is loaded during
  // tile it and stored after it into the buffer of tile it - TPB, which every
  // wave finished before the barrier that ended the previous group of TPB tiles.
  for (int it = 0; it < ntiles; ++it) {
    const uint8_t* kb = s_buf + (it % NBUF) * G::BUF;
    const int k0 = it * kExtKeys;
    // loads of a later tile first: they have this tile's compute to land
    if (it + TPB < ntiles) load_keys(k0 + TPB * kExtKeys);

    // ---- scores S^T[key, row] ----------------------------------------------
    f32x4 s[kExtMK][NBR];
#pragma unroll
    for (int mk = 0; mk < kExtMK; ++mk)
#pragma unroll
      for (int nb = 0; nb < NBR; ++nb) s[mk][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // the K operands of K-step ks + 1 are read while step ks's MFMAs run
    auto kread = [&](int ks, int mk) {
      return *reinterpret_cast<const u32x4*>(kb + (16 * mk + la) * G::KSTR + 64 * ks + 16 * gq);
    };
    u32x4 kf[2][kExtMK];
#pragma unroll
    for (int mk = 0; mk < kExtMK; ++mk) kf[0][mk] = kread(0, mk);
#pragma unroll
    for (int ks = 0; ks < KSQ; ++ks) {
      if (ks + 1 < KSQ) {
#pragma unroll
        for (int mk = 0; mk < kExtMK; ++mk) kf[(ks + 1) & 1][mk] = kread(ks + 1, mk);
      }
#pragma unroll
      for (int mk = 0; mk < kExtMK; ++mk)
#pragma unroll
        for (int nb = 0; nb < NBR; ++nb) s[mk][nb] = mfma16x16x32_f16(kf[ks & 1][mk], qf[nb][ks], s[mk][nb]);
      if (ks + 1 < KSQ) {
        __builtin_amdgcn_sched_group_barrier(0x100, kExtMK, 0);  // the next step's reads
        __builtin_amdgcn_sched_group_barrier(0x008, kExtMK * NBR, 0);
      }
    }

    // ---- softmax (row = 16 nb + la; keys 16 mk + 4 gq + i) -------------------
    // Scores stay in raw units (the scale c2 > 0 is applied inside the exp2's
    // argument, by one FMA). A tile that ends before the block's first query
    // position needs no causal mask (rows past the last query, qp = -1, stay
    // masked).
    const bool open = k0 + kExtKeys - 1 <= qfirst;
#pragma unroll
    for (int nb = 0; nb < NBR; ++nb) {
      // key k0 + 16 mk + 4 gq + i is visible to the row when 16 mk + i <= lim
      const int lim = qp[nb] < 0 ? -1 : (open ? kExtKeys : qp[nb] - k0 - 4 * gq);
#pragma unroll
      for (int mk = 0; mk < kExtMK; ++mk)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[mk][nb][i] = 16 * mk + i <= lim ? s[mk][nb][i] : kExtMasked;
    }
    float mx[NBR];
    uint64_t need[NBR];  // lanes whose row passes its reference by more than the slack
#pragma unroll
    for (int nb = 0; nb < NBR; ++nb) {
      mx[nb] = kExtMasked;
#pragma unroll
      for (int mk = 0; mk < kExtMK; ++mk)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx[nb] = fmaxf(mx[nb], s[mk][nb][i]);
      mx[nb] *= c2;  // log2 units (a masked maximum stays far below any reference)
      need[nb] = __builtin_amdgcn_ballot_w64(it > 0 && mx[nb] > m_ref[nb] + kExtSlack);
    }
    // the first tile sets each row's reference (key 0 is visible to every row)
    if (it == 0) {
#pragma unroll
      for (int nb = 0; nb < NBR; ++nb) m_ref[nb] = max_over_rows(mx[nb]) + kExtHeadroom;
    }
    // rows past the slack: reference to the tile's maximum + 8, O and the sum
    // scaled by the difference (O's lane holds rows 4 gq + i, whose factors
    // come from the lanes whose row la is that row)
#pragma unroll
    for (int nb = 0; nb < NBR; ++nb) {
      float fj[4] = {1.f, 1.f, 1.f, 1.f};
      if (need[nb]) {
        const float mt = max_over_rows(mx[nb]);
        const float mn = mt > m_ref[nb] + kExtSlack ? mt + kExtHeadroom : m_ref[nb];
        const float f = __builtin_amdgcn_exp2f(m_ref[nb] - mn);
        l_run[nb] *= f;
        m_ref[nb] = mn;
#pragma unroll
        for (int i = 0; i < 4; ++i) fj[i] = __shfl(f, 4 * gq + i);
      }
      static_assert(ND % 16 == 0, "rescale in groups of 16 column blocks");
#pragma unroll
      for (int nd = 0; nd < ND; nd += 16)
        scale_acc16(*reinterpret_cast<f32x4(*)[16]>(&acc_o[nb][nd]), fj, need[nb]);
    }
    u32x4 pf[kExtKH][NBR];
#pragma unroll
    for (int kh = 0; kh < kExtKH; ++kh)
#pragma unroll
      for (int nb = 0; nb < NBR; ++nb) {
        float p[2][4];
#pragma unroll
        for (int mk = 0; mk < 2; ++mk)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[mk][i] = __builtin_amdgcn_exp2f(fmaf(s[2 * kh + mk][nb][i], c2, -m_ref[nb]));  // masked: 0
          }
        pf[kh][nb] = u32x4{pack_f16(p[0][0], p[0][1]), pack_f16(p[0][2], p[0][3]), pack_f16(p[1][0], p[1][1]),
                           pack_f16(p[1][2], p[1][3])};
        // the row sum of the fp16 probabilities the output MFMA uses
#pragma unroll
        for (int d = 0; d < 4; ++d) l_run[nb] = sum_f16x2(pf[kh][nb][d], l_run[nb]);
      }

    // ---- O[row, d] += P . V --------------------------------------------------
#pragma unroll
    for (int kh = 0; kh < kExtKH; ++kh)
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        const uint8_t* kv = kb + 32 * kh * G::KSTR;
        const u32x2 v0 = read_v_tr(kv, G::KSTR, gq, la, nd, 0), v1 = read_v_tr(kv, G::KSTR, gq, la, nd, 1);
        const u32x4 vf = {v0.x, v0.y, v1.x, v1.y};
#pragma unroll
        for (int nb = 0; nb < NBR; ++nb) acc_o[nb][nd] = mfma16x16x32_f16(pf[kh][nb], vf, acc_o[nb][nd]);
      }

    // ---- tile it + TPB into the buffer of tile it - TPB ---------------------
    if (it + TPB < ntiles) store_keys(s_buf + ((it + TPB) % NBUF) * G::BUF);
    if (it % TPB == TPB - 1 || it + 1 == ntiles) __syncthreads();
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
    const int lds = G::NBUF * G::BUF;                                                                         \
    const hipError_t e = hipFuncSetAttribute((const void*)extend_kernel<DD, RR>,                        \
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds);          \
    if (e != hipSuccess) return e;                                                                      \
    hipLaunchKernelGGL((extend_gather_kernel<DD, RR>), dim3((unsigned)a.B, 64), dim3(256), 0, stream, a); \
    hipLaunchKernelGGL((extend_kernel<DD, RR>), grid, dim3(64 * G::WAVES), lds, stream, a);             \
    return hipGetLastError();                                                                           \
  }
  ROLAQ_EXT(256, 32)
  ROLAQ_EXT(512, 64)
#undef ROLAQ_EXT
  return hipErrorInvalidValue;
}
