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
// 32. Each tile is built in LDS by the whole block -- latent+rope rows for the
// scores and the latent transposed for the output -- while the previous tile
// is being consumed, double-buffered. Per wave and tile:
//   S^T[32 keys, RW rows] = K . Q^T   on MFMA 16x16x32 (Q held in registers)
//   online softmax in the log2 domain, lazy rescaling (the running maximum is
//   only moved when a tile exceeds it by more than 2^8)
//   O[RW rows, D] += P . V           on MFMA 16x16x32, the keys of each lane
//                                     taken in the order the score MFMA left them,
//                                     P split into bf16 hi + lo (FP32-level accuracy).
#include "rolaq_common.h"
#include "rolaq_args.h"

namespace rolaq {

constexpr int kExtKeys = 32;          // keys per tile
constexpr float kExtLazy = 8.0f;      // log2 slack before the running max moves
constexpr float kExtMasked = -1.0e30f;

template <int D, int R>
struct ExtGeo {
  static constexpr int DR = D + R;
  static constexpr int KSQ = DR / 32;               // K-steps of the score MFMA
  static constexpr int NBR = D == 256 ? 2 : 1;      // 16-row blocks per wave
  static constexpr int RW = 16 * NBR;               // query rows per wave
  static constexpr int BM = 4 * RW;                 // query rows per block
  static constexpr int ND = D / 16;                 // output column blocks
  static constexpr int KSTR = 2 * DR + 16;          // bytes per key row in LDS
  static constexpr int VSTR = 2 * kExtKeys + 16;    // bytes per latent column in LDS
  static constexpr int KBYTES = kExtKeys * KSTR;
  static constexpr int BUF = KBYTES + D * VSTR;     // one tile
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
  u32x4 lat[4][OPT];  // bf16 rows, or the codes of the octets in lat[k][0].x
  u32x4 rope[4];      // rope octet o (threads o < R / 8)
  f32x2 prm[4];       // (scale, zero) of the INT2 rows' group
  uint32_t mode;      // 2 bits per key: 0 zero, 1 bf16, 2 int2
};

template <int D, int R>
__device__ __forceinline__ void load_tile(const ExtendArgs& a, TileRaw<D, R>& t, int k0, int kq, int o,
                                          int64_t qo0, int64_t prefix, int64_t L, int64_t req,
                                          int64_t kv0, int kend) {
  constexpr int NG = D / 128, OPT = ExtGeo<D, R>::OPT;
  t.mode = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int kp = k0 + 4 * kq + k;
#pragma unroll
    for (int j = 0; j < OPT; ++j) t.lat[k][j] = u32x4{0u, 0u, 0u, 0u};
    t.rope[k] = u32x4{0u, 0u, 0u, 0u};
    t.prm[k] = f32x2{0.f, 0.f};
    if (kp >= kend) continue;
    const int dlo = 8 * OPT * o;  // first latent column of this thread
    if (kp >= prefix) {
      // a row of the chunk itself: the given BF16 key
      const uint16_t* src = a.kc + (qo0 + kp - prefix) * a.kc_st;
#pragma unroll
      for (int j = 0; j < OPT; ++j) t.lat[k][j] = *reinterpret_cast<const u32x4*>(src + dlo + 8 * j);
      if (o < R / 8) t.rope[k] = *reinterpret_cast<const u32x4*>(src + D + 8 * o);
      t.mode |= 1u << (2 * k);
      continue;
    }
    const int64_t slot = (int64_t)a.kv_indices[kv0 + (kp >> a.page_shift)] * (1 << a.page_shift) +
                         (kp & ((1 << a.page_shift) - 1));
    if (o < R / 8) t.rope[k] = *reinterpret_cast<const u32x4*>(a.rope + slot * R + 8 * o);
    if (kp < a.P || kp >= L - a.W) {
      const int inner = kp < a.P ? kp : a.P + (kp - a.P) % (a.W > 0 ? a.W : 1);
      const uint16_t* src = a.hp + (1 + req * (a.P + a.W) + inner) * D;
#pragma unroll
      for (int j = 0; j < OPT; ++j) t.lat[k][j] = *reinterpret_cast<const u32x4*>(src + dlo + 8 * j);
      t.mode |= 1u << (2 * k);
    } else {
      const int g = dlo / 128, e0 = dlo % 128;
      const uint8_t* crow = a.codes + slot * (D / 4) + 4 * (NG * (e0 / 16) + g);
      if constexpr (OPT == 2) {
        t.lat[k][0].x = *reinterpret_cast<const uint32_t*>(crow);
      } else {
        t.lat[k][0].x = *reinterpret_cast<const uint16_t*>(crow + 2 * ((e0 / 8) & 1));
      }
      t.prm[k] = *reinterpret_cast<const f32x2*>(a.params + slot * 2 * NG + 2 * g);
      t.mode |= 2u << (2 * k);
    }
  }
}

// Dequantize (INT2 rows) and store one tile: key rows for the scores, the
// latent transposed for the output (keys of a column in the order the score
// MFMA leaves them in its lanes: position 8 gq + j holds key tau(gq, j)).
template <int D, int R>
__device__ __forceinline__ void store_tile(const TileRaw<D, R>& t, uint8_t* buf, int kq, int o) {
  using G = ExtGeo<D, R>;
  constexpr int OPT = G::OPT;
  uint8_t* kb = buf;
  uint8_t* vb = buf + G::KBYTES;
  const int vpos = 2 * (8 * (kq & 3) + 4 * (kq >> 2));
#pragma unroll
  for (int j = 0; j < OPT; ++j) {
    u32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t m = (t.mode >> (2 * k)) & 3u;
      if (m == 2u) {
        // (code - zero) * scale, rounded to bf16 as the reference's QDQ rows are
        const uint32_t bits = OPT == 2 ? (t.lat[k][0].x >> (16 * j)) : t.lat[k][0].x;
        const float sc = t.prm[k].x, z = t.prm[k].y;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (float((bits >> (2 * e)) & 3u) - z) * sc;
        v[k] = u32x4{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])};
      } else {
        v[k] = t.lat[k][j];
      }
      *reinterpret_cast<u32x4*>(kb + (4 * kq + k) * G::KSTR + 16 * (OPT * o + j)) = v[k];
    }
    // transpose 4 keys x 8 columns -> 8 columns x 4 keys
    const int d0 = 8 * (OPT * o + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // columns d0 + 2e (low halves) and d0 + 2e + 1 (high halves)
      const uint32_t lo01 = __builtin_amdgcn_perm(v[1][e], v[0][e], 0x05040100u);
      const uint32_t lo23 = __builtin_amdgcn_perm(v[3][e], v[2][e], 0x05040100u);
      const uint32_t hi01 = __builtin_amdgcn_perm(v[1][e], v[0][e], 0x07060302u);
      const uint32_t hi23 = __builtin_amdgcn_perm(v[3][e], v[2][e], 0x07060302u);
      *reinterpret_cast<u32x2*>(vb + (d0 + 2 * e) * G::VSTR + vpos) = u32x2{lo01, lo23};
      *reinterpret_cast<u32x2*>(vb + (d0 + 2 * e + 1) * G::VSTR + vpos) = u32x2{hi01, hi23};
    }
  }
  if (o < R / 8) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      *reinterpret_cast<u32x4*>(kb + (4 * kq + k) * G::KSTR + 2 * D + 16 * o) = t.rope[k];
  }
}

template <int D, int R>
__global__ __launch_bounds__(256, 1) void extend_kernel(ExtendArgs a) {
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
  const int64_t kv0 = a.kv_indptr[b];
  // last query token of the block -> keys 0 .. prefix + t_last
  const int64_t t_last = min(nrows - 1, r0 + BM - 1) / a.H;
  const int kend = (int)(prefix + t_last + 1);
  const int ntiles = (kend + kExtKeys - 1) / kExtKeys;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gq = lane >> 4, la = lane & 15;
  const int kq = tid >> 5, o = tid & 31;  // loader role

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

  f32x4 acc_o[NBR][ND];
#pragma unroll
  for (int nb = 0; nb < NBR; ++nb)
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) acc_o[nb][nd] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[NBR], l_run[NBR];
#pragma unroll
  for (int nb = 0; nb < NBR; ++nb) {
    m_run[nb] = kExtMasked;
    l_run[nb] = 0.f;
  }
  const float c2 = a.sm_scale * kLog2e;

  TileRaw<D, R> raw;
  load_tile<D, R>(a, raw, 0, kq, o, qo0, prefix, L, req, kv0, kend);
  store_tile<D, R>(raw, s_buf, kq, o);
  if (ntiles > 1) load_tile<D, R>(a, raw, kExtKeys, kq, o, qo0, prefix, L, req, kv0, kend);
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const uint8_t* kb = s_buf + (it & 1) * G::BUF;
    const uint8_t* vb = kb + G::KBYTES;
    const int k0 = it * kExtKeys;

    // ---- scores S^T[key, row] ----------------------------------------------
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

    // ---- online softmax (row = 16 nb + la; keys 16 mk + 4 gq + i) -------------
    u32x4 pf[NBR], pl[NBR];
    bool need = false;
    float tmax[NBR];
#pragma unroll
    for (int nb = 0; nb < NBR; ++nb) {
      float mx = kExtMasked;
#pragma unroll
      for (int mk = 0; mk < 2; ++mk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kp = k0 + 16 * mk + 4 * gq + i;
          const float v = kp <= qpos[nb] ? s[mk][nb][i] * c2 : kExtMasked;
          s[mk][nb][i] = v;
          mx = fmaxf(mx, v);
        }
      tmax[nb] = max_over_rows(mx);
      need |= tmax[nb] > m_run[nb] + kExtLazy;
    }
    if (__any(need)) {
#pragma unroll
      for (int nb = 0; nb < NBR; ++nb) {
        const float mn = fmaxf(m_run[nb], tmax[nb]);
        const float f = __builtin_amdgcn_exp2f(m_run[nb] - mn);
        m_run[nb] = mn;
        l_run[nb] *= f;
        // rows 16 nb + 4 gq + i of the output layout live in lanes 4 gq + i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float fi = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (4 * gq + i), __float_as_int(f)));
#pragma unroll
          for (int nd = 0; nd < ND; ++nd) acc_o[nb][nd][i] *= fi;
        }
      }
    }
#pragma unroll
    for (int nb = 0; nb < NBR; ++nb) {
      float p[2][4];
#pragma unroll
      for (int mk = 0; mk < 2; ++mk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = s[mk][nb][i];
          p[mk][i] = v > kExtMasked ? __builtin_amdgcn_exp2f(v - m_run[nb]) : 0.f;
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

    // ---- O[row, d] += P . V --------------------------------------------------
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      const u32x4 vf = *reinterpret_cast<const u32x4*>(vb + (16 * nd + la) * G::VSTR + 16 * gq);
#pragma unroll
      for (int nb = 0; nb < NBR; ++nb) {
        acc_o[nb][nd] = mfma16x16x32(pf[nb], vf, acc_o[nb][nd]);
        acc_o[nb][nd] = mfma16x16x32(pl[nb], vf, acc_o[nb][nd]);
      }
    }

    // ---- next tile: store the one loaded, load the one after -----------------
    if (it + 1 < ntiles) {
      store_tile<D, R>(raw, s_buf + ((it + 1) & 1) * G::BUF, kq, o);
      if (it + 2 < ntiles) load_tile<D, R>(a, raw, (it + 2) * kExtKeys, kq, o, qo0, prefix, L, req, kv0, kend);
    }
    __syncthreads();
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
    hipLaunchKernelGGL((extend_kernel<DD, RR>), grid, dim3(256), lds, stream, a);                       \
    return hipGetLastError();                                                                           \
  }
  ROLAQ_EXT(256, 32)
  ROLAQ_EXT(512, 64)
#undef ROLAQ_EXT
  return hipErrorInvalidValue;
}
