// Row quantizer/packer for rows that need no rotation on the GPU, and the
// split-count helper.
//
// pack_rows_kernel restates the Lloyd INT2 codec of mla_quant/oscar.py:130-144
// per 128-group (mean, std = sqrt(mean((x - mean)^2) + 1e-8), code = number of
// thresholds -t, 0, +t at or below (x - mean) / std, scale = fp32(span/3 g) std,
// zero = 1.5 - mean / scale) and writes the packed row. It serves
//  * scatter_pack_rows (deployment/patches/rolaq_sglang.patch:9-34): FP32 rows
//    already in the rotated frame;
//  * the writer of an un-rotated layer (mla_fused_writer.py:150 with r None):
//    bf16 rows plus the rope / window / ownership stores of _aux
//    (mla_fused_writer.py:36-51).
#include "rolaq_common.h"
#include "rolaq_args.h"

namespace rolaq {


__device__ __forceinline__ void row_window(const AuxArgs& x, int64_t row, int64_t slot, bool& keep,
                                           int64_t& ring) {
  const int64_t seq = x.seq_lens[row];
  const int64_t pos = x.positions ? x.positions[row] : seq - 1;
  const int64_t req = x.req_idx[row];
  keep = ((pos < x.P) || (pos >= seq - x.W)) && req < x.max_reqs && req >= 0 && slot > 0;
  const int64_t inner = pos < x.P ? pos : x.P + (pos - x.P > 0 ? pos - x.P : 0) % (x.W > 0 ? x.W : 1);
  ring = 1 + req * (x.P + x.W) + inner;
}

// One row per D/8 lanes, 8 consecutive elements per lane.
template <int D, typename T, bool AUX>
__global__ __launch_bounds__(256) void pack_rows_kernel(const T* __restrict__ x, int64_t xs,
                                                        const int32_t* __restrict__ slots32,
                                                        const int64_t* __restrict__ slots64,
                                                        int64_t n, float thr, float kscale,
                                                        uint8_t* __restrict__ codes,
                                                        float* __restrict__ params, AuxArgs aux) {
  constexpr int LPR = D / 8;
  constexpr int RPW = 64 / LPR;
  constexpr int NG = D / 128;
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
  if (row >= n) return;  // all lanes of a row share it, so shuffles stay within live rows
  const int l = lane % LPR;
  const int g = l / 16, e0 = 8 * (l % 16);
  const int64_t slot = slots32 ? (int64_t)slots32[row] : slots64[row];
  float v[8];
  if constexpr (sizeof(T) == 4) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(x + row * xs + 8 * l);
    const f32x4 b = *reinterpret_cast<const f32x4*>(x + row * xs + 8 * l + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4*>(x + row * xs + 8 * l);
    v[0] = bf16_lo(a.x); v[1] = bf16_hi(a.x); v[2] = bf16_lo(a.y); v[3] = bf16_hi(a.y);
    v[4] = bf16_lo(a.z); v[5] = bf16_hi(a.z); v[6] = bf16_lo(a.w); v[7] = bf16_hi(a.w);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += v[i];
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o);
  const float mean = s * (1.0f / 128.0f);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) { v[i] -= mean; q = fmaf(v[i], v[i], q); }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) q += __shfl_xor(q, o);
  const float std_ = sqrtf(q * (1.0f / 128.0f) + 1e-08f);
  // code = #{-t, 0, t <= (x - mean) / std} (correctly rounded quotient,
  // oscar.py:135-140), compared through the row's thresholds on x - mean
  const double sd = (double)std_;
  const float ylo = y_threshold(sd, below_midpoint(-thr), threshold_inclusive(-thr));
  const float y0 = y_threshold(sd, below_midpoint(0.0f), true);
  const float yhi = y_threshold(sd, below_midpoint(thr), threshold_inclusive(thr));
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t c = uint32_t(v[i] >= ylo) + uint32_t(v[i] >= y0) + uint32_t(v[i] >= yhi);
    bits |= c << (2 * i);
  }
  // elements 8l .. 8l+7 of the row: bytes 2l, 2l+1 (element j at byte j/4, bits 2(j%4))
  uint16_t* dst = reinterpret_cast<uint16_t*>(codes + slot * (D / 4)) + l;
  *dst = uint16_t(bits);
  if ((l & 15) == 0) {
    const float scale = kscale * std_;
    const float zero = kZeroOffset - mean / scale;
    *reinterpret_cast<f32x2*>(params + slot * 2 * NG + 2 * g) = f32x2{scale, zero};
  }
  if constexpr (AUX) {
    bool keep;
    int64_t ring;
    row_window(aux, row, slot, keep, ring);
    if (keep) {
      // bf16 of the (un-rotated) row: the input itself
      *reinterpret_cast<u32x4*>(aux.hp + ring * D + 8 * l) =
          *reinterpret_cast<const u32x4*>(x + row * xs + 8 * l);
    }
    if (slot > 0) {
      for (int r = l; r < aux.R; r += LPR) aux.rope[slot * aux.R + r] = aux.k_pe[row * aux.pe_s0 + r * aux.pe_s1];
      if (l == 0) {
        aux.row_of_slot[slot] = keep ? int32_t(ring) : -1;
        if (keep) aux.owner_of_row[ring] = int32_t(slot);
      }
    }
  }
}

__global__ void prepare_splits_kernel(const int32_t* __restrict__ splits, int32_t* __restrict__ quant,
                                      int32_t* __restrict__ merge, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t qv = max(splits[i] - 1, 1);
  quant[i] = qv;
  merge[i] = qv + 1;
}

}  // namespace rolaq

hipError_t rolaq_launch_pack_f32(const float* x, int64_t xs, const int32_t* slots, int64_t n, int D,
                                 float thr, float kscale, uint8_t* codes, float* params,
                                 hipStream_t stream) {
  using namespace rolaq;
  AuxArgs aux{};
  const int rows_per_block = 4 * (64 / (D / 8));
  const dim3 grid((unsigned)((n + rows_per_block - 1) / rows_per_block));
  if (D == 512)
    hipLaunchKernelGGL((pack_rows_kernel<512, float, false>), grid, dim3(256), 0, stream, x, xs, slots,
                       nullptr, n, thr, kscale, codes, params, aux);
  else if (D == 256)
    hipLaunchKernelGGL((pack_rows_kernel<256, float, false>), grid, dim3(256), 0, stream, x, xs, slots,
                       nullptr, n, thr, kscale, codes, params, aux);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t rolaq_launch_pack_bf16_aux(const uint16_t* x, int64_t xs, const int64_t* loc, int64_t n,
                                      int D, float thr, float kscale, uint8_t* codes, float* params,
                                      const rolaq::AuxArgs& aux, hipStream_t stream) {
  using namespace rolaq;
  const int rows_per_block = 4 * (64 / (D / 8));
  const dim3 grid((unsigned)((n + rows_per_block - 1) / rows_per_block));
  if (D == 512)
    hipLaunchKernelGGL((pack_rows_kernel<512, uint16_t, true>), grid, dim3(256), 0, stream, x, xs,
                       nullptr, loc, n, thr, kscale, codes, params, aux);
  else if (D == 256)
    hipLaunchKernelGGL((pack_rows_kernel<256, uint16_t, true>), grid, dim3(256), 0, stream, x, xs,
                       nullptr, loc, n, thr, kscale, codes, params, aux);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t rolaq_launch_prepare_splits(const int32_t* splits, int32_t* quant, int32_t* merge, int64_t n,
                                       hipStream_t stream) {
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(rolaq::prepare_splits_kernel, dim3(blocks), dim3(256), 0, stream, splits, quant, merge, n);
  return hipGetLastError();
}
