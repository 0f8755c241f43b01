// C ABI of the packed-INT2 RoLaQ MLA path (declarations: include/rolaq_mla.h).
// Validates every argument on the host before any launch; allocates nothing.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/rolaq_mla.h"

#include "rolaq_args.h"

namespace {

thread_local char g_err[512] = "";

// Decode runs one block per 16 heads; this bounds the grid, not the kernels.
constexpr int kMaxHeads = 128;

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(ROLAQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  g_err[0] = '\0';
  return ROLAQ_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// The Lloyd scale constant: span / 3 * gain in float64, then cast to FP32
// (mla_quant/oscar.py:141-142 multiplies a Python float by an FP32 tensor).
float lloyd_kscale(double gain) {
  const double c0 = -1.5095585584640503, c3 = 1.5095585584640503;
  return static_cast<float>((c3 - c0) / 3.0 * gain);
}

bool good_params(float thr, double gain) {
  return std::isfinite(thr) && std::isfinite(gain) && thr > 0.f && gain > 0.0;
}

int cu_count() {
  static thread_local int dev = -1, cus = 0;
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess) return 256;
  if (d != dev) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || c <= 0) c = 256;
    dev = d;
    cus = c;
  }
  return cus;
}

}  // namespace

extern "C" {

const char* rolaq_last_error(void) { return g_err; }

int rolaq_abi_version(void) { return 4; }

int rolaq_scatter_pack_rows(const float* x, int64_t x_stride, const int32_t* slots, int64_t n, int D,
                            int group_size, float threshold, double gain, uint8_t* codes, float* params,
                            void* stream) {
  if (n < 0) return fail(ROLAQ_ERR_INVALID, "scatter_pack_rows: n < 0");
  if (n == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  if (group_size != 128) return fail(ROLAQ_ERR_INVALID, "scatter_pack_rows: group_size must be 128");
  if (D != 512 && D != 256) return fail(ROLAQ_ERR_INVALID, "scatter_pack_rows: D must be 256 or 512, got %d", D);
  if (!x || !slots || !codes || !params) return fail(ROLAQ_ERR_INVALID, "scatter_pack_rows: null pointer");
  if (x_stride < D || x_stride % 4 || !aligned(x, 16))
    return fail(ROLAQ_ERR_INVALID, "scatter_pack_rows: x must be 16-byte aligned with a row stride >= D, multiple of 4");
  if (!good_params(threshold, gain)) return fail(ROLAQ_ERR_INVALID, "scatter_pack_rows: invalid threshold/gain");
  if (!aligned(codes, 4) || !aligned(params, 8)) return fail(ROLAQ_ERR_INVALID, "scatter_pack_rows: misaligned cache buffers");
  return hip_status(rolaq_launch_pack_f32(x, x_stride, slots, n, D, threshold, lloyd_kscale(gain), codes, params,
                                          static_cast<hipStream_t>(stream)),
                    "scatter_pack_rows launch");
}

}  // extern "C"

namespace {

// Checks shared by the writer entry points; returns ROLAQ_OK or the failure.
int check_writer(const char* fn, const void* latent, int64_t latent_stride, const void* k_pe,
                 const void* rotation_t, const int64_t* loc, const int64_t* seq_lens, const int64_t* req_idx,
                 int D, int R, int P, int W, int max_reqs, float threshold, double gain, const uint8_t* codes,
                 const float* params, const void* rope_buf, const void* hp_c, const int32_t* row_of_slot,
                 const int32_t* owner_of_row) {
  if (!((D == 512 && R == 64) || (D == 256 && R == 32)))
    return fail(ROLAQ_ERR_INVALID, "%s: (D, R) must be (512, 64) or (256, 32), got (%d, %d)", fn, D, R);
  if (!latent || !k_pe || !loc || !seq_lens || !req_idx || !codes || !params || !rope_buf || !hp_c ||
      !row_of_slot || !owner_of_row)
    return fail(ROLAQ_ERR_INVALID, "%s: null pointer", fn);
  if (latent_stride < D || latent_stride % 8 || latent_stride >= (1 << 24) || !aligned(latent, 16))
    return fail(ROLAQ_ERR_INVALID,
                "%s: latent must be 16-byte aligned with a row stride >= D, multiple of 8, below 2^24", fn);
  if (rotation_t && !aligned(rotation_t, 16)) return fail(ROLAQ_ERR_INVALID, "%s: rotation must be 16-byte aligned", fn);
  if (P < 0 || W < 0 || max_reqs < 0) return fail(ROLAQ_ERR_INVALID, "%s: negative window or max_reqs", fn);
  if (!good_params(threshold, gain)) return fail(ROLAQ_ERR_INVALID, "%s: invalid threshold/gain", fn);
  if (!aligned(codes, 4) || !aligned(params, 8) || !aligned(hp_c, 8))
    return fail(ROLAQ_ERR_INVALID, "%s: misaligned cache buffers", fn);
  return ROLAQ_OK;
}

rolaq::WriterArgs writer_args(const void* latent, int64_t latent_stride, const void* k_pe, int64_t pe_stride0,
                              int64_t pe_stride1, const void* rotation_t, const int64_t* loc,
                              const int64_t* seq_lens, const int64_t* positions, const int64_t* req_idx,
                              int64_t n, int R, int P, int W, int max_reqs, float threshold, double gain,
                              uint8_t* codes, float* params, void* rope_buf, void* hp_c, int32_t* row_of_slot,
                              int32_t* owner_of_row) {
  rolaq::WriterArgs a{};
  a.x = static_cast<const uint16_t*>(latent);
  a.xs = latent_stride;
  a.rt = static_cast<const uint16_t*>(rotation_t);
  a.loc = loc;
  a.n = n;
  a.thr = threshold;
  a.kscale = lloyd_kscale(gain);
  a.codes = codes;
  a.params = params;
  a.k_pe = static_cast<const uint16_t*>(k_pe);
  a.pe_s0 = pe_stride0;
  a.pe_s1 = pe_stride1;
  a.seq_lens = seq_lens;
  a.positions = positions;
  a.req_idx = req_idx;
  a.R = R;
  a.P = P;
  a.W = W;
  a.max_reqs = max_reqs;
  a.rope = static_cast<uint16_t*>(rope_buf);
  a.hp = static_cast<uint16_t*>(hp_c);
  a.row_of_slot = row_of_slot;
  a.owner_of_row = owner_of_row;
  return a;
}

}  // namespace

extern "C" {

int rolaq_write_rows(const void* latent, int64_t latent_stride, const void* k_pe, int64_t pe_stride0,
                     int64_t pe_stride1, const void* rotation_t, const int64_t* loc, const int64_t* seq_lens,
                     const int64_t* positions, const int64_t* req_idx, int64_t n, int D, int R, int P, int W,
                     int max_reqs, float threshold, double gain, uint8_t* codes, float* params, void* rope_buf,
                     void* hp_c, int32_t* row_of_slot, int32_t* owner_of_row, void* stream) {
  if (n < 0) return fail(ROLAQ_ERR_INVALID, "write_rows: n < 0");
  if (n == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  const int rc = check_writer("write_rows", latent, latent_stride, k_pe, rotation_t, loc, seq_lens, req_idx, D, R, P,
                              W, max_reqs, threshold, gain, codes, params, rope_buf, hp_c, row_of_slot, owner_of_row);
  if (rc != ROLAQ_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!rotation_t) {
    rolaq::AuxArgs aux{static_cast<const uint16_t*>(k_pe), pe_stride0, pe_stride1, seq_lens, positions, req_idx,
                       R, P, W, max_reqs, static_cast<uint16_t*>(rope_buf), static_cast<uint16_t*>(hp_c),
                       row_of_slot, owner_of_row};
    return hip_status(rolaq_launch_pack_bf16_aux(static_cast<const uint16_t*>(latent), latent_stride, loc, n, D,
                                                 threshold, lloyd_kscale(gain), codes, params, aux, s),
                      "write_rows (un-rotated) launch");
  }
  const rolaq::WriterArgs a = writer_args(latent, latent_stride, k_pe, pe_stride0, pe_stride1, rotation_t, loc,
                                          seq_lens, positions, req_idx, n, R, P, W, max_reqs, threshold, gain, codes,
                                          params, rope_buf, hp_c, row_of_slot, owner_of_row);
  return hip_status(rolaq_launch_writer(a, D, cu_count(), s), "write_rows launch");
}

int rolaq_norm_write_rows(const void* kv_a, int64_t kv_a_stride, const void* norm_weight, float eps,
                          void* latent_out, int64_t latent_out_stride, const void* k_pe, int64_t pe_stride0,
                          int64_t pe_stride1, const void* rotation_t, const int64_t* loc, const int64_t* seq_lens,
                          const int64_t* positions, const int64_t* req_idx, int64_t n, int D, int R, int P, int W,
                          int max_reqs, float threshold, double gain, uint8_t* codes, float* params,
                          void* rope_buf, void* hp_c, int32_t* row_of_slot, int32_t* owner_of_row, void* stream) {
  if (n < 0) return fail(ROLAQ_ERR_INVALID, "norm_write_rows: n < 0");
  if (n == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  const int rc = check_writer("norm_write_rows", kv_a, kv_a_stride, k_pe, rotation_t, loc, seq_lens, req_idx, D, R,
                              P, W, max_reqs, threshold, gain, codes, params, rope_buf, hp_c, row_of_slot,
                              owner_of_row);
  if (rc != ROLAQ_OK) return rc;
  if (!rotation_t)
    return fail(ROLAQ_ERR_INVALID, "norm_write_rows: rotation_t is required (the identity for an un-rotated layer)");
  if (!norm_weight || !aligned(norm_weight, 16)) return fail(ROLAQ_ERR_INVALID, "norm_write_rows: norm_weight must be a 16-byte aligned pointer");
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(ROLAQ_ERR_INVALID, "norm_write_rows: eps must be finite and >= 0");
  if (latent_out &&
      (latent_out_stride < D || latent_out_stride % 8 || latent_out_stride >= (1 << 24) || !aligned(latent_out, 16)))
    return fail(ROLAQ_ERR_INVALID,
                "norm_write_rows: latent_out must be 16-byte aligned with a row stride >= D, multiple of 8, below 2^24");
  rolaq::WriterArgs a = writer_args(kv_a, kv_a_stride, k_pe, pe_stride0, pe_stride1, rotation_t, loc, seq_lens,
                                    positions, req_idx, n, R, P, W, max_reqs, threshold, gain, codes, params,
                                    rope_buf, hp_c, row_of_slot, owner_of_row);
  a.gamma = static_cast<const uint16_t*>(norm_weight);
  a.eps = eps;
  a.y = static_cast<uint16_t*>(latent_out);
  a.ys = latent_out_stride;
  return hip_status(rolaq_launch_writer(a, D, cu_count(), static_cast<hipStream_t>(stream)), "norm_write_rows launch");
}

int rolaq_prepare_gf_splits(const int32_t* splits, int32_t* quant, int32_t* merge, int64_t n, void* stream) {
  if (n < 0) return fail(ROLAQ_ERR_INVALID, "prepare_gf_splits: n < 0");
  if (n == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  if (!splits || !quant || !merge) return fail(ROLAQ_ERR_INVALID, "prepare_gf_splits: null pointer");
  return hip_status(rolaq_launch_prepare_splits(splits, quant, merge, n, static_cast<hipStream_t>(stream)),
                    "prepare_gf_splits launch");
}

}  // extern "C"

namespace {

// Validates the stage-1 arguments shared by decode_fwd and decode_partials and
// fills the kernel argument block.
int decode_args(const char* who, const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* codes,
                const float* params, const void* rope_buf, const void* hp_c, const int32_t* kv_indptr,
                const int32_t* kv_indices, int page_size, const int64_t* seq_lens, const int64_t* req_idx,
                int max_reqs, const int32_t* num_kv_splits, int max_kv_splits, int B, int H, int D, int R, int P,
                int W, float sm_scale, float* attn_logits, float* attn_lse, rolaq::DecodeArgs* a) {
  if (!((D == 512 && R == 64) || (D == 256 && R == 32)))
    return fail(ROLAQ_ERR_INVALID, "%s: (D, R) must be (512, 64) or (256, 32), got (%d, %d)", who, D, R);
  if (H <= 0 || H > kMaxHeads) return fail(ROLAQ_ERR_INVALID, "%s: head count %d outside 1..%d", who, H, kMaxHeads);
  if (!q || !codes || !params || !rope_buf || !hp_c || !kv_indptr || !kv_indices || !req_idx || !num_kv_splits ||
      !attn_logits || !attn_lse)
    return fail(ROLAQ_ERR_INVALID, "%s: null pointer", who);
  if (page_size < 1 || (page_size & (page_size - 1)))
    return fail(ROLAQ_ERR_INVALID, "%s: page_size must be a power of two, got %d", who, page_size);
  if (!seq_lens && page_size != 1) return fail(ROLAQ_ERR_INVALID, "%s: seq_lens required when page_size > 1", who);
  if (max_kv_splits < 1 || max_kv_splits > 4096) return fail(ROLAQ_ERR_INVALID, "%s: max_kv_splits out of range", who);
  if (P < 0 || W < 0 || P + W > 32) return fail(ROLAQ_ERR_INVALID, "%s: need 0 <= P, W and P + W <= 32", who);
  if (max_reqs < 0) return fail(ROLAQ_ERR_INVALID, "%s: max_reqs < 0", who);
  if (!aligned(attn_logits, 16)) return fail(ROLAQ_ERR_INVALID, "%s: attn_logits must be 16-byte aligned", who);
  if (!aligned(q, 16) || q_stride_b % 8 || q_stride_h % 8 || q_stride_h < D + R)
    return fail(ROLAQ_ERR_INVALID, "%s: q must be 16-byte aligned with strides multiple of 8 and q_stride_h >= D+R", who);
  if (!aligned(codes, 16) || !aligned(params, 16) || !aligned(rope_buf, 16) || !aligned(hp_c, 16))
    return fail(ROLAQ_ERR_INVALID, "%s: cache buffers must be 16-byte aligned", who);
  if (!(sm_scale > 0.f) || !std::isfinite(sm_scale)) return fail(ROLAQ_ERR_INVALID, "%s: invalid sm_scale", who);
  int shift = 0;
  while ((1 << shift) < page_size) ++shift;
  *a = rolaq::DecodeArgs{};
  a->q = static_cast<const uint16_t*>(q);
  a->q_sb = q_stride_b;
  a->q_sh = q_stride_h;
  a->codes = codes;
  a->params = params;
  a->rope = static_cast<const uint16_t*>(rope_buf);
  a->hp = static_cast<const uint16_t*>(hp_c);
  a->kv_indptr = kv_indptr;
  a->kv_indices = kv_indices;
  a->page_shift = shift;
  a->seq_lens = seq_lens;
  a->req_idx = req_idx;
  a->num_kv_splits = num_kv_splits;
  a->split_cap = max_kv_splits;
  a->neutral = 1;
  a->S1 = max_kv_splits + 1;
  a->max_reqs = max_reqs;
  a->B = B;
  a->H = H;
  a->P = P;
  a->W = W;
  a->sm_scale = sm_scale;
  a->logits = attn_logits;
  a->lse = attn_lse;
  return ROLAQ_OK;
}

// The split count the fused decode uses at most: enough quantized splits for
// one working block per compute unit over the batch's (sequence, head block)
// pairs, plus the window split, and never more than the caller's maximum.
// Every request then takes min(its num_kv_splits, this); the merged output
// does not depend on the split count (up to FP32 summation order).
int fused_split_cap(int B, int H, int D, int max_kv_splits) {
  const int64_t units = int64_t(B) * rolaq_decode_head_blocks(D, H);
  const int64_t quant = (cu_count() + units - 1) / units;
  const int64_t cap = (quant < 1 ? 1 : quant) + 1;
  return cap < max_kv_splits ? int(cap) : max_kv_splits;
}

// The fused call's use of its scratch: the capped split count, no neutral
// window-split partial, and the partials stored at a stride of the capped
// count rather than max_kv_splits + 1 (attn_logits [B, H, S1c, D] and
// attn_lse [B, H, S1c] from the start of the buffers, S1c = min(cap - 1,
// max_kv_splits) + 1 <= max_kv_splits + 1): the partials of one (sequence,
// head) stay contiguous whatever max_kv_splits is, instead of being spread
// over a buffer sized for the largest split count.
void fused_layout(rolaq::DecodeArgs* a, int B, int H, int D, int max_kv_splits) {
  a->split_cap = fused_split_cap(B, H, D, max_kv_splits);
  a->neutral = 0;
  a->S1 = std::max(std::min(a->split_cap - 1, max_kv_splits), 1) + 1;
}

}  // namespace

extern "C" {

int rolaq_decode_split_cap(int B, int H, int D, int max_kv_splits, int* cap) {
  if (B < 1 || H <= 0 || H > kMaxHeads || (D != 512 && D != 256) || max_kv_splits < 1 || max_kv_splits > 4096 ||
      !cap)
    return fail(ROLAQ_ERR_INVALID, "decode_split_cap: invalid B, H, D, max_kv_splits or null cap");
  *cap = fused_split_cap(B, H, D, max_kv_splits);
  g_err[0] = '\0';
  return ROLAQ_OK;
}

int rolaq_decode_fwd(const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* codes,
                     const float* params, const void* rope_buf, const void* hp_c, const int32_t* kv_indptr,
                     const int32_t* kv_indices, int page_size, const int64_t* seq_lens, const int64_t* req_idx,
                     int max_reqs, const int32_t* num_kv_splits, int max_kv_splits, int B, int H, int D, int R,
                     int P, int W,
                     float sm_scale, float* attn_logits, float* attn_lse, void* out, int64_t out_stride_b,
                     int64_t out_stride_h, void* stream) {
  if (B < 0) return fail(ROLAQ_ERR_INVALID, "decode_fwd: B < 0");
  if (B == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  rolaq::DecodeArgs a;
  const int rc = decode_args("decode_fwd", q, q_stride_b, q_stride_h, codes, params, rope_buf, hp_c, kv_indptr,
                             kv_indices, page_size, seq_lens, req_idx, max_reqs, num_kv_splits, max_kv_splits, B, H,
                             D, R, P, W, sm_scale, attn_logits, attn_lse, &a);
  if (rc != ROLAQ_OK) return rc;
  if (!out) return fail(ROLAQ_ERR_INVALID, "decode_fwd: null pointer");
  fused_layout(&a, B, H, D, max_kv_splits);
  return hip_status(rolaq_launch_decode(a, D, R, max_kv_splits, static_cast<uint16_t*>(out), out_stride_b,
                                        out_stride_h, kStagePartials | kStageMerge, static_cast<hipStream_t>(stream)),
                    "decode_fwd launch");
}

int rolaq_decode_fwd_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* codes,
                             const float* params, const void* rope_buf, const void* hp_c, const int32_t* kv_indptr,
                             const int32_t* kv_indices, int page_size, const int64_t* seq_lens,
                             const int64_t* req_idx, int max_reqs, const int32_t* num_kv_splits, int max_kv_splits,
                             int B, int H, int D, int R, int P, int W, float sm_scale, void* out,
                             int64_t out_stride_b, int64_t out_stride_h, void* stream) {
  if (B < 0) return fail(ROLAQ_ERR_INVALID, "decode_fwd_noalloc: B < 0");
  if (B == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  if (H <= 0 || (D != 512 && D != 256) || max_kv_splits < 1 || max_kv_splits > 4096)
    return fail(ROLAQ_ERR_INVALID, "decode_fwd_noalloc: invalid H, D or max_kv_splits");
  // workspace: attn_logits [B, H, S1, D] fp32, then attn_lse [B, H, S1] fp32 at a 256-byte boundary
  const uint64_t rows = uint64_t(B) * uint64_t(H) * uint64_t(max_kv_splits + 1);
  const uint64_t logit_bytes = (rows * uint64_t(D) * 4 + 255) / 256 * 256;
  const uint64_t need = logit_bytes + rows * 4;
  if (need > kNoAllocScratchBytes)
    return fail(ROLAQ_ERR_INVALID,
                "decode_fwd_noalloc: workspace of %llu bytes (B*H*(max_kv_splits+1)*(D+1)*4) exceeds the "
                "%llu-byte static scratch; use rolaq_decode_fwd with caller-owned attn_logits/attn_lse",
                (unsigned long long)need, (unsigned long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  const int hrc = hip_status(rolaq_noalloc_scratch(&ws), "decode_fwd_noalloc scratch lookup");
  if (hrc != ROLAQ_OK) return hrc;
  float* logits = static_cast<float*>(ws);
  float* lse = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + logit_bytes);
  rolaq::DecodeArgs a;
  const int rc = decode_args("decode_fwd_noalloc", q, q_stride_b, q_stride_h, codes, params, rope_buf, hp_c,
                             kv_indptr, kv_indices, page_size, seq_lens, req_idx, max_reqs, num_kv_splits,
                             max_kv_splits, B, H, D, R, P, W, sm_scale, logits, lse, &a);
  if (rc != ROLAQ_OK) return rc;
  if (!out) return fail(ROLAQ_ERR_INVALID, "decode_fwd_noalloc: null pointer");
  fused_layout(&a, B, H, D, max_kv_splits);
  return hip_status(rolaq_launch_decode(a, D, R, max_kv_splits, static_cast<uint16_t*>(out), out_stride_b,
                                        out_stride_h, kStagePartials | kStageMerge, static_cast<hipStream_t>(stream)),
                    "decode_fwd_noalloc launch");
}

int rolaq_decode_partials(const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* codes,
                          const float* params, const void* rope_buf, const void* hp_c, const int32_t* kv_indptr,
                          const int32_t* kv_indices, int page_size, const int64_t* seq_lens,
                          const int64_t* req_idx, int max_reqs, const int32_t* num_kv_splits, int max_kv_splits,
                          int B, int H, int D, int R, int P, int W, float sm_scale, float* attn_logits,
                          float* attn_lse, void* stream) {
  if (B < 0) return fail(ROLAQ_ERR_INVALID, "decode_partials: B < 0");
  if (B == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  rolaq::DecodeArgs a;
  const int rc = decode_args("decode_partials", q, q_stride_b, q_stride_h, codes, params, rope_buf, hp_c, kv_indptr,
                             kv_indices, page_size, seq_lens, req_idx, max_reqs, num_kv_splits, max_kv_splits, B, H,
                             D, R, P, W, sm_scale, attn_logits, attn_lse, &a);
  if (rc != ROLAQ_OK) return rc;
  return hip_status(rolaq_launch_decode(a, D, R, max_kv_splits, nullptr, 0, 0, kStagePartials,
                                        static_cast<hipStream_t>(stream)),
                    "decode_partials launch");
}

int rolaq_decode_merge(const float* attn_logits, const float* attn_lse, const int32_t* num_kv_splits,
                       int max_kv_splits, int B, int H, int D, void* out, int64_t out_stride_b,
                       int64_t out_stride_h, void* stream) {
  if (B < 0) return fail(ROLAQ_ERR_INVALID, "decode_merge: B < 0");
  if (B == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  if (D != 512 && D != 256) return fail(ROLAQ_ERR_INVALID, "decode_merge: D must be 256 or 512, got %d", D);
  if (H <= 0 || H > kMaxHeads) return fail(ROLAQ_ERR_INVALID, "decode_merge: head count %d outside 1..%d", H, kMaxHeads);
  if (max_kv_splits < 1 || max_kv_splits > 4096) return fail(ROLAQ_ERR_INVALID, "decode_merge: max_kv_splits out of range");
  if (!attn_logits || !attn_lse || !num_kv_splits || !out) return fail(ROLAQ_ERR_INVALID, "decode_merge: null pointer");
  if (!aligned(attn_logits, 16)) return fail(ROLAQ_ERR_INVALID, "decode_merge: attn_logits must be 16-byte aligned");
  rolaq::DecodeArgs a{};
  a.num_kv_splits = num_kv_splits;
  a.split_cap = max_kv_splits;
  a.neutral = 1;
  a.S1 = max_kv_splits + 1;
  a.B = B;
  a.H = H;
  a.logits = const_cast<float*>(attn_logits);
  a.lse = const_cast<float*>(attn_lse);
  return hip_status(rolaq_launch_decode(a, D, D == 512 ? 64 : 32, max_kv_splits, static_cast<uint16_t*>(out),
                                        out_stride_b, out_stride_h, kStageMerge, static_cast<hipStream_t>(stream)),
                    "decode_merge launch");
}

int rolaq_extend_fwd(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_chunk,
                     int64_t kc_stride_t, const int32_t* qo_indptr, const int32_t* kv_indptr,
                     const int32_t* kv_indices, int page_size, const int64_t* prefix_lens,
                     const int64_t* req_idx, int max_reqs, const uint8_t* codes, const float* params,
                     const void* rope_buf, const void* hp_c, int B, int H, int D, int R, int P, int W, int max_q_len,
                     float sm_scale, void* workspace, int64_t workspace_rows, int64_t key_rows, void* out,
                     int64_t out_stride_t, int64_t out_stride_h, void* stream) {
  if (B < 0 || max_q_len < 0) return fail(ROLAQ_ERR_INVALID, "extend_fwd: B < 0 or max_q_len < 0");
  if (B == 0 || max_q_len == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  if (!((D == 256 && R == 32) || (D == 512 && R == 64)))
    return fail(ROLAQ_ERR_INVALID, "extend_fwd: (D, R) must be (256, 32) or (512, 64), got (%d, %d)", D, R);
  if (H <= 0 || H > 4096) return fail(ROLAQ_ERR_INVALID, "extend_fwd: head count %d out of range", H);
  if (!q || !k_chunk || !qo_indptr || !kv_indptr || !kv_indices || !prefix_lens || !req_idx || !codes || !params ||
      !rope_buf || !hp_c || !out || !workspace)
    return fail(ROLAQ_ERR_INVALID, "extend_fwd: null pointer");
  if (workspace_rows < 1 || !aligned(workspace, 16))
    return fail(ROLAQ_ERR_INVALID, "extend_fwd: workspace must be 16-byte aligned with at least one row");
  if (key_rows < 0 || workspace_rows < key_rows)
    return fail(ROLAQ_ERR_INVALID,
                "extend_fwd: workspace of %lld rows is short of the %lld key rows (sum of prefix_lens and chunk "
                "lengths) it must hold",
                (long long)workspace_rows, (long long)key_rows);
  if (page_size < 1 || (page_size & (page_size - 1)))
    return fail(ROLAQ_ERR_INVALID, "extend_fwd: page_size must be a power of two, got %d", page_size);
  if (P < 0 || W < 0) return fail(ROLAQ_ERR_INVALID, "extend_fwd: negative window");
  if (max_reqs < 0) return fail(ROLAQ_ERR_INVALID, "extend_fwd: max_reqs < 0");
  if (!aligned(q, 16) || q_stride_t % 8 || q_stride_h % 8 || q_stride_h < D + R)
    return fail(ROLAQ_ERR_INVALID, "extend_fwd: q must be 16-byte aligned with strides multiple of 8 and q_stride_h >= D+R");
  if (!aligned(k_chunk, 16) || kc_stride_t % 8 || kc_stride_t < D + R)
    return fail(ROLAQ_ERR_INVALID, "extend_fwd: k_chunk must be 16-byte aligned with a row stride >= D+R, multiple of 8");
  if (!aligned(codes, 16) || !aligned(params, 16) || !aligned(rope_buf, 16) || !aligned(hp_c, 16))
    return fail(ROLAQ_ERR_INVALID, "extend_fwd: cache buffers must be 16-byte aligned");
  if (!(sm_scale > 0.f) || !std::isfinite(sm_scale)) return fail(ROLAQ_ERR_INVALID, "extend_fwd: invalid sm_scale");
  int shift = 0;
  while ((1 << shift) < page_size) ++shift;
  rolaq::ExtendArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.kc = static_cast<const uint16_t*>(k_chunk);
  a.kc_st = kc_stride_t;
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.page_shift = shift;
  a.prefix_lens = prefix_lens;
  a.req_idx = req_idx;
  a.codes = codes;
  a.params = params;
  a.rope = static_cast<const uint16_t*>(rope_buf);
  a.hp = static_cast<const uint16_t*>(hp_c);
  a.B = B;
  a.H = H;
  a.P = P;
  a.W = W;
  a.max_reqs = max_reqs;
  a.sm_scale = sm_scale;
  a.ws = static_cast<uint16_t*>(workspace);
  a.ws_rows = workspace_rows;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  return hip_status(rolaq_launch_extend(a, D, R, max_q_len, static_cast<hipStream_t>(stream)), "extend_fwd launch");
}

int rolaq_assemble_rows(const int64_t* slots, int64_t n, const uint8_t* codes, const float* params,
                        const void* rope_buf, const void* hp_c, const int32_t* row_of_slot,
                        const int32_t* owner_of_row, const void* rotation, int D, int R, void* out,
                        int64_t out_stride, void* stream) {
  if (n < 0) return fail(ROLAQ_ERR_INVALID, "assemble_rows: n < 0");
  if (n == 0) { g_err[0] = '\0'; return ROLAQ_OK; }
  if (!((D == 512 && R == 64) || (D == 256 && R == 32)))
    return fail(ROLAQ_ERR_INVALID, "assemble_rows: (D, R) must be (512, 64) or (256, 32), got (%d, %d)", D, R);
  if (!slots || !codes || !params || !rope_buf || !hp_c || !row_of_slot || !owner_of_row || !out)
    return fail(ROLAQ_ERR_INVALID, "assemble_rows: null pointer");
  if (!aligned(codes, 4) || !aligned(params, 8) || !aligned(rope_buf, 16) || !aligned(hp_c, 16) || !aligned(out, 16) ||
      (rotation && !aligned(rotation, 16)))
    return fail(ROLAQ_ERR_INVALID, "assemble_rows: misaligned buffers");
  if (out_stride < D + R || out_stride % 8)
    return fail(ROLAQ_ERR_INVALID, "assemble_rows: out row stride must be >= D + R and a multiple of 8");
  rolaq::AssembleArgs a{};
  a.slots = slots;
  a.n = n;
  a.codes = codes;
  a.params = params;
  a.rope = static_cast<const uint16_t*>(rope_buf);
  a.hp = static_cast<const uint16_t*>(hp_c);
  a.row_of_slot = row_of_slot;
  a.owner_of_row = owner_of_row;
  a.rot = static_cast<const uint16_t*>(rotation);
  a.R = R;
  a.out = static_cast<uint16_t*>(out);
  a.out_st = out_stride;
  return hip_status(rolaq_launch_assemble(a, D, static_cast<hipStream_t>(stream)), "assemble_rows launch");
}

}  // extern "C"


