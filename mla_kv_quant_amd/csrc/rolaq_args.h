// Kernel argument blocks shared by the host launchers and the C ABI layer.
#pragma once

#include <stdint.h>

namespace rolaq {

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint8_t* codes;
  const float* params;
  const uint16_t* rope;
  const uint16_t* hp;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  int page_shift;
  const int64_t* seq_lens;
  const int64_t* req_idx;
  const int32_t* num_kv_splits;
  int split_cap;  // request b uses min(num_kv_splits[b], split_cap) splits
  int neutral;    // 1: split nq carries the window split's neutral partial; 0: no such partial (fused call)
  int S1;        // max_kv_splits + 1
  int max_reqs;  // requests with ring rows; req_idx outside [0, max_reqs) reads no window rows
  int B, H, P, W;
  float sm_scale;
  float* logits;  // [B, H, S1, D]
  float* lse;     // [B, H, S1]
};

struct AuxArgs {
  const uint16_t* k_pe;
  int64_t pe_s0, pe_s1;
  const int64_t* seq_lens;
  const int64_t* positions;
  const int64_t* req_idx;
  int R, P, W, max_reqs;
  uint16_t* rope;
  uint16_t* hp;
  int32_t* row_of_slot;
  int32_t* owner_of_row;
};

struct WriterArgs {
  const uint16_t* x;
  int64_t xs;
  const uint16_t* rt;  // R_eff^T [D, D] bf16
  const int64_t* loc;
  int64_t n;
  float thr, kscale;
  uint8_t* codes;
  float* params;
  const uint16_t* k_pe;
  int64_t pe_s0, pe_s1;
  const int64_t* seq_lens;
  const int64_t* positions;
  const int64_t* req_idx;
  int R, P, W, max_reqs;
  uint16_t* rope;
  uint16_t* hp;
  int32_t* row_of_slot;
  int32_t* owner_of_row;
  int nstripes;
  int pe_vec;  // k_pe rows copied as dword pairs (set by the launcher)
  // kv_a_layernorm fused in front of the rotation: x is the pre-norm kv_a
  // row, gamma the norm weight [D] (bf16), or null for no norm; y [n, ys]
  // receives the normalized rows (bf16), or null
  const uint16_t* gamma;
  float eps;
  uint16_t* y;
  int64_t ys;
};

struct ExtendArgs {
  const uint16_t* q;        // [T, H, D + R] bf16, strides (q_st, q_sh)
  int64_t q_st, q_sh;
  const uint16_t* kc;       // chunk keys [T, D + R] bf16, row stride kc_st
  int64_t kc_st;
  const int32_t* qo_indptr;  // [B + 1] chunk token offsets
  const int32_t* kv_indptr;  // prefix page (or token) lists
  const int32_t* kv_indices;
  int page_shift;
  const int64_t* prefix_lens;
  const int64_t* req_idx;
  const uint8_t* codes;
  const float* params;
  const uint16_t* rope;
  const uint16_t* hp;
  int B, H, P, W;
  int max_reqs;             // req_idx outside [0, max_reqs) reads no window rows
  float sm_scale;
  uint16_t* ws;             // workspace: key rows [ws_rows, D + R] bf16 (gathered per call)
  int64_t ws_rows;
  uint16_t* out;            // [T, H, D] bf16, strides (o_st, o_sh)
  int64_t o_st, o_sh;
};

struct AssembleArgs {
  const int64_t* slots;       // [n] token slots
  int64_t n;
  const uint8_t* codes;
  const float* params;
  const uint16_t* rope;
  const uint16_t* hp;
  const int32_t* row_of_slot;
  const int32_t* owner_of_row;
  const uint16_t* rot;        // R_eff [D, D] bf16 row-major, or null (rotated frame)
  int R;
  uint16_t* out;              // [n, out_st] bf16: latent (D) then rope (R)
  int64_t out_st;
};

}  // namespace rolaq

// Host launchers (defined next to their kernels).
#include <hip/hip_runtime.h>
// stages: kStagePartials (split partials + LSE), kStageMerge (LSE merge -> out), or both
constexpr int kStagePartials = 1, kStageMerge = 2;
hipError_t rolaq_launch_decode(const rolaq::DecodeArgs& a, int D, int R, int max_splits, uint16_t* out,
                               int64_t o_sb, int64_t o_sh, int stages, hipStream_t stream);
// Blocks of 16 * head-groups heads that one (sequence, split) of decode launches.
int rolaq_decode_head_blocks(int D, int H);
// Device address, on the current device, of the allocation-free decode's
// static workspace of kNoAllocScratchBytes bytes (looked up once per device).
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
hipError_t rolaq_noalloc_scratch(void** ptr);
hipError_t rolaq_launch_pack_f32(const float* x, int64_t xs, const int32_t* slots, int64_t n, int D,
                                 float thr, float kscale, uint8_t* codes, float* params, hipStream_t stream);
hipError_t rolaq_launch_pack_bf16_aux(const uint16_t* x, int64_t xs, const int64_t* loc, int64_t n, int D,
                                      float thr, float kscale, uint8_t* codes, float* params,
                                      const rolaq::AuxArgs& aux, hipStream_t stream);
hipError_t rolaq_launch_prepare_splits(const int32_t* splits, int32_t* quant, int32_t* merge, int64_t n,
                                       hipStream_t stream);
hipError_t rolaq_launch_writer(const rolaq::WriterArgs& a, int D, int num_cus, hipStream_t stream);
hipError_t rolaq_launch_extend(const rolaq::ExtendArgs& a, int D, int R, int max_q_len, hipStream_t stream);
hipError_t rolaq_launch_assemble(const rolaq::AssembleArgs& a, int D, hipStream_t stream);
