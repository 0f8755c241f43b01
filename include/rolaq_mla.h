/*
 * rolaq_mla.h -- C ABI of the MI355X (gfx950) packed-INT2 RoLaQ MLA cache path.
 *
 * Every entry point takes raw device pointers, sizes and a HIP stream
 * (hipStream_t passed as void*; NULL = the null stream). The caller owns all
 * memory; nothing here allocates device memory, synchronises the stream or
 * branches on device data on the host, so every launch is graph-capturable.
 * Return value: ROLAQ_OK, or an error code with a message from
 * rolaq_last_error() (thread-local). Invalid arguments are rejected before any
 * launch and leave every buffer untouched.
 *
 * bf16 tensors are passed as void* holding IEEE bfloat16 bit patterns.
 * Strides are in elements. Index tensors use the dtypes SGLang hands over.
 *
 * Cache layout per layer (num_slots token slots, D = kv_lora_rank, R = rope
 * dim, NG = D / 128 quantization groups, P sink + W recent BF16 rows):
 *   codes        uint8  [num_slots, D / 4]  2-bit codes, LSB first: element
 *                j of the row at byte j / 4, bits 2 (j % 4) (group g = bytes
 *                32g .. 32g + 31).
 *   params       fp32   [num_slots, NG, 2]  (scale, zero) per group
 *   rope_buf     bf16   [num_slots, R]
 *   hp_c         bf16   [1 + max_reqs * (P + W), D]  rotated latent of the
 *                sink/recent rows; ring row of (req, pos) is
 *                1 + req*(P+W) + (pos < P ? pos : P + (pos - P) % W)
 *   row_of_slot  int32  [num_slots]  ring row or -1 (shared by all layers)
 *   owner_of_row int32  [1 + max_reqs * (P + W)]  slot owning a ring row
 */
#ifndef ROLAQ_MLA_H
#define ROLAQ_MLA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ROLAQ_OK 0
#define ROLAQ_ERR_INVALID 1 /* argument rejected; nothing launched */
#define ROLAQ_ERR_HIP 2     /* a HIP launch failed */

/* Message of the last error on the calling thread ("" if none). */
const char* rolaq_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int rolaq_abi_version(void);

/*
 * Quantize FP32 rows that are already in the rotated frame into the packed
 * cache: Lloyd INT2 codes (thresholds -t, 0, +t on the group-normalised value),
 * FP32 (scale, zero) per 128-group.
 * Replaces: scatter_pack_rows(x, slots, codes_buf, params_buf, group_size,
 *   lloyd_max, bits=2, quantizer_params=None)
 *   (deployment/patches/rolaq_sglang.patch:9-34; codec of
 *   mla_quant/oscar.py:120-144).
 * x: fp32 [n, D] with row stride x_stride; slots: int32 [n].
 * gain is the Lloyd stretch g; scale = fp32(span/3 * g) * std.
 * n == 0 is a no-op. D must be 256 or 512, group_size 128.
 */
int rolaq_scatter_pack_rows(const float* x, int64_t x_stride, const int32_t* slots, int64_t n,
                            int D, int group_size, float threshold, double gain,
                            uint8_t* codes, float* params, void* stream);

/*
 * Fused cache writer: rotate each latent row by the layer's rotation on bf16
 * MFMA (FP32 accumulate), quantize + pack it, and store the BF16 rope key,
 * the BF16 rotated row of sink/recent tokens and the ring ownership maps.
 * Replaces: try_fast_decode_store(pool, layer_id, loc, c_kv, k_pe) ->
 *   _pack_and_aux (deployment/sglang/QuantKernel/mla_fused_writer.py:16-51,
 *   54-107, 110-224), generalised to prefill chunks (positions given).
 * latent: bf16 [n, D] (row stride latent_stride); k_pe: bf16 [n, R] with
 * strides (pe_stride0, pe_stride1); rotation_t: bf16 [D, D] holding the
 * transpose of R_eff = bf16(R) (row j = column j of R), or NULL for an
 * un-rotated layer. loc/seq_lens/req_idx: int64 [n]; positions: int64 [n] or
 * NULL (then position = seq_len - 1, a decode step). A row keeps a ring row
 * iff (pos < P or pos >= seq_len - W) and 0 <= req < max_reqs and slot > 0.
 * Rows with slot 0 (graph padding) write codes/params only.
 */
int rolaq_write_rows(const void* latent, int64_t latent_stride, const void* k_pe,
                     int64_t pe_stride0, int64_t pe_stride1, const void* rotation_t,
                     const int64_t* loc, const int64_t* seq_lens, const int64_t* positions,
                     const int64_t* req_idx, int64_t n, int D, int R, int P, int W, int max_reqs,
                     float threshold, double gain, uint8_t* codes, float* params, void* rope_buf,
                     void* hp_c, int32_t* row_of_slot, int32_t* owner_of_row, void* stream);

/*
 * kv_a_layernorm fused in front of the writer: every row of kv_a (the
 * pre-norm compressed latent, bf16 [n, D], row stride kv_a_stride) becomes
 *   c = bf16(norm_weight * bf16(x * rsqrt(mean(x^2) + eps)))
 * (FP32 statistics) and is then rotated, quantized and stored exactly as
 * rolaq_write_rows stores c. latent_out (bf16 [n, D], row stride
 * latent_out_stride) receives c when not NULL (the un-rotated latent that
 * an MHA prefill feeds to kv_b_proj). norm_weight: bf16 [D]. rotation_t is
 * required (pass the identity for an un-rotated layer: the products stay exact).
 * Replaces: self.kv_a_layernorm(kv_a) followed by try_fast_decode_store
 *   (norm: DeepseekV2RMSNorm.forward, transformers
 *   models/deepseek_v2/modeling_deepseek_v2.py:166-171, whose output the
 *   reference's quantizer hooks, mla_quant/objectives.py:25-29 and
 *   mla_quant/calibrate.py:40; writer as rolaq_write_rows).
 */
int rolaq_norm_write_rows(const void* kv_a, int64_t kv_a_stride, const void* norm_weight, float eps,
                          void* latent_out, int64_t latent_out_stride, const void* k_pe,
                          int64_t pe_stride0, int64_t pe_stride1, const void* rotation_t,
                          const int64_t* loc, const int64_t* seq_lens, const int64_t* positions,
                          const int64_t* req_idx, int64_t n, int D, int R, int P, int W,
                          int max_reqs, float threshold, double gain, uint8_t* codes, float* params,
                          void* rope_buf, void* hp_c, int32_t* row_of_slot, int32_t* owner_of_row,
                          void* stream);

/*
 * quant[i] = max(splits[i] - 1, 1); merge[i] = quant[i] + 1 (one launch).
 * Replaces: prepare_gf_splits(splits, quant, merge)
 *   (deployment/patches/rolaq_sglang.patch:81-92). int32 [n] each.
 */
int rolaq_prepare_gf_splits(const int32_t* splits, int32_t* quant, int32_t* merge, int64_t n,
                            void* stream);

/*
 * Absorbed MLA decode attention over the packed cache, split-K + LSE merge.
 * Replaces: packed_mla_decode_gf_fwd(q, ..., pool, max_kv_splits, attn_logits,
 *   attn_lse, ...) with its quantized stage 1, _fwd_hp_window_stage1 and the
 *   stage-2 merge (call site deployment/patches/rolaq_sglang.patch:51-111).
 * q: bf16 [B, H, D + R] = (q_lat | q_rope), strides (q_stride_b, q_stride_h).
 * Token t of request b lives in slot
 *   kv_indices[kv_indptr[b] + t / page_size] * page_size + t % page_size
 * (page_size a power of two; 1 = SGLang's token-level kv_indices).
 * seq_lens: int64 [B] or NULL (then L_b = kv_indptr[b+1] - kv_indptr[b],
 * page_size must be 1). req_idx: int64 [B] ring-row request index; a request
 * outside [0, max_reqs) has no ring rows (the writer stores none for it) and
 * is read entirely from its codes. hp_c must hold 1 + max_reqs * (P + W) rows.
 * Cache rows are the reference's stored rows: an INT2 row is
 * bf16((code - zero) * scale) (FP32 arithmetic, then rounded to bf16), a
 * window row (t < P or t >= L_b - W) the hp_c ring row. Window rows are read
 * by position, which matches the writer's ring as long as a request's
 * positions are written in order (SGLang serves RoLaQ with its radix cache
 * disabled, deployment/serve.py:149).
 * num_kv_splits: int32 [B] requested splits ns_b (1 <= ns_b <= max_kv_splits);
 * request b uses ns'_b = min(ns_b, cap) splits, cap as rolaq_decode_split_cap
 * returns it (about one working block per compute unit: more splits only
 * add partials to write and merge, and SGLang reads only the merged output;
 * the output does not depend on the split count beyond FP32 summation order).
 * Positions P <= t < L_b - W and the window rows are split over
 * nq_b = max(ns'_b - 1, 1) splits (the window rows go with split 0); the
 * reference's separate window split has no partial of its own here.
 * attn_logits (fp32, 16-byte aligned, at least B * H * (max_kv_splits + 1) * D
 * floats) and attn_lse (fp32, at least B * H * (max_kv_splits + 1)) are
 * scratch: the call uses their first B * H * S1c * D and B * H * S1c floats as
 * [B, H, S1c, D] and [B, H, S1c], S1c = min(cap - 1, max_kv_splits) + 1, and
 * writes partials (normalised output, natural-log LSE; empty splits 0 / -1e4)
 * to slots 0 .. nq_b - 1 of each (b, h). The merged output goes to out: bf16
 * [B, H, D] with strides (out_stride_b, out_stride_h), in the rotated frame.
 * Supported shapes: (D, R) = (512, 64) or (256, 32), 1 <= H <= 128; window
 * P + W <= 32. Latent values (query, stored levels, window rows) are carried
 * in fp16 on the way to the MFMAs: magnitudes above 65504 make that
 * request's output non-finite.
 */
int rolaq_decode_fwd(const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* codes,
                     const float* params, const void* rope_buf, const void* hp_c,
                     const int32_t* kv_indptr, const int32_t* kv_indices, int page_size,
                     const int64_t* seq_lens, const int64_t* req_idx, int max_reqs,
                     const int32_t* num_kv_splits, int max_kv_splits, int B, int H, int D, int R,
                     int P, int W, float sm_scale, float* attn_logits, float* attn_lse,
                     void* out, int64_t out_stride_b, int64_t out_stride_h, void* stream);

/*
 * rolaq_decode_fwd without the attn_logits / attn_lse workspace, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference: it exists only for those callers. Same arguments, rules and
 * results as rolaq_decode_fwd; the partials go to a static per-GPU scratch
 * array of 32 MiB held by the library until the process ends, so
 * B * H * (max_kv_splits + 1) * (D + 1) * 4 bytes (plus up to 255 bytes of
 * alignment) must fit in 32 MiB, else ROLAQ_ERR_INVALID. The call allocates
 * nothing. Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (other streams, other threads) race, and the array keeps the last
 * call's partials (no part of it needs clearing: each call writes every
 * partial it reads).
 */
int rolaq_decode_fwd_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* codes,
                             const float* params, const void* rope_buf, const void* hp_c,
                             const int32_t* kv_indptr, const int32_t* kv_indices, int page_size,
                             const int64_t* seq_lens, const int64_t* req_idx, int max_reqs,
                             const int32_t* num_kv_splits, int max_kv_splits, int B, int H, int D, int R,
                             int P, int W, float sm_scale, void* out, int64_t out_stride_b,
                             int64_t out_stride_h, void* stream);

/*
 * The split cap of rolaq_decode_fwd and rolaq_decode_fwd_noalloc on the
 * current device: ceil(CUs / (B * head blocks)) + 1, at most max_kv_splits
 * (a head block is 16 heads at D = 512 and up to 48 at D = 256), written to
 * *cap. Host only: no launch, no synchronisation. No counterpart in the
 * reference, whose stage 1 runs every requested split.
 */
int rolaq_decode_split_cap(int B, int H, int D, int max_kv_splits, int* cap);

/*
 * Stage 1 of rolaq_decode_fwd alone: the split partials and their LSE, with
 * the same arguments and rules (no output), every request at its requested
 * split count ns_b (no cap). Replaces the quantized stage-1
 * grid plus _fwd_hp_window_stage1 of packed_mla_decode_gf_fwd
 * (deployment/patches/rolaq_sglang.patch:94-111), for callers that merge
 * themselves or time the stages apart.
 */
int rolaq_decode_partials(const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* codes,
                          const float* params, const void* rope_buf, const void* hp_c,
                          const int32_t* kv_indptr, const int32_t* kv_indices, int page_size,
                          const int64_t* seq_lens, const int64_t* req_idx, int max_reqs,
                          const int32_t* num_kv_splits, int max_kv_splits, int B, int H, int D,
                          int R, int P, int W, float sm_scale, float* attn_logits, float* attn_lse,
                          void* stream);

/*
 * Stage 2 of rolaq_decode_fwd alone: out[b, h] = sum_s exp(lse_s - LSE) *
 * attn_logits[b, h, s] over the max(ns_b - 1, 1) + 1 partials of request b,
 * as bf16. Replaces the softmax-reduce stage that merges ns_merge splits
 * (ns_merge = quant + 1, deployment/patches/rolaq_sglang.patch:81-92).
 */
int rolaq_decode_merge(const float* attn_logits, const float* attn_lse, const int32_t* num_kv_splits,
                       int max_kv_splits, int B, int H, int D, void* out, int64_t out_stride_b,
                       int64_t out_stride_h, void* stream);

/*
 * Absorbed MLA extend (chunked prefill) attention over the packed cache.
 * Replaces: the packed pool's extend reader behind the MLA attention call of
 *   the patched forward_absorb (deployment/patches/rolaq_sglang.patch:208-235;
 *   kernel in the un-vendored fork), with the HF cache's row semantics
 *   (mla_quant/cache.py:1030-1039).
 * Sequence b has chunk tokens qo_indptr[b] .. qo_indptr[b+1]-1 at positions
 * prefix_lens[b] + j, over its prefix (slots from kv_indptr/kv_indices, pages
 * of page_size) and the chunk itself, causally. Prefix position t is read as
 * the BF16 window row (hp_c ring row of req_idx[b]) when t < P or
 * t >= prefix_lens[b] + chunk length - W, else dequantized from the INT2 row
 * ((code - zero) * scale, rounded to bf16); a request outside [0, max_reqs)
 * has no window rows. Chunk rows are k_chunk: bf16
 * [T, D + R] (latent | rope), row stride kc_stride_t.
 * q: bf16 [T, H, D + R] (q_lat | q_rope), strides (q_stride_t, q_stride_h).
 * out: bf16 [T, H, D], strides (out_stride_t, out_stride_h), rotated frame.
 * max_q_len >= every chunk length (sizes the grid). (D, R) = (256, 32) or
 * (512, 64).
 * workspace: caller-owned scratch of 16-bit elements [workspace_rows, D + R],
 * 16-byte aligned; the call first gathers every key row of the extended
 * sequences into it as fp16 (sequence b at rows koff_b .., koff_b = sum over
 * b' < b of prefix_lens[b'] + chunk length b'). key_rows is that sum over all
 * b, sum_b (prefix_lens[b] + chunk length b), as the caller knows it on the
 * host (SGLang: extend_prefix_lens_cpu and the token count): a workspace
 * shorter than key_rows is rejected (ROLAQ_ERR_INVALID, nothing launched).
 * Rows past workspace_rows are never written; a sequence whose rows do not
 * fit (key_rows short of the device-side sum) gets NaN outputs.
 * Latent values are carried in fp16 as for rolaq_decode_fwd.
 */
int rolaq_extend_fwd(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_chunk,
                     int64_t kc_stride_t, const int32_t* qo_indptr, const int32_t* kv_indptr,
                     const int32_t* kv_indices, int page_size, const int64_t* prefix_lens,
                     const int64_t* req_idx, int max_reqs, const uint8_t* codes, const float* params,
                     const void* rope_buf, const void* hp_c, int B, int H, int D, int R, int P, int W,
                     int max_q_len, float sm_scale, void* workspace, int64_t workspace_rows, int64_t key_rows,
                     void* out, int64_t out_stride_t, int64_t out_stride_h, void* stream);

/*
 * Cache rows as bf16 [latent | rope] rows (MHA-style prefill over a packed
 * prefix). Replaces: the fork's _assemble_rows_kernel
 *   (deployment/patches/rolaq_sglang.patch:5-6) and the un-rotation of the
 *   latent for kv_b_proj (deployment/sglang/srt/mem_cache/rolaq_mla.py:60-61).
 * Row i of out (stride out_stride elements) gets slot slots[i]: the BF16
 * window row if row_of_slot[slot] = r >= 0 and owner_of_row[r] == slot, else
 * the INT2 row dequantized ((code - zero) * scale, rounded to bf16); with
 * rotation (R_eff = bf16(R), [D, D] row-major) the latent is multiplied by
 * R_eff^T in FP32 and rounded to bf16 (rotate_quantize's cast order,
 * mla_quant/quantizer.py:117-122); without it the rotated frame is returned.
 * Columns D .. D + R - 1 are the rope row.
 */
int rolaq_assemble_rows(const int64_t* slots, int64_t n, const uint8_t* codes, const float* params,
                        const void* rope_buf, const void* hp_c, const int32_t* row_of_slot,
                        const int32_t* owner_of_row, const void* rotation, int D, int R, void* out,
                        int64_t out_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ROLAQ_MLA_H */
