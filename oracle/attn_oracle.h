/*
 * CPU oracle for the paged-attention hot path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker, never the product: only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 * The shipped path (libccinfer_attn.so) never links or calls it.
 *
 * It restates, in plain C with fp32 accumulation, the algorithm of the
 * reference's attention path (7QiC/ccInfer):
 *   - bf16 <-> fp32 conversion, round-to-nearest-even (the semantics of
 *     __float2bfloat16_rn used throughout the reference kernels);
 *   - orc_kv_base_offset      : src/kernel/attention/attn_common.cuh:7-27
 *   - orc_write_kv_cache      : src/kernel/attention/write_kv_cache.cu:12-34
 *   - orc_decode_attention    : tests/kernel/test_decode_attn.cu:24-86 (math) with the
 *                               edge cases of src/kernel/attention/decode_attn.cu:384-473
 *   - orc_prefill_attention   : src/kernel/attention/prefill_attn.cu:80-241 with the
 *                               causal contract of src/backend/params.h:140-146
 *   - orc_naive_attention     : tests/kernel/test_naive_attn.cu:16-65 (dense causal)
 *   - orc_lcg_fill            : tests/kernel/test_naive_attn.cu:67-74
 *   - orc_split_qkv           : src/kernel/elementwise/elementwise.cu:34-64
 *   - orc_rms_norm            : src/kernel/norm/rms_norm.cu:22-88 with the reduction order
 *                               of src/kernel/cuda_common.cuh:14-62
 *   - orc_rope                : src/kernel/pos/rope.cu:14-43
 *   - orc_qkv_prologue        : the sequence of src/model/qwen3/qwen3_model.cpp:174-244
 *   - orc_build_batch_metadata: the arrays of src/worker/batch_translator.cpp:213-302 and
 *                               the checks of src/model/model_runner.h:102-171
 *   - orc_*_fp8 / orc_*e4m3*  : an fp8 (OCP E4M3) KV cache with one fp32 scale per cache
 *                               row. No counterpart in the reference (its cache is bf16;
 *                               src/base/traits.h:117-124 anticipates other profiles):
 *                               pinned by torch.float8_e4m3fn and closed forms instead.
 *
 * Every function is pinned by tests/test_oracle.py (known-answer vectors from the
 * reference tests, closed forms, torch's float64 scaled_dot_product_attention as an
 * independent library routine, and cross-identities between the functions).
 *
 * bf16 values travel as uint16_t bit patterns.
 */
#ifndef CCINFER_ATTN_ORACLE_H
#define CCINFER_ATTN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_array(const float* src, uint16_t* dst, int64_t n);

/* Returns 1 and sets *out when ctx_pos maps to a valid cache row, else 0. */
int orc_kv_base_offset(int ctx_pos, int kv_head, int head_dim, int num_kv_heads,
                       int cache_block_size, int max_blocks_per_req,
                       const int32_t* req_blocks, int64_t* out);

/* Scatter k_new/v_new[t][h][d] into cache[slot_mapping[t]][h][d]; slots outside
 * [0, max_slots) are skipped. */
void orc_write_kv_cache(const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_cache,
                        uint16_t* v_cache, const int32_t* slot_mapping, int total_tokens,
                        int n_kv_heads, int head_dim, int max_slots);

/* out: fp32 [batch][num_q_heads][head_dim]. nthreads <= 1 runs single-threaded. */
void orc_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                          const int32_t* block_table, const int32_t* context_lens, float* out,
                          int batch_size, int max_blocks_per_req, int num_q_heads,
                          int num_kv_heads, int head_dim, int cache_block_size, int nthreads);

/* Same as orc_decode_attention restricted to the (request, q_head) pairs listed in
 * pairs[2*i], pairs[2*i+1] (used to time a bounded sample of a large batch). */
void orc_decode_attention_pairs(const uint16_t* q, const uint16_t* k_cache,
                                const uint16_t* v_cache, const int32_t* block_table,
                                const int32_t* context_lens, float* out, int batch_size,
                                int max_blocks_per_req, int num_q_heads, int num_kv_heads,
                                int head_dim, int cache_block_size, const int32_t* pairs,
                                int num_pairs, int nthreads);

/* out: fp32 [total_query_tokens][num_q_heads][head_dim]; rows the reference leaves
 * unwritten (malformed metadata) are left untouched. */
void orc_prefill_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           const int32_t* block_table, const int32_t* query_start_loc,
                           const int32_t* context_lens, float* out, int batch_size,
                           int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                           int num_kv_heads, int head_dim, int cache_block_size, int nthreads);

/* Same as orc_prefill_attention restricted to the (query token, q_head) pairs listed. */
void orc_prefill_attention_pairs(const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, const int32_t* block_table,
                                 const int32_t* query_start_loc, const int32_t* context_lens,
                                 float* out, int batch_size, int total_query_tokens,
                                 int max_blocks_per_req, int num_q_heads, int num_kv_heads,
                                 int head_dim, int cache_block_size, const int32_t* pairs,
                                 int num_pairs, int nthreads);

/* Dense causal attention on contiguous q[T][Hq][D], k/v[T][Hkv][D]; out fp32. */
void orc_naive_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, float* out,
                         int num_tokens, int n_q_heads, int n_kv_heads, int head_dim);

/* The reference tests' LCG fill: values in [-0.5, 0.5) rounded to bf16. */
void orc_lcg_fill(uint16_t* data, int n, unsigned int seed);

/* Decode-side prologue (qwen3_model.cpp:174-244). */
void orc_split_qkv(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T, int nq,
                   int nkv, int hd);
void orc_rms_norm(const uint16_t* input, const uint16_t* weight, uint16_t* output, int rows,
                  int dim, float eps);
void orc_rope(uint16_t* q, uint16_t* k, const int32_t* positions, const float* rope_cache,
              int T, int nq, int nkv, int hd, int rotary_dim, int rope_cache_max_position);
void orc_qkv_prologue(const uint16_t* qkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                      const int32_t* positions, const float* rope_cache,
                      const int32_t* slot_mapping, uint16_t* q_out, uint16_t* k_tmp,
                      uint16_t* v_tmp, uint16_t* k_cache, uint16_t* v_cache, int T, int nq,
                      int nkv, int hd, int rope_cache_max_position, int max_slots, float eps);

/* Per-step attention metadata from compact per-item records (one item = one sequence of
 * the batch). item_flags: bit 0 = decode item (exactly one new token), bit 1 = sample the
 * item's last token (a prefill chunk that needs logits); decode items are always sampled.
 * item_block_start [B + 1] indexes `blocks`, the concatenated block tables (after this
 * step's allocation) of the items; `blocks` holds total_blocks entries, and an item whose
 * range does not lie inside it is treated as having no blocks. Returns 0, or 6 (InvalidArgument) when a check fails;
 * failing entries are written sanitised (slot -1, table entry -1). */
#define ORC_ITEM_DECODE 1
#define ORC_ITEM_SAMPLE 2
int orc_build_batch_metadata(const int32_t* item_kv_written, const int32_t* item_new_tokens,
                             const int32_t* item_flags, const int32_t* item_block_start,
                             const int32_t* blocks, int batch_size, int num_tokens,
                             int total_blocks, int max_blocks_per_req, int block_size,
                             int num_cache_blocks,
                             int32_t* positions, int32_t* slot_mapping, int32_t* block_table,
                             int32_t* query_start_loc, int32_t* context_lens,
                             int32_t* logits_indices);

/* fp8 KV cache: OCP E4M3 values, one fp32 scale per (slot, kv_head) row stored at
 * orc_fp8_scale_index(slot, kv_head) = ((slot / bs) * Hkv + kv_head) * bs + slot % bs. */
uint8_t orc_f32_to_e4m3(float x);
float orc_e4m3_to_f32(uint8_t b);
int64_t orc_fp8_scale_index(int slot, int kv_head, int num_kv_heads, int block_size);
float orc_fp8_row_scale(float amax);
void orc_quantize_row_fp8(const uint16_t* x, int n, uint8_t* q, float* scale);
void orc_write_kv_cache_fp8(const uint16_t* k_new, const uint16_t* v_new, uint8_t* k_cache,
                            uint8_t* v_cache, float* k_scale, float* v_scale,
                            const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                            int head_dim, int max_slots, int block_size);
void orc_decode_attention_fp8(const uint16_t* q, const uint8_t* k_cache, const uint8_t* v_cache,
                              const float* k_scale, const float* v_scale,
                              const int32_t* block_table, const int32_t* context_lens,
                              float* out, int batch_size, int max_blocks_per_req,
                              int num_q_heads, int num_kv_heads, int head_dim,
                              int cache_block_size, int nthreads);
void orc_prefill_attention_fp8(const uint16_t* q, const uint8_t* k_cache, const uint8_t* v_cache,
                               const float* k_scale, const float* v_scale,
                               const int32_t* block_table, const int32_t* query_start_loc,
                               const int32_t* context_lens, float* out, int batch_size,
                               int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                               int num_kv_heads, int head_dim, int cache_block_size,
                               int nthreads);

#ifdef __cplusplus
}
#endif

#endif
