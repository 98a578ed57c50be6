// Host-side entry points of the HIP kernels, used by the C ABI (capi.cpp).
// Every function only enqueues work on `stream`; none allocates memory or syncs.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ccinfer::hipk {

// ---- KV-cache write --------------------------------------------------------
hipError_t write_kv_cache(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                          const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                          int head_dim, int max_slots, hipStream_t stream);

// ---- decode ---------------------------------------------------------------
// Split-KV plan. Fixed mode: `splits` partitions of `split_tokens` tokens per (request,
// kv_head), sized from the longest possible context. Flat mode (decode batches of 4 or more
// requests): on the device, the batch's 32-token chunks laid end to end are cut into
// wave_target equal ranges per kv_head, one per wavefront, across request boundaries, so
// every wavefront streams the same number of tokens whatever the spread of context
// lengths; `slots` bounds the number of splits per kv_head. Past kFlatMaxItems requests,
// or at 4096 wavefronts and more, an index kernel writes the plan first; at 4096 and more
// it also snaps the ranges to request boundaries or gives each request its own ranges.
struct DecodePlan {
    int splits = 1;
    int split_tokens = 0;  // multiple of 32
    bool flat = false;  // the on-device flat plan (equal chunk ranges across items)
    int slots = 0;
    int wave_target = 0;
    bool group = false;  // one workgroup per (item, kv_head), parts merged in LDS
    bool flat_index = false;  // the flat plan's index kernel runs first
    bool flat_snap = false;   // the index reshapes the ranges (snapped or whole requests)
};

// Requests the flat plan's in-kernel scan covers; larger batches get the index kernel.
constexpr int kFlatMaxItems = 256;

// Returns the plan for a batch whose longest context is max_ctx tokens. allow_flat: the
// flat mode may be used (it resolves items through DecodeItems like the kernel does).
DecodePlan plan_decode(int num_items, int num_q_heads, int num_kv_heads, int head_dim,
                       int max_ctx, bool allow_flat, bool fp8 = false, bool allow_group = true);

// The plan for the single-token items of a prefill batch (at most num_items of them).
DecodePlan plan_decode_items(int num_items, int num_q_heads, int num_kv_heads, int head_dim,
                             int max_ctx, bool fp8 = false);

// Scratch bytes the split-KV decode needs for `num_items` query rows.
size_t decode_workspace_bytes(int num_items, int num_q_heads, int head_dim,
                              const DecodePlan& plan);

// Whether the MFMA split-KV decode kernel supports this shape (bf16 cache). Head dims that
// are multiples of 8 up to 128 (of 16 up to 256) run at the next MFMA size of 64 / 128 / 256
// with the missing dims zero.
bool decode_fast_supported(int num_q_heads, int num_kv_heads, int head_dim, int block_size);

// The MFMA head dim (64 / 128 / 256) that a head_dim runs at, or 0 if none does.
int decode_mfma_dim(int head_dim);

// The same for an fp8 cache: head dims 64, 128 and 256 only.
bool decode_fp8_supported(int num_q_heads, int num_kv_heads, int head_dim, int block_size);

// Query rows to attend, described either densely (item i is request i, query row i)
// or through a device list written by the prefill planner.
struct DecodeItems {
    int num_items = 0;                    // upper bound on items (grid size)
    const int32_t* item_count = nullptr;  // device: actual count (nullptr -> num_items)
    const int32_t* item_req = nullptr;    // device: request of item i (nullptr -> i)
    const int32_t* query_start_loc = nullptr;  // device: q row = qsl[req] (nullptr -> req)
    float denom_eps = 1e-6f;              // decode adds 1e-6 to the softmax sum; prefill 0
    bool zero_invalid = true;             // decode writes zeros for bad ctx; prefill skips
    // Optional: request r's new token (bf16 [B][Hkv][head_dim]) is written to the cache slot
    // of its last position (if that block id is >= 0 and the slot < max_slots) before it is
    // read; bf16 caches only.
    const void* new_k = nullptr;
    const void* new_v = nullptr;
    int max_slots = 0;
};

// Request b's new token (bf16 [B][Hkv][head_dim]) into the cache slot of its last position
// (the separate-launch form of DecodeItems::new_k / new_v).
hipError_t write_last_tokens(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                             const int32_t* block_table, const int32_t* context_lens,
                             int batch_size, int max_blocks_per_req, int n_kv_heads, int head_dim,
                             int max_slots, hipStream_t stream);

hipError_t decode_attention(const void* q, const void* k_cache, const void* v_cache,
                            const int32_t* block_table, const int32_t* context_lens, void* output,
                            const DecodeItems& items, int max_blocks_per_req, int num_q_heads,
                            int num_kv_heads, int head_dim, int block_size,
                            const DecodePlan& plan, void* workspace, hipStream_t stream);

// Decode of a batch whose requests may share cached prompt prefixes (leading block ids equal
// across table rows): each group's common prefix is read once per subgroup of up to 16 / G
// requests, the rest as in decode_attention. Plain decode semantics (zeros for invalid rows,
// 1e-6 in the denominator); bf16 cache, head dims of decode_fast_supported, G <= 8.
bool decode_shared_supported(int batch_size, int num_q_heads, int num_kv_heads, int head_dim,
                             int block_size);
size_t decode_shared_workspace_bytes(int batch_size, int max_blocks_per_req, int num_q_heads,
                                     int num_kv_heads, int head_dim);
hipError_t decode_attention_shared(const void* q, const void* k_cache, const void* v_cache,
                                   const int32_t* block_table, const int32_t* context_lens,
                                   void* output, int batch_size, int max_blocks_per_req,
                                   int num_q_heads, int num_kv_heads, int head_dim,
                                   void* workspace, hipStream_t stream);

// ---- prefill --------------------------------------------------------------
bool prefill_fast_supported(int num_q_heads, int num_kv_heads, int head_dim,
                            int max_blocks_per_req);

// The fp8 prefill (pipelined path, head_dim 64 / 128, table row staged in LDS).
bool prefill_fp8_supported(int head_dim, int max_blocks_per_req);

size_t prefill_workspace_bytes(int batch_size, int total_query_tokens, int max_blocks_per_req,
                               int num_q_heads, int num_kv_heads, int head_dim,
                               int block_size);

// Caller-owned side stream and events a mixed batch's decode items may run on (see
// ccinfer_prefill_attention_overlap).
struct PrefillOverlap {
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr;
    hipEvent_t join = nullptr;
};

hipError_t prefill_attention(const void* q, const void* k_cache, const void* v_cache,
                             const int32_t* block_table, const int32_t* query_start_loc,
                             const int32_t* context_lens, void* output, int batch_size,
                             int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                             int num_kv_heads, int head_dim, int block_size, void* workspace,
                             hipStream_t stream, const PrefillOverlap* overlap = nullptr);

// ---- fp8 (OCP E4M3) KV cache, one fp32 scale per cache row -------------------------
// Scale of (slot, kv_head) at ((slot / kFp8Block) * Hkv + kv_head) * kFp8Block + slot % 16.
constexpr int kFp8Block = 16;

hipError_t write_kv_cache_fp8(const void* k_new, const void* v_new, void* k_cache,
                              void* v_cache, float* k_scale, float* v_scale,
                              const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                              int head_dim, int max_slots, hipStream_t stream);

// Decode over the fp8 cache: the bf16 decode's plan, workspace and items, with K/V bytes
// dequantised in registers and the row scales applied to scores (K) and probabilities (V).
hipError_t decode_attention_fp8(const void* q, const void* k_cache, const void* v_cache,
                                const float* k_scale, const float* v_scale,
                                const int32_t* block_table, const int32_t* context_lens,
                                void* output, const DecodeItems& items, int max_blocks_per_req,
                                int num_q_heads, int num_kv_heads, int head_dim,
                                const DecodePlan& plan, void* workspace, hipStream_t stream);

// Prefill over the fp8 cache (head_dim 64 / 128, the pipelined path): the bf16 prefill's
// planner, workspace layout and semantics; single-token requests use decode_attention_fp8.
hipError_t prefill_attention_fp8(const void* q, const void* k_cache, const void* v_cache,
                                 const float* k_scale, const float* v_scale,
                                 const int32_t* block_table, const int32_t* query_start_loc,
                                 const int32_t* context_lens, void* output, int batch_size,
                                 int total_query_tokens, int max_blocks_per_req,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 void* workspace, hipStream_t stream,
                                 const PrefillOverlap* overlap = nullptr);

// ---- per-step batch metadata built on the device ------------------------------
constexpr int kItemDecode = 1;  // item flag: decode item (exactly one new token)
constexpr int kItemSample = 2;  // item flag: sample the item's last token

hipError_t build_batch_metadata(const int32_t* item_kv_written, const int32_t* item_new_tokens,
                                const int32_t* item_flags, const int32_t* item_block_start,
                                const int32_t* blocks, int batch_size, int num_tokens,
                                int total_blocks, int max_blocks_per_req, int block_size,
                                int num_cache_blocks, int32_t* positions, int32_t* slot_mapping,
                                int32_t* block_table, int32_t* query_start_loc,
                                int32_t* context_lens, int32_t* logits_indices, int32_t* status,
                                hipStream_t stream);

// ---- fused decode-side prologue: split QKV, q/k RMSNorm, RoPE, KV write -----
bool qkv_prologue_fast_supported(int head_dim);

hipError_t qkv_prologue(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                        const int32_t* positions, const void* rope_cache,
                        const int32_t* slot_mapping, void* q_out, void* k_cache, void* v_cache,
                        int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                        int rope_cache_max_position, int max_slots, float eps,
                        hipStream_t stream);

// ---- any-layout prefill on the MFMA tile kernel: head dims <= 256, any block size, any
// 2-byte alignment, any table length; single-token requests run as one-row tiles ----
bool prefill_any_supported(int num_q_heads, int num_kv_heads, int head_dim,
                           int max_blocks_per_req);
size_t prefill_any_workspace_bytes(int batch_size, int total_query_tokens, int num_q_heads,
                                   int num_kv_heads, int head_dim);
hipError_t prefill_attention_any(const void* q, const void* k_cache, const void* v_cache,
                                 const int32_t* block_table, const int32_t* query_start_loc,
                                 const int32_t* context_lens, void* output, int batch_size,
                                 int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                                 int num_kv_heads, int head_dim, int block_size,
                                 void* workspace, hipStream_t stream);

// Workspace bytes of a bf16 / fp8 decode call of this shape on the MFMA kernels; `staged`
// adds the q and output row copies a call with 2-byte-aligned q / output uses (defined with
// the C ABI, which lays those copies out).
size_t decode_bytes_for(int batch_size, int max_blocks_per_req, int num_q_heads,
                        int num_kv_heads, int head_dim, int cache_block_size, bool staged);

// Copies `elems` bf16 (a multiple of 8) between a 2-byte-aligned view and a 16-byte-aligned
// buffer: gather reads the view, scatter writes it.
hipError_t gather_rows(const void* src, void* dst, int64_t elems, hipStream_t stream);
hipError_t scatter_rows(const void* src, void* dst, int64_t elems, hipStream_t stream);

// Rewrites a [rows, max_blocks_per_req] table of (16·k)-token blocks as a
// [rows, max_blocks_per_req·k] table of 16-token blocks over the same cache rows.
hipError_t expand_block_table(const int32_t* block_table, int32_t* out, int rows,
                              int max_blocks_per_req, int k, hipStream_t stream);

}  // namespace ccinfer::hipk
