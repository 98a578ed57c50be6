/*
 * ccinfer_attn.h -- C ABI of the MI355X (gfx950) paged-attention hot path.
 *
 * Drop-in for the three kernel launchers of 7QiC/ccInfer declared in
 * src/kernel/cuda_kernels.h:61-84, with the same argument meaning, the same KV-cache layout
 * ([slot][num_kv_heads][head_dim] bf16, slot = block_id * cache_block_size + offset,
 * src/cache/kv_cache_storage.cpp:75-136) and the same block-table contract (int32
 * [batch][max_blocks_per_req], -1 padding, src/worker/batch_translator.cpp:213-293).
 *
 * Plain pointers and sizes only. All pointers except `stream` are device pointers.
 * `stream` is a hipStream_t (NULL = the default stream). Every call only enqueues work on
 * `stream`: no host synchronisation and no device allocation. Split-KV partials and the
 * prefill work list live in a caller-provided workspace sized by the *_workspace_size
 * queries (the reference launchers take no workspace; the C++ drop-in wrappers in
 * ccinfer_amd/csrc/dropin supply one owned per stream). Workspace contents need no
 * initialisation and are scratch between calls.
 *
 * Return value: 0 on success, otherwise the numeric value of the reference's
 * ccinfer::ErrorCode (src/base/error_code.h:8-45) -- the same codes the reference returns
 * through Result<void>.
 *
 * Thread safety: re-entrant. The C ABI keeps no global state except the per-device scratch
 * array of ccinfer_decode_attention_noalloc (and that array's cached device address), so
 * concurrent calls on different streams need only different workspaces -- apart from that
 * entry, whose calls on one GPU share the array. The C++ drop-in layer above it
 * (ccinfer_amd/csrc/dropin) adds one more piece of global state: the reference-signature
 * launchers' workspaces, one per (device, stream), reserved explicitly by
 * reserve_launcher_workspace and kept in a map behind a mutex (launches only read it; none
 * allocates). HipBackend holds its own reserved workspace and needs no global state.
 *
 * Alignment: the reference launchers accept any bf16 (2-byte aligned) view. The MFMA paths
 * move q, output and K/V cache rows in 16-byte pieces. A bf16 decode / prefill call whose
 * q or output view is only 2-byte aligned copies q (and, for prefill, output) into the
 * workspace, runs the MFMA kernels there and copies the output rows back (same bits as an
 * aligned call). A k_cache or v_cache pointer that is not 16-byte aligned runs the decode
 * MFMA kernels with 4-byte or 2-byte loads (same bits, ~1.1x / ~1.7x the time) and the
 * any-layout prefill tile kernel (~2.2x). The fp8 calls, which have the MFMA paths only, return
 * CCINFER_ERR_INVALID_ARGUMENT for any such pointer (and for k_scale / v_scale not 16-byte
 * aligned).
 */
#ifndef CCINFER_ATTN_H
#define CCINFER_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Numeric values of ccinfer::ErrorCode (src/base/error_code.h:8-45). */
enum ccinfer_status {
    CCINFER_OK = 0,
    CCINFER_ERR_DEVICE_OUT_OF_MEMORY = 1,  /* ErrorCode::CudaOutOfMemory   */
    CCINFER_ERR_LAUNCH_FAILED = 2,         /* ErrorCode::CudaLaunchFailed  */
    CCINFER_ERR_DEVICE_INVALID_VALUE = 3,  /* ErrorCode::CudaInvalidValue  */
    CCINFER_ERR_DEVICE_RUNTIME = 4,        /* ErrorCode::CudaRuntimeError  */
    CCINFER_ERR_INVALID_ARGUMENT = 6,      /* ErrorCode::InvalidArgument   */
    CCINFER_ERR_UNSUPPORTED = 26,          /* ErrorCode::Unsupported       */
    CCINFER_ERR_INTERNAL = 27              /* ErrorCode::InternalError     */
};

/* Replaces launch_write_kv_cache (src/kernel/cuda_kernels.h:80-83,
 * src/kernel/attention/write_kv_cache.cu:38-50).
 * k_new/v_new: [total_tokens][n_kv_heads][head_dim] bf16; k_cache/v_cache: one layer,
 * [max_slots][n_kv_heads][head_dim] bf16; slot_mapping: [total_tokens] int32. Tokens whose
 * slot is outside [0, max_slots) are skipped. Bit-exact copy. */
int ccinfer_write_kv_cache(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                           const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                           int head_dim, int max_slots, void* stream);

/* Fused attention prologue for one layer: replaces the five launches
 * launch_split_qkv, launch_rms_norm (q), launch_rms_norm (k), launch_rope and
 * launch_write_kv_cache (src/kernel/cuda_kernels.h, called in sequence by
 * src/model/qwen3/qwen3_model.cpp:174-244).
 * qkv: [num_tokens][(num_q_heads + 2 num_kv_heads) head_dim] bf16, the packed projection;
 * q_norm_weight, k_norm_weight: [head_dim] bf16 or NULL (no norm for that side);
 * positions: [num_tokens] int32; rope_cache: [rope_cache_max_position][head_dim/2] float
 * (cos, sin) pairs (src/model/rope_cache.cpp); q_out: [num_tokens][num_q_heads][head_dim]
 * bf16; k_cache/v_cache as in ccinfer_write_kv_cache. Rotation is skipped for positions
 * outside [0, rope_cache_max_position); tokens whose slot is outside [0, max_slots) write no
 * K/V. head_dim must be even and at most 1024; eps > 0 (backend.h:84). Results match the five reference kernels
 * in sequence (bf16 rounding between steps, the same reduction order). */
int ccinfer_qkv_prologue(const void* qkv, const void* q_norm_weight, const void* k_norm_weight,
                         const int32_t* positions, const void* rope_cache,
                         const int32_t* slot_mapping, void* q_out, void* k_cache, void* v_cache,
                         int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                         int rope_cache_max_position, int max_slots, float eps, void* stream);

/* Item flags of ccinfer_build_batch_metadata. */
#define CCINFER_ITEM_DECODE 1 /* decode item: exactly one new token, always sampled */
#define CCINFER_ITEM_SAMPLE 2 /* prefill chunk whose last token needs logits */

/* Builds one step's attention metadata on the device, replacing the host array building
 * and uploads of BatchTranslator::translate (src/worker/batch_translator.cpp:213-302,
 * 305-420) and ModelRunner's blocking copy-back validation (src/model/model_runner.h:
 * 102-171). Inputs (device, int32): per item i < batch_size the tokens already in the
 * cache (item_kv_written), the new tokens (item_new_tokens), flags (CCINFER_ITEM_*), and
 * its block list after this step's allocation, as blocks[item_block_start[i] ..
 * item_block_start[i + 1]) (total_blocks entries in all; blocks may be NULL when 0).
 * Outputs (device, int32): positions[num_tokens], slot_mapping[num_tokens],
 * block_table[batch_size][max_blocks_per_req] (-1 padded), query_start_loc[batch_size + 1],
 * context_lens[batch_size], logits_indices[batch_size] (-1 = no sample), exactly as the
 * reference's host loops write them; and status[0] = 0, or CCINFER_ERR_INVALID_ARGUMENT
 * when a check of model_runner.h fails (entries that fail are written as -1). The status
 * word is written by every call (no clearing needed) and is read by the caller when it
 * chooses -- the call itself never synchronises. */
int ccinfer_build_batch_metadata(const int32_t* item_kv_written, const int32_t* item_new_tokens,
                                 const int32_t* item_flags, const int32_t* item_block_start,
                                 const int32_t* blocks, int batch_size, int num_tokens,
                                 int total_blocks, int max_blocks_per_req, int block_size,
                                 int num_cache_blocks, int32_t* positions, int32_t* slot_mapping,
                                 int32_t* block_table, int32_t* query_start_loc,
                                 int32_t* context_lens, int32_t* logits_indices, int32_t* status,
                                 void* stream);

/* Workspace bytes ccinfer_decode_attention (and ccinfer_decode_attention_fp8) needs for this
 * batch shape; 0 for invalid shapes. The figure includes two copies of the
 * q rows, which only a call with a 2-byte-aligned q or output uses; an aligned call accepts
 * a workspace that much smaller. */
size_t ccinfer_decode_workspace_size(int batch_size, int max_blocks_per_req, int num_q_heads,
                                     int num_kv_heads, int head_dim, int cache_block_size);

/* Replaces launch_decode_attention (src/kernel/cuda_kernels.h:72-77,
 * src/kernel/attention/decode_attn.cu:515-570).
 * q, output: [batch_size][num_q_heads][head_dim] bf16; block_table: [batch_size]
 * [max_blocks_per_req] int32; context_lens: [batch_size] int32, including the current
 * token (whose K/V must already be written). cache_block_size must be 16 and head_dim one
 * of {32,64,80,96,112,120,128,192,256} (as in the reference); all of them run the MFMA
 * kernels (32, 96 and 192 in tiles of their own; 80 and 112-120 padded to 128 with
 * zeros), for any query group
 * size (groups above 16 heads run as several groups of at most 16 over the same KV head).
 * Unlike the reference, there is no
 * context-length ceiling (split-KV). Batches of at most 16 (request, q-head) rows with
 * table rows of at most 512 positions run in a single launch and need no workspace. */
int ccinfer_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                             const int32_t* block_table, const int32_t* context_lens,
                             void* output, int batch_size, int max_blocks_per_req,
                             int num_q_heads, int num_kv_heads, int head_dim,
                             int cache_block_size, void* workspace, size_t workspace_bytes,
                             void* stream);

/* One decode step: ccinfer_write_kv_cache of each request's new token into the slot of its
 * last position, then ccinfer_decode_attention. No single counterpart in the reference: it
 * replaces the pair launch_write_kv_cache + launch_decode_attention
 * (src/kernel/cuda_kernels.h:61-77) as src/model/qwen3/qwen3_model.cpp:230-262 issues them
 * for a decode batch, where token b is request b's newest position. k_new, v_new:
 * [batch_size][num_kv_heads][head_dim] bf16. The slot of request b's token is derived from
 * its table row: block_table[b][(ctx_b - 1) / 16] * 16 + (ctx_b - 1) % 16; rows with ctx_b
 * outside [1, max_blocks_per_req * 16], a negative block id there or a slot >= max_slots
 * write nothing (their output follows ccinfer_decode_attention). Requirement (true of any
 * decode batch): no other request of the batch reads those slots. On the MFMA path the
 * writes happen inside the decode launch (the wavefront that reads the slot writes it
 * first); otherwise a separate launch writes them first. Workspace as
 * ccinfer_decode_workspace_size. */
int ccinfer_decode_attention_write_kv(const void* q, const void* k_new, const void* v_new,
                                      void* k_cache, void* v_cache, const int32_t* block_table,
                                      const int32_t* context_lens, void* output, int batch_size,
                                      int max_blocks_per_req, int num_q_heads, int num_kv_heads,
                                      int head_dim, int cache_block_size, int max_slots,
                                      void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes ccinfer_decode_attention_shared_prefix needs for this batch shape. */
size_t ccinfer_decode_shared_workspace_size(int batch_size, int max_blocks_per_req,
                                            int num_q_heads, int num_kv_heads, int head_dim,
                                            int cache_block_size);

/* ccinfer_decode_attention for batches whose requests share cached prompt prefixes. No
 * single counterpart in the reference: its prefix cache hands several requests the same
 * leading block ids (KVCacheManager::lookup_prefix_cache, src/cache/kv_cache_manager.cpp:
 * 93-173, counted in BlockTable::shared_count, src/cache/block.h:85-97), and its decode
 * then reads those blocks once per request. Here the call finds, on the device, the groups
 * of requests whose table rows start with the same block ids and attends each group's
 * common prefix (whole 32-token chunks before every member's last position) once per
 * subgroup of up to 16 / (num_q_heads / num_kv_heads) requests, which fill one MFMA tile
 * together; positions after the prefix, and requests in no group, run as in
 * ccinfer_decode_attention, and the parts are combined by the log-sum-exp merge. Same
 * arguments, semantics and tolerance as ccinfer_decode_attention; a batch in which nothing
 * is shared gives the same bits. Shapes outside the fast path (query groups above 8 heads,
 * more than 2048 requests, misaligned views, non-16 blocks) run ccinfer_decode_attention
 * (the workspace size covers it). */
int ccinfer_decode_attention_shared_prefix(const void* q, const void* k_cache,
                                           const void* v_cache, const int32_t* block_table,
                                           const int32_t* context_lens, void* output,
                                           int batch_size, int max_blocks_per_req,
                                           int num_q_heads, int num_kv_heads, int head_dim,
                                           int cache_block_size, void* workspace,
                                           size_t workspace_bytes, void* stream);

/* ccinfer_decode_attention without a workspace and without any allocation. No counterpart
 * in the reference: for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The split-KV scratch is
 * one static 32 MiB device array per GPU, resolved on the first call on each device and
 * held until the process ends; shapes whose ccinfer_decode_workspace_size exceeds 32 MiB
 * return CCINFER_ERR_INVALID_ARGUMENT (configs of batch 64 x 4096 or 32 x 32768 tokens need
 * under 9 MiB). Calls that overlap on one GPU (concurrent streams) share the array and
 * race; otherwise identical results to ccinfer_decode_attention. */
int ccinfer_decode_attention_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                     const int32_t* block_table, const int32_t* context_lens,
                                     void* output, int batch_size, int max_blocks_per_req,
                                     int num_q_heads, int num_kv_heads, int head_dim,
                                     int cache_block_size, void* stream);

/* fp8 KV cache (no counterpart in the reference, whose cache is bf16 only; its KV profile
 * list, src/base/traits.h:117-124, anticipates other element types). Same [slot][n_kv_heads]
 * [head_dim] layout and block-table contract, one OCP E4M3 byte per element, plus one fp32
 * scale per cache row in k_scale / v_scale, indexed ((slot / 16) * n_kv_heads + kv_head) * 16
 * + slot % 16 (arrays of ceil(max_slots / 16) * 16 * n_kv_heads floats). A row x is stored
 * as e4m3(clamp(x / P, +-448)) with scale P, the smallest power of two >= 2^-126 with
 * max|x| <= 448 P (round to nearest even; an all-zero row stores zeros and scale 0); its
 * value is byte * scale. The attention entries accept any fp32 scale; a power of two takes
 * the faster conversion in the fp8 prefill. Halves decode bytes.
 *
 * Replaces launch_write_kv_cache (src/kernel/cuda_kernels.h:80-83) for an fp8 cache:
 * quantises each new token's K and V rows into its slot; tokens whose slot is outside
 * [0, max_slots) are skipped. head_dim even, <= 512. */
int ccinfer_write_kv_cache_fp8(const void* k_new, const void* v_new, void* k_cache,
                               void* v_cache, float* k_scale, float* v_scale,
                               const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                               int head_dim, int max_slots, void* stream);

/* Replaces launch_decode_attention (src/kernel/cuda_kernels.h:72-77) for an fp8 cache: the
 * same semantics, plan and workspace (ccinfer_decode_workspace_size) as
 * ccinfer_decode_attention, with K/V read as byte * row scale. head_dim 64, 128 or 256
 * (CCINFER_ERR_UNSUPPORTED otherwise). */
int ccinfer_decode_attention_fp8(const void* q, const void* k_cache, const void* v_cache,
                                 const float* k_scale, const float* v_scale,
                                 const int32_t* block_table, const int32_t* context_lens,
                                 void* output, int batch_size, int max_blocks_per_req,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 int cache_block_size, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Workspace bytes ccinfer_prefill_attention (and the fp8 / overlap variants) needs for this
 * batch shape; 0 for invalid shapes. As for decode, it includes two copies of
 * the q rows used only by a call with a 2-byte-aligned q or output. */
size_t ccinfer_prefill_workspace_size(int batch_size, int total_query_tokens,
                                      int max_blocks_per_req, int num_q_heads,
                                      int num_kv_heads, int head_dim, int cache_block_size);

/* Replaces launch_prefill_attention (src/kernel/cuda_kernels.h:61-66,
 * src/kernel/attention/prefill_attn.cu:246-279).
 * q, output: [total_query_tokens][num_q_heads][head_dim] bf16; query_start_loc:
 * [batch_size + 1]; context_lens[r] = prefix_r + query_len_r; query i of request r sees
 * cache positions [0, prefix_r + i]. Mixed batches (single-token decode items next to
 * prompt chunks) are accepted, as in the reference. head_dim <= 256. As in the reference,
 * neither the batch size nor the table length is bounded. The MFMA path covers every
 * query group size and head dims that are multiples of 8 up to 128 (at any size; those
 * below 64 / 128 run padded with zeros) or multiples of 16 up to 256 (up to 4096 blocks per
 * table row, counted in 16-token blocks), with cache blocks of any multiple of 16 tokens
 * (read through a 16-token table the call builds in the workspace). Other block sizes,
 * head dims up to 256 and table lengths run an MFMA tile kernel that stages rows
 * element-wise. A mixed batch's decode items run on `stream` ahead of the prompt tiles. */
int ccinfer_prefill_attention(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_table, const int32_t* query_start_loc,
                              const int32_t* context_lens, void* output, int batch_size,
                              int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                              int num_kv_heads, int head_dim, int cache_block_size,
                              void* workspace, size_t workspace_bytes, void* stream);

/* ccinfer_prefill_attention with the decode items of a mixed batch (of at least 32
 * requests) run on the caller's side_stream (a hipStream_t) concurrently with the prompt
 * tiles on `stream`: the call records fork_event on `stream`, makes side_stream wait for
 * it, and joins back by recording join_event on side_stream and making `stream` wait for it
 * -- event records and waits only, so it can be captured into a graph. fork_event and
 * join_event are caller-owned hipEvent_t (hipEventDisableTiming is enough); side_stream
 * NULL runs as ccinfer_prefill_attention. No counterpart in the reference (one stream);
 * HipBackend owns such a side stream. Concurrent calls must not share the side stream's
 * events. */
int ccinfer_prefill_attention_overlap(const void* q, const void* k_cache, const void* v_cache,
                                      const int32_t* block_table,
                                      const int32_t* query_start_loc,
                                      const int32_t* context_lens, void* output, int batch_size,
                                      int total_query_tokens, int max_blocks_per_req,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      int cache_block_size, void* workspace,
                                      size_t workspace_bytes, void* stream, void* side_stream,
                                      void* fork_event, void* join_event);

/* Replaces launch_prefill_attention (src/kernel/cuda_kernels.h:61-66) for an fp8 cache
 * (layout and scales as for ccinfer_write_kv_cache_fp8): the same semantics, planner and
 * workspace (ccinfer_prefill_workspace_size) as ccinfer_prefill_attention, with K/V read as
 * byte * row scale; single-token requests of a mixed batch go through the fp8 decode.
 * head_dim 64 or 128 and at most 4096 blocks per table row on the MFMA path
 * (CCINFER_ERR_UNSUPPORTED otherwise). */
int ccinfer_prefill_attention_fp8(const void* q, const void* k_cache, const void* v_cache,
                                  const float* k_scale, const float* v_scale,
                                  const int32_t* block_table, const int32_t* query_start_loc,
                                  const int32_t* context_lens, void* output, int batch_size,
                                  int total_query_tokens, int max_blocks_per_req,
                                  int num_q_heads, int num_kv_heads, int head_dim,
                                  int cache_block_size, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* ccinfer_prefill_attention_fp8 with the decode items of a mixed batch on side_stream, as
 * for ccinfer_prefill_attention_overlap. */
int ccinfer_prefill_attention_fp8_overlap(
    const void* q, const void* k_cache, const void* v_cache, const float* k_scale,
    const float* v_scale, const int32_t* block_table, const int32_t* query_start_loc,
    const int32_t* context_lens, void* output, int batch_size, int total_query_tokens,
    int max_blocks_per_req, int num_q_heads, int num_kv_heads, int head_dim,
    int cache_block_size, void* workspace, size_t workspace_bytes, void* stream,
    void* side_stream, void* fork_event, void* join_event);

/* Human-readable text for a status code (the reference's error_message()). */
const char* ccinfer_error_message(int code);

/* Library version, "major.minor.patch". */
const char* ccinfer_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CCINFER_ATTN_H */
