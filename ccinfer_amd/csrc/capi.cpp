// C ABI of the paged-attention hot path: argument validation, shape dispatch and
// error-code mapping. Declarations and contracts: include/ccinfer_attn.h.
//
// Validation mirrors the reference's two layers:
//   - DeviceBackend::{write_kv_cache, decode_attention, prefill_attention}
//     (src/backend/backend.h:172-223): null pointers, non-positive sizes, Hq % Hkv != 0
//     -> InvalidArgument;
//   - the launchers: decode requires cache_block_size == 16 and a supported head_dim
//     (src/kernel/attention/decode_attn.cu:488, :521-569), prefill requires
//     head_dim <= 256 (src/kernel/attention/prefill_attn.cu:257-259).
// Device errors map as in src/backend/cuda/cuda_utils.h:13-36.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstring>
#include <algorithm>
#include <cstdint>

#include "ccinfer_attn.h"
#include "kernels.hpp"

namespace {

using namespace ccinfer::hipk;

int map_hip_error(hipError_t err) {
    switch (err) {
        case hipSuccess:
            return CCINFER_OK;
        case hipErrorOutOfMemory:
            return CCINFER_ERR_DEVICE_OUT_OF_MEMORY;
        case hipErrorInvalidValue:
        case hipErrorInvalidDevice:
        case hipErrorInvalidDevicePointer:
        case hipErrorInvalidConfiguration:
            return CCINFER_ERR_DEVICE_INVALID_VALUE;
        case hipErrorLaunchFailure:
        case hipErrorLaunchOutOfResources:
        case hipErrorIllegalAddress:
            return CCINFER_ERR_LAUNCH_FAILED;
        default:
            return CCINFER_ERR_DEVICE_RUNTIME;
    }
}

bool decode_head_dim_ok(int d) {
    switch (d) {
        case 32: case 64: case 80: case 96: case 112: case 120: case 128: case 192: case 256:
            return true;
        default:
            return false;
    }
}

bool fits_int(int64_t v) { return v >= 0 && v <= INT_MAX; }

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// The native MFMA paths move q, output and cache rows in 16-byte pieces; the reference
// launchers take any bf16 (2-byte aligned) view, so bf16 calls with a less aligned pointer
// take the routes below, and fp8 calls are rejected.
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool fast_aligned(const void* q, const void* k_cache, const void* v_cache, const void* output) {
    return aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(output);
}

// A bf16 call whose caches are 16-byte aligned but whose q or output view is only 2-byte
// aligned still runs the MFMA kernels: q (and, for prefill, the output rows the call may
// leave untouched) are copied into 16-byte-aligned workspace regions, the kernels run on
// those, and the output rows are copied back -- two or three passes over rows that are
// small next to the cache reads. Caches that are not 16-byte aligned run decode with 2-byte
// piece loads and prefill on the any-layout tile kernel. The workspace size queries
// include these regions; a call checks only the bytes it uses.
constexpr size_t kWsAlign = 256;

size_t ws_align(size_t v) { return (v + kWsAlign - 1) / kWsAlign * kWsAlign; }

// Bytes of one workspace copy of `rows` x Hq x D bf16.
size_t row_copy_bytes(int64_t rows, int num_q_heads, int head_dim) {
    return ws_align(static_cast<size_t>(rows) * num_q_heads * head_dim * 2);
}

bool caches_aligned(const void* k_cache, const void* v_cache) {
    return aligned16(k_cache) && aligned16(v_cache);
}

bool decode_shape_ok(int batch_size, int max_blocks_per_req, int num_q_heads, int num_kv_heads,
                     int head_dim, int cache_block_size) {
    if (batch_size <= 0 || max_blocks_per_req <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
        head_dim <= 0 || cache_block_size <= 0)
        return false;
    if (num_q_heads % num_kv_heads != 0) return false;
    if (cache_block_size != 16 || !decode_head_dim_ok(head_dim)) return false;
    return fits_int(static_cast<int64_t>(max_blocks_per_req) * cache_block_size) &&
           fits_int(static_cast<int64_t>(batch_size) * num_q_heads);
}

bool prefill_shape_ok(int batch_size, int total_query_tokens, int max_blocks_per_req,
                      int num_q_heads, int num_kv_heads, int head_dim, int cache_block_size) {
    if (batch_size <= 0 || total_query_tokens <= 0 || max_blocks_per_req <= 0 ||
        num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || cache_block_size <= 0)
        return false;
    if (num_q_heads % num_kv_heads != 0 || head_dim > 256) return false;
    return fits_int(static_cast<int64_t>(max_blocks_per_req) * cache_block_size) &&
           fits_int(static_cast<int64_t>(total_query_tokens) * num_q_heads);
}

bool prefill_uses_fast(int batch_size, int max_blocks_per_req, int num_q_heads,
                       int num_kv_heads, int head_dim, int cache_block_size) {
    (void)batch_size;
    return cache_block_size == 16 &&
           prefill_fast_supported(num_q_heads, num_kv_heads, head_dim, max_blocks_per_req) &&
           decode_fast_supported(num_q_heads, num_kv_heads, head_dim, cache_block_size);
}

// How a bf16 prefill of this shape runs on the MFMA kernels: cache blocks of 16·k tokens are
// read through a table of 16-token blocks (`expand` = k) built in the workspace; the
// workspace holds the kernels' region, then that table, then the q / output row copies.
struct PrefillRoute {
    bool fast = false;
    int expand = 1;
    int mbpr16 = 0;
    size_t table_off = 0;
    size_t rows_off = 0;
    size_t rows_bytes = 0;
    size_t need(bool staged) const { return rows_off + (staged ? 2 * rows_bytes : 0); }
};

PrefillRoute prefill_route(int batch_size, int total_query_tokens, int max_blocks_per_req,
                           int num_q_heads, int num_kv_heads, int head_dim,
                           int cache_block_size) {
    PrefillRoute r;
    if (cache_block_size % 16 != 0) return r;
    r.expand = cache_block_size / 16;
    const int64_t mbpr16 = static_cast<int64_t>(max_blocks_per_req) * r.expand;
    if (!fits_int(mbpr16) || !fits_int(mbpr16 * batch_size)) return r;
    r.mbpr16 = static_cast<int>(mbpr16);
    if (!prefill_uses_fast(batch_size, r.mbpr16, num_q_heads, num_kv_heads, head_dim, 16))
        return r;
    r.fast = true;
    r.table_off = ws_align(prefill_workspace_bytes(batch_size, total_query_tokens, r.mbpr16,
                                                   num_q_heads, num_kv_heads, head_dim, 16));
    r.rows_off = r.table_off +
                 (r.expand > 1 ? ws_align(static_cast<size_t>(mbpr16) * batch_size * 4) : 0);
    r.rows_bytes = row_copy_bytes(total_query_tokens, num_q_heads, head_dim);
    return r;
}

// A side stream needs both events; the events may not be NULL with a side stream.
bool overlap_ok(void* side_stream, void* fork_event, void* join_event) {
    return side_stream == nullptr || (fork_event != nullptr && join_event != nullptr);
}

int prefill_entry(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_table, const int32_t* query_start_loc,
                              const int32_t* context_lens, void* output, int batch_size,
                              int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                              int num_kv_heads, int head_dim, int cache_block_size,
                              void* workspace, size_t workspace_bytes, void* stream,
                              const PrefillOverlap* overlap) {
    if (!q || !k_cache || !v_cache || !block_table || !query_start_loc || !context_lens ||
        !output)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (!prefill_shape_ok(batch_size, total_query_tokens, max_blocks_per_req, num_q_heads,
                          num_kv_heads, head_dim, cache_block_size))
        return CCINFER_ERR_INVALID_ARGUMENT;
    const PrefillRoute rt = prefill_route(batch_size, total_query_tokens, max_blocks_per_req,
                                          num_q_heads, num_kv_heads, head_dim,
                                          cache_block_size);
    if (!rt.fast || !caches_aligned(k_cache, v_cache)) {
        // Other block sizes, head dims, cache alignments, and head dims above 128 past 4096
        // table blocks: the MFMA tile kernel with element-wise staging.
        if (!prefill_any_supported(num_q_heads, num_kv_heads, head_dim, max_blocks_per_req))
            return CCINFER_ERR_INTERNAL;  // the shape check above admits no other shape
        const size_t need_any = prefill_any_workspace_bytes(
            batch_size, total_query_tokens, num_q_heads, num_kv_heads, head_dim);
        if (workspace == nullptr || workspace_bytes < need_any)
            return CCINFER_ERR_INVALID_ARGUMENT;
        return map_hip_error(prefill_attention_any(
            q, k_cache, v_cache, block_table, query_start_loc, context_lens, output,
            batch_size, total_query_tokens, max_blocks_per_req, num_q_heads, num_kv_heads,
            head_dim, cache_block_size, workspace, as_stream(stream)));
    }
    const bool staged = !(aligned16(q) && aligned16(output));
    if (workspace == nullptr || workspace_bytes < rt.need(staged))
        return CCINFER_ERR_INVALID_ARGUMENT;
    char* ws = static_cast<char*>(workspace);
    hipStream_t s = as_stream(stream);
    const int32_t* table = block_table;
    if (rt.expand > 1) {
        int32_t* t16 = reinterpret_cast<int32_t*>(ws + rt.table_off);
        const hipError_t err =
            expand_block_table(block_table, t16, batch_size, max_blocks_per_req, rt.expand, s);
        if (err != hipSuccess) return map_hip_error(err);
        table = t16;
    }
    const void* q_run = q;
    void* out_run = output;
    const int64_t elems = static_cast<int64_t>(total_query_tokens) * num_q_heads * head_dim;
    if (staged) {
        q_run = ws + rt.rows_off;
        out_run = ws + rt.rows_off + rt.rows_bytes;
        // the output copy starts as the caller's rows: rows of no request, or of a request
        // whose context is shorter than its query, are not written and must come back as
        // they were
        hipError_t err = gather_rows(q, ws + rt.rows_off, elems, s);
        if (err == hipSuccess) err = gather_rows(output, out_run, elems, s);
        if (err != hipSuccess) return map_hip_error(err);
    }
    const hipError_t err = prefill_attention(
        q_run, k_cache, v_cache, table, query_start_loc, context_lens, out_run, batch_size,
        total_query_tokens, rt.mbpr16, num_q_heads, num_kv_heads, head_dim, 16, workspace, s,
        overlap);
    if (err != hipSuccess || !staged) return map_hip_error(err);
    return map_hip_error(scatter_rows(out_run, output, elems, s));
}

int prefill_fp8_entry(const void* q, const void* k_cache, const void* v_cache,
                                  const float* k_scale, const float* v_scale,
                                  const int32_t* block_table, const int32_t* query_start_loc,
                                  const int32_t* context_lens, void* output, int batch_size,
                                  int total_query_tokens, int max_blocks_per_req,
                                  int num_q_heads, int num_kv_heads, int head_dim,
                                  int cache_block_size, void* workspace, size_t workspace_bytes,
                                  void* stream, const PrefillOverlap* overlap) {
    if (!q || !k_cache || !v_cache || !k_scale || !v_scale || !block_table ||
        !query_start_loc || !context_lens || !output)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (!prefill_shape_ok(batch_size, total_query_tokens, max_blocks_per_req, num_q_heads,
                          num_kv_heads, head_dim, cache_block_size))
        return CCINFER_ERR_INVALID_ARGUMENT;
    // fp8 has the pipelined MFMA path only (head_dim 64 / 128)
    if (!prefill_uses_fast(batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                           cache_block_size) ||
        !prefill_fp8_supported(head_dim, max_blocks_per_req))
        return CCINFER_ERR_UNSUPPORTED;
    if (!fast_aligned(q, k_cache, v_cache, output) || !aligned16(k_scale) || !aligned16(v_scale))
        return CCINFER_ERR_INVALID_ARGUMENT;
    const size_t need =
        prefill_workspace_bytes(batch_size, total_query_tokens, max_blocks_per_req,
                                num_q_heads, num_kv_heads, head_dim, cache_block_size);
    if (workspace == nullptr || workspace_bytes < need) return CCINFER_ERR_INVALID_ARGUMENT;
    return map_hip_error(prefill_attention_fp8(
        q, k_cache, v_cache, k_scale, v_scale, block_table, query_start_loc, context_lens,
        output, batch_size, total_query_tokens, max_blocks_per_req, num_q_heads, num_kv_heads,
        head_dim, workspace, as_stream(stream), overlap));
}

}  // namespace

namespace ccinfer::hipk {

size_t decode_bytes_for(int batch_size, int max_blocks_per_req, int num_q_heads,
                        int num_kv_heads, int head_dim, int cache_block_size, bool staged) {
    // One size serves ccinfer_decode_attention and ccinfer_decode_attention_fp8, whose flat
    // plans differ in wavefront count.
    size_t bytes = 0;
    for (const bool fp8 : {false, true}) {
        const DecodePlan plan =
            plan_decode(batch_size, num_q_heads, num_kv_heads, head_dim,
                        max_blocks_per_req * cache_block_size, true, fp8);
        bytes = std::max(bytes, decode_workspace_bytes(batch_size, num_q_heads, head_dim, plan));
    }
    if (staged) bytes = ws_align(bytes) + 2 * row_copy_bytes(batch_size, num_q_heads, head_dim);
    return bytes;
}

}  // namespace ccinfer::hipk

extern "C" {

int ccinfer_write_kv_cache(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                           const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                           int head_dim, int max_slots, void* stream) {
    if (!k_new || !v_new || !k_cache || !v_cache || !slot_mapping)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (total_tokens <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_slots <= 0)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (!fits_int(static_cast<int64_t>(n_kv_heads) * head_dim * 2))
        return CCINFER_ERR_INVALID_ARGUMENT;
    return map_hip_error(write_kv_cache(k_new, v_new, k_cache, v_cache, slot_mapping,
                                        total_tokens, n_kv_heads, head_dim, max_slots,
                                        as_stream(stream)));
}

int ccinfer_qkv_prologue(const void* qkv, const void* q_norm_weight, const void* k_norm_weight,
                         const int32_t* positions, const void* rope_cache,
                         const int32_t* slot_mapping, void* q_out, void* k_cache, void* v_cache,
                         int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                         int rope_cache_max_position, int max_slots, float eps, void* stream) {
    if (!qkv || !positions || !rope_cache || !slot_mapping || !q_out || !k_cache || !v_cache)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (num_tokens <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_slots <= 0 ||
        rope_cache_max_position <= 0)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 1024) return CCINFER_ERR_INVALID_ARGUMENT;
    // eps > 0 (backend.h:84); NaN and inf are tested on the bits, which stays correct when
    // the compiler is told that NaNs do not occur.
    uint32_t eps_bits;
    std::memcpy(&eps_bits, &eps, sizeof eps_bits);
    if ((eps_bits & 0x7f800000u) == 0x7f800000u || !(eps > 0.0f))
        return CCINFER_ERR_INVALID_ARGUMENT;
    const int64_t rows = static_cast<int64_t>(num_tokens) * (num_q_heads + num_kv_heads);
    if (!fits_int(rows) ||
        !fits_int(static_cast<int64_t>(num_q_heads + 2 * static_cast<int64_t>(num_kv_heads)) *
                  head_dim))
        return CCINFER_ERR_INVALID_ARGUMENT;
    return map_hip_error(qkv_prologue(qkv, q_norm_weight, k_norm_weight, positions, rope_cache,
                                      slot_mapping, q_out, k_cache, v_cache, num_tokens,
                                      num_q_heads, num_kv_heads, head_dim,
                                      rope_cache_max_position, max_slots, eps,
                                      as_stream(stream)));
}

int ccinfer_build_batch_metadata(const int32_t* item_kv_written, const int32_t* item_new_tokens,
                                 const int32_t* item_flags, const int32_t* item_block_start,
                                 const int32_t* blocks, int batch_size, int num_tokens,
                                 int total_blocks, int max_blocks_per_req, int block_size,
                                 int num_cache_blocks, int32_t* positions, int32_t* slot_mapping,
                                 int32_t* block_table, int32_t* query_start_loc,
                                 int32_t* context_lens, int32_t* logits_indices, int32_t* status,
                                 void* stream) {
    if (!item_kv_written || !item_new_tokens || !item_flags || !item_block_start || !positions ||
        !slot_mapping || !block_table || !query_start_loc || !context_lens || !logits_indices ||
        !status)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (total_blocks > 0 && !blocks) return CCINFER_ERR_INVALID_ARGUMENT;
    if (batch_size <= 0 || num_tokens <= 0 || total_blocks < 0 || max_blocks_per_req <= 0 ||
        block_size <= 0 || num_cache_blocks <= 0)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (!fits_int(static_cast<int64_t>(batch_size) * max_blocks_per_req) ||
        !fits_int(static_cast<int64_t>(num_cache_blocks) * block_size))
        return CCINFER_ERR_INVALID_ARGUMENT;
    return map_hip_error(build_batch_metadata(
        item_kv_written, item_new_tokens, item_flags, item_block_start, blocks, batch_size,
        num_tokens, total_blocks, max_blocks_per_req, block_size, num_cache_blocks, positions,
        slot_mapping, block_table, query_start_loc, context_lens, logits_indices, status,
        as_stream(stream)));
}

size_t ccinfer_decode_workspace_size(int batch_size, int max_blocks_per_req, int num_q_heads,
                                     int num_kv_heads, int head_dim, int cache_block_size) {
    if (!decode_shape_ok(batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                         cache_block_size))
        return 0;
    if (!decode_fast_supported(num_q_heads, num_kv_heads, head_dim, cache_block_size)) return 0;
    return decode_bytes_for(batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                            cache_block_size, true);
}

namespace {

// Decode, optionally writing each request's new token first (new_k != nullptr).
int decode_entry(const void* q, const void* k_cache, const void* v_cache,
                 const int32_t* block_table, const int32_t* context_lens, void* output,
                 int batch_size, int max_blocks_per_req, int num_q_heads, int num_kv_heads,
                 int head_dim, int cache_block_size, void* workspace, size_t workspace_bytes,
                 void* stream, const void* new_k, const void* new_v, int max_slots) {
    if (!q || !k_cache || !v_cache || !block_table || !context_lens || !output)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (!decode_shape_ok(batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                         cache_block_size))
        return CCINFER_ERR_INVALID_ARGUMENT;
    // Every decode shape the validation admits runs the MFMA kernels (caches that are only
    // 2-byte aligned with 2-byte piece loads).
    if (!decode_fast_supported(num_q_heads, num_kv_heads, head_dim, cache_block_size))
        return CCINFER_ERR_INTERNAL;
    const bool staged = !(aligned16(q) && aligned16(output));
    const DecodePlan plan = plan_decode(batch_size, num_q_heads, num_kv_heads, head_dim,
                                        max_blocks_per_req * cache_block_size, true);
    // the size the query returns without the row copies, which only a call with unaligned
    // q / output uses (it covers the fp8 entry's plan too)
    const size_t need = decode_bytes_for(batch_size, max_blocks_per_req, num_q_heads,
                                         num_kv_heads, head_dim, cache_block_size, staged);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return CCINFER_ERR_INVALID_ARGUMENT;
    // The new tokens go in with the decode launch when its kernels can write them (4-byte
    // aligned new rows, 16-byte aligned cache rows), else by a separate launch before it.
    const bool fused = new_k != nullptr && caches_aligned(k_cache, v_cache) &&
                       ((reinterpret_cast<uintptr_t>(new_k) | reinterpret_cast<uintptr_t>(new_v)) &
                        3u) == 0;
    if (new_k != nullptr && !fused) {
        const hipError_t err = write_last_tokens(
            new_k, new_v, const_cast<void*>(k_cache), const_cast<void*>(v_cache), block_table,
            context_lens, batch_size, max_blocks_per_req, num_kv_heads, head_dim, max_slots,
            as_stream(stream));
        if (err != hipSuccess) return map_hip_error(err);
    }
    DecodeItems items;
    items.num_items = batch_size;
    if (fused) {
        items.new_k = new_k;
        items.new_v = new_v;
        items.max_slots = max_slots;
    }
    const void* q_run = q;
    void* out_run = output;
    const int64_t elems = static_cast<int64_t>(batch_size) * num_q_heads * head_dim;
    if (staged) {
        char* rows = static_cast<char*>(workspace) +
                     ws_align(decode_bytes_for(batch_size, max_blocks_per_req, num_q_heads,
                                               num_kv_heads, head_dim, cache_block_size, false));
        q_run = rows;
        out_run = rows + row_copy_bytes(batch_size, num_q_heads, head_dim);
        const hipError_t err = gather_rows(q, rows, elems, as_stream(stream));
        if (err != hipSuccess) return map_hip_error(err);
    }
    const hipError_t err = decode_attention(q_run, k_cache, v_cache, block_table, context_lens,
                                            out_run, items, max_blocks_per_req, num_q_heads,
                                            num_kv_heads, head_dim, cache_block_size, plan,
                                            workspace, as_stream(stream));
    if (err != hipSuccess || !staged) return map_hip_error(err);
    // every output row is written (zeros for rows with no context)
    return map_hip_error(scatter_rows(out_run, output, elems, as_stream(stream)));
}

}  // namespace

int ccinfer_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                             const int32_t* block_table, const int32_t* context_lens,
                             void* output, int batch_size, int max_blocks_per_req,
                             int num_q_heads, int num_kv_heads, int head_dim,
                             int cache_block_size, void* workspace, size_t workspace_bytes,
                             void* stream) {
    return decode_entry(q, k_cache, v_cache, block_table, context_lens, output, batch_size,
                        max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                        cache_block_size, workspace, workspace_bytes, stream, nullptr, nullptr,
                        0);
}

size_t ccinfer_decode_shared_workspace_size(int batch_size, int max_blocks_per_req,
                                            int num_q_heads, int num_kv_heads, int head_dim,
                                            int cache_block_size) {
    const size_t plain = ccinfer_decode_workspace_size(batch_size, max_blocks_per_req,
                                                       num_q_heads, num_kv_heads, head_dim,
                                                       cache_block_size);
    if (!decode_shape_ok(batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                         cache_block_size) ||
        !decode_shared_supported(batch_size, num_q_heads, num_kv_heads, head_dim,
                                 cache_block_size))
        return plain;
    return std::max(plain, decode_shared_workspace_bytes(batch_size, max_blocks_per_req,
                                                         num_q_heads, num_kv_heads, head_dim));
}

int ccinfer_decode_attention_shared_prefix(const void* q, const void* k_cache,
                                           const void* v_cache, const int32_t* block_table,
                                           const int32_t* context_lens, void* output,
                                           int batch_size, int max_blocks_per_req,
                                           int num_q_heads, int num_kv_heads, int head_dim,
                                           int cache_block_size, void* workspace,
                                           size_t workspace_bytes, void* stream) {
    if (!q || !k_cache || !v_cache || !block_table || !context_lens || !output)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (!decode_shape_ok(batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                         cache_block_size))
        return CCINFER_ERR_INVALID_ARGUMENT;
    const bool shared = decode_shared_supported(batch_size, num_q_heads, num_kv_heads,
                                                head_dim, cache_block_size) &&
                        fast_aligned(q, k_cache, v_cache, output);
    if (!shared)
        return decode_entry(q, k_cache, v_cache, block_table, context_lens, output, batch_size,
                            max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                            cache_block_size, workspace, workspace_bytes, stream, nullptr,
                            nullptr, 0);
    const size_t need = ccinfer_decode_shared_workspace_size(
        batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim, cache_block_size);
    if (workspace == nullptr || workspace_bytes < need) return CCINFER_ERR_INVALID_ARGUMENT;
    return map_hip_error(decode_attention_shared(q, k_cache, v_cache, block_table, context_lens,
                                                 output, batch_size, max_blocks_per_req,
                                                 num_q_heads, num_kv_heads, head_dim, workspace,
                                                 as_stream(stream)));
}

int ccinfer_decode_attention_write_kv(const void* q, const void* k_new, const void* v_new,
                                      void* k_cache, void* v_cache, const int32_t* block_table,
                                      const int32_t* context_lens, void* output, int batch_size,
                                      int max_blocks_per_req, int num_q_heads, int num_kv_heads,
                                      int head_dim, int cache_block_size, int max_slots,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    if (!k_new || !v_new || max_slots <= 0) return CCINFER_ERR_INVALID_ARGUMENT;
    return decode_entry(q, k_cache, v_cache, block_table, context_lens, output, batch_size,
                        max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                        cache_block_size, workspace, workspace_bytes, stream, k_new, v_new,
                        max_slots);
}

int ccinfer_write_kv_cache_fp8(const void* k_new, const void* v_new, void* k_cache,
                               void* v_cache, float* k_scale, float* v_scale,
                               const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                               int head_dim, int max_slots, void* stream) {
    if (!k_new || !v_new || !k_cache || !v_cache || !k_scale || !v_scale || !slot_mapping)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (total_tokens <= 0 || n_kv_heads <= 0 || max_slots <= 0) return CCINFER_ERR_INVALID_ARGUMENT;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 512) return CCINFER_ERR_INVALID_ARGUMENT;
    if (!fits_int(static_cast<int64_t>(total_tokens) * n_kv_heads * 2))
        return CCINFER_ERR_INVALID_ARGUMENT;
    return map_hip_error(write_kv_cache_fp8(k_new, v_new, k_cache, v_cache, k_scale, v_scale,
                                            slot_mapping, total_tokens, n_kv_heads, head_dim,
                                            max_slots, as_stream(stream)));
}

int ccinfer_decode_attention_fp8(const void* q, const void* k_cache, const void* v_cache,
                                 const float* k_scale, const float* v_scale,
                                 const int32_t* block_table, const int32_t* context_lens,
                                 void* output, int batch_size, int max_blocks_per_req,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 int cache_block_size, void* workspace, size_t workspace_bytes,
                                 void* stream) {
    if (!q || !k_cache || !v_cache || !k_scale || !v_scale || !block_table || !context_lens ||
        !output)
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (!decode_shape_ok(batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                         cache_block_size))
        return CCINFER_ERR_INVALID_ARGUMENT;
    if (!decode_fp8_supported(num_q_heads, num_kv_heads, head_dim, cache_block_size))
        return CCINFER_ERR_UNSUPPORTED;  // fp8 has the MFMA path only
    if (!fast_aligned(q, k_cache, v_cache, output) || !aligned16(k_scale) || !aligned16(v_scale))
        return CCINFER_ERR_INVALID_ARGUMENT;
    const DecodePlan plan =
        plan_decode(batch_size, num_q_heads, num_kv_heads, head_dim,
                    max_blocks_per_req * cache_block_size, true, true);
    const size_t need = ccinfer_decode_workspace_size(batch_size, max_blocks_per_req,
                                                      num_q_heads, num_kv_heads, head_dim,
                                                      cache_block_size);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return CCINFER_ERR_INVALID_ARGUMENT;
    DecodeItems items;
    items.num_items = batch_size;
    return map_hip_error(decode_attention_fp8(q, k_cache, v_cache, k_scale, v_scale, block_table,
                                              context_lens, output, items, max_blocks_per_req,
                                              num_q_heads, num_kv_heads, head_dim, plan,
                                              workspace, as_stream(stream)));
}

size_t ccinfer_prefill_workspace_size(int batch_size, int total_query_tokens,
                                      int max_blocks_per_req, int num_q_heads,
                                      int num_kv_heads, int head_dim, int cache_block_size) {
    if (!prefill_shape_ok(batch_size, total_query_tokens, max_blocks_per_req, num_q_heads,
                          num_kv_heads, head_dim, cache_block_size))
        return 0;
    const PrefillRoute rt = prefill_route(batch_size, total_query_tokens, max_blocks_per_req,
                                          num_q_heads, num_kv_heads, head_dim,
                                          cache_block_size);
    // the MFMA-kernel route (it covers the fp8 entry too: 16-token blocks, aligned views)
    // and the any-layout route, which a call takes for caches that are not 16-byte aligned
    // or shapes the first does not take
    const size_t fast = rt.fast ? rt.need(true) : 0;
    const size_t any = prefill_any_supported(num_q_heads, num_kv_heads, head_dim,
                                             max_blocks_per_req)
                           ? prefill_any_workspace_bytes(batch_size, total_query_tokens,
                                                         num_q_heads, num_kv_heads, head_dim)
                           : 0;
    return std::max(fast, any);
}

int ccinfer_prefill_attention(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_table, const int32_t* query_start_loc,
                              const int32_t* context_lens, void* output, int batch_size,
                              int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                              int num_kv_heads, int head_dim, int cache_block_size,
                              void* workspace, size_t workspace_bytes, void* stream) {
    return prefill_entry(q, k_cache, v_cache, block_table, query_start_loc, context_lens, output,
                         batch_size, total_query_tokens, max_blocks_per_req, num_q_heads,
                         num_kv_heads, head_dim, cache_block_size, workspace, workspace_bytes,
                         stream, nullptr);
}

int ccinfer_prefill_attention_overlap(const void* q, const void* k_cache, const void* v_cache,
                                      const int32_t* block_table,
                                      const int32_t* query_start_loc,
                                      const int32_t* context_lens, void* output, int batch_size,
                                      int total_query_tokens, int max_blocks_per_req,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      int cache_block_size, void* workspace,
                                      size_t workspace_bytes, void* stream, void* side_stream,
                                      void* fork_event, void* join_event) {
    if (!overlap_ok(side_stream, fork_event, join_event)) return CCINFER_ERR_INVALID_ARGUMENT;
    const PrefillOverlap ov{as_stream(side_stream), static_cast<hipEvent_t>(fork_event),
                            static_cast<hipEvent_t>(join_event)};
    return prefill_entry(q, k_cache, v_cache, block_table, query_start_loc, context_lens, output,
                         batch_size, total_query_tokens, max_blocks_per_req, num_q_heads,
                         num_kv_heads, head_dim, cache_block_size, workspace, workspace_bytes,
                         stream, &ov);
}

int ccinfer_prefill_attention_fp8(const void* q, const void* k_cache, const void* v_cache,
                                  const float* k_scale, const float* v_scale,
                                  const int32_t* block_table, const int32_t* query_start_loc,
                                  const int32_t* context_lens, void* output, int batch_size,
                                  int total_query_tokens, int max_blocks_per_req,
                                  int num_q_heads, int num_kv_heads, int head_dim,
                                  int cache_block_size, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    return prefill_fp8_entry(q, k_cache, v_cache, k_scale, v_scale, block_table, query_start_loc,
                             context_lens, output, batch_size, total_query_tokens,
                             max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                             cache_block_size, workspace, workspace_bytes, stream, nullptr);
}

int ccinfer_prefill_attention_fp8_overlap(
    const void* q, const void* k_cache, const void* v_cache, const float* k_scale,
    const float* v_scale, const int32_t* block_table, const int32_t* query_start_loc,
    const int32_t* context_lens, void* output, int batch_size, int total_query_tokens,
    int max_blocks_per_req, int num_q_heads, int num_kv_heads, int head_dim,
    int cache_block_size, void* workspace, size_t workspace_bytes, void* stream,
    void* side_stream, void* fork_event, void* join_event) {
    if (!overlap_ok(side_stream, fork_event, join_event)) return CCINFER_ERR_INVALID_ARGUMENT;
    const PrefillOverlap ov{as_stream(side_stream), static_cast<hipEvent_t>(fork_event),
                            static_cast<hipEvent_t>(join_event)};
    return prefill_fp8_entry(q, k_cache, v_cache, k_scale, v_scale, block_table, query_start_loc,
                             context_lens, output, batch_size, total_query_tokens,
                             max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                             cache_block_size, workspace, workspace_bytes, stream, &ov);
}

const char* ccinfer_error_message(int code) {
    switch (code) {
        case CCINFER_OK: return "ok";
        case CCINFER_ERR_DEVICE_OUT_OF_MEMORY: return "device out of memory";
        case CCINFER_ERR_LAUNCH_FAILED: return "kernel launch failed";
        case CCINFER_ERR_DEVICE_INVALID_VALUE: return "device invalid value";
        case CCINFER_ERR_DEVICE_RUNTIME: return "device runtime error";
        case CCINFER_ERR_INVALID_ARGUMENT: return "invalid argument";
        case CCINFER_ERR_UNSUPPORTED: return "unsupported operation";
        case CCINFER_ERR_INTERNAL: return "internal error";
        default: return "unknown error";
    }
}

const char* ccinfer_version(void) { return "0.1.0"; }

}  // extern "C"
