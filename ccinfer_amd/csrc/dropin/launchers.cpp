// The reference-signature launchers (kernel/hip_kernels.h) on top of the C ABI.
//
// The reference launchers take no workspace argument, so the split-KV partials / prefill
// work list come from a buffer kept per (device, stream), reserved explicitly by
// reserve_launcher_workspace. A launch only looks its buffer up (under the map's mutex) and
// checks the size: no allocation, free or synchronisation happens inside a launch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "ccinfer_attn.h"
#include "kernel/hip_kernels.h"

namespace ccinfer {
namespace {

struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};

std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

Result<void> hip_result(hipError_t e) {
    switch (e) {
        case hipSuccess: return {};
        case hipErrorOutOfMemory: return unexpected(ErrorCode::CudaOutOfMemory);
        case hipErrorInvalidValue: return unexpected(ErrorCode::CudaInvalidValue);
        default: return unexpected(ErrorCode::CudaRuntimeError);
    }
}

Result<void> status_result(int s) {
    if (s != CCINFER_OK) return unexpected(static_cast<ErrorCode>(s));
    return {};
}

// The reserved buffer of (current device, stream) if it holds at least `bytes`.
Result<void> lookup(hipStream_t stream, size_t bytes, void** out) {
    *out = nullptr;
    if (bytes == 0) return {};
    int dev = 0;
    if (auto r = hip_result(hipGetDevice(&dev)); !r) return r;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    const auto it = g_ws.find({dev, stream});
    if (it == g_ws.end() || it->second.bytes < bytes) return unexpected(ErrorCode::InvalidArgument);
    *out = it->second.ptr;
    return {};
}

}  // namespace

size_t attn_workspace_bytes(const AttnWorkspaceLimits& lim) {
    if (lim.max_batch_size <= 0 || lim.max_blocks_per_req <= 0 || lim.num_q_heads <= 0 ||
        lim.num_kv_heads <= 0 || lim.head_dim <= 0 || lim.cache_block_size <= 0 ||
        lim.num_q_heads % lim.num_kv_heads != 0)
        return 0;
    // The plans change form with the batch size (a group plan for tiny batches, splits sized
    // per batch below the flat plan's minimum, the flat plan above it), so the size is taken
    // over every batch up to 8 and at the limit; beyond 8 requests it grows with the batch,
    // the query tokens and the table row.
    size_t best = 0;
    auto consider = [&](int b) {
        const int tokens = lim.max_query_tokens > b ? lim.max_query_tokens : b;
        const size_t d = ccinfer_decode_workspace_size(b, lim.max_blocks_per_req, lim.num_q_heads,
                                                       lim.num_kv_heads, lim.head_dim,
                                                       lim.cache_block_size);
        const size_t p = ccinfer_prefill_workspace_size(b, tokens, lim.max_blocks_per_req,
                                                        lim.num_q_heads, lim.num_kv_heads,
                                                        lim.head_dim, lim.cache_block_size);
        best = std::max(best, std::max(d, p));
    };
    for (int b = 1; b <= std::min(8, lim.max_batch_size); ++b) consider(b);
    consider(lim.max_batch_size);
    return best;
}

Result<void> reserve_launcher_workspace(hipStream_t stream, const AttnWorkspaceLimits& lim) {
    const size_t bytes = attn_workspace_bytes(lim);
    if (bytes == 0) return unexpected(ErrorCode::InvalidArgument);
    int dev = 0;
    if (auto r = hip_result(hipGetDevice(&dev)); !r) return r;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Workspace& w = g_ws[{dev, stream}];
    if (w.bytes >= bytes) return {};
    if (w.ptr != nullptr) {
        // queued kernels on the stream may still read the old buffer
        if (auto r = hip_result(hipStreamSynchronize(stream)); !r) return r;
        (void)hipFree(w.ptr);
        w = Workspace{};
    }
    if (auto r = hip_result(hipMalloc(&w.ptr, bytes)); !r) return r;
    w.bytes = bytes;
    return {};
}

Result<void> launch_prefill_attention(const __hip_bfloat16* q, const __hip_bfloat16* k_cache,
                                      const __hip_bfloat16* v_cache, const int32_t* block_table,
                                      const int32_t* query_start_loc, const int32_t* context_lens,
                                      __hip_bfloat16* output, int batch_size,
                                      int total_query_tokens, int max_blocks_per_req,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      int cache_block_size, hipStream_t stream) {
    if (!q || !k_cache || !v_cache || !block_table || !query_start_loc || !context_lens ||
        !output)
        return unexpected(ErrorCode::InvalidArgument);
    const size_t need = ccinfer_prefill_workspace_size(batch_size, total_query_tokens,
                                                       max_blocks_per_req, num_q_heads,
                                                       num_kv_heads, head_dim, cache_block_size);
    void* ws = nullptr;
    if (auto r = lookup(stream, need, &ws); !r) return r;
    return status_result(ccinfer_prefill_attention(
        q, k_cache, v_cache, block_table, query_start_loc, context_lens, output, batch_size,
        total_query_tokens, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
        cache_block_size, ws, need, stream));
}

Result<void> launch_decode_attention(const __hip_bfloat16* q, const __hip_bfloat16* k_cache,
                                     const __hip_bfloat16* v_cache, const int32_t* block_table,
                                     const int32_t* context_lens, __hip_bfloat16* output,
                                     int batch_size, int max_blocks_per_req, int num_q_heads,
                                     int num_kv_heads, int head_dim, int cache_block_size,
                                     hipStream_t stream) {
    if (!q || !k_cache || !v_cache || !block_table || !context_lens || !output)
        return unexpected(ErrorCode::InvalidArgument);
    const size_t need = ccinfer_decode_workspace_size(batch_size, max_blocks_per_req,
                                                      num_q_heads, num_kv_heads, head_dim,
                                                      cache_block_size);
    void* ws = nullptr;
    if (auto r = lookup(stream, need, &ws); !r) return r;
    return status_result(ccinfer_decode_attention(
        q, k_cache, v_cache, block_table, context_lens, output, batch_size, max_blocks_per_req,
        num_q_heads, num_kv_heads, head_dim, cache_block_size, ws, need, stream));
}

Result<void> launch_write_kv_cache(const __hip_bfloat16* k_new, const __hip_bfloat16* v_new,
                                   __hip_bfloat16* k_cache, __hip_bfloat16* v_cache,
                                   const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                                   int head_dim, int max_slots, hipStream_t stream) {
    return status_result(ccinfer_write_kv_cache(k_new, v_new, k_cache, v_cache, slot_mapping,
                                                total_tokens, n_kv_heads, head_dim, max_slots,
                                                stream));
}

void release_launcher_workspaces() {
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if (!g_ws.empty()) (void)hipDeviceSynchronize();
    for (auto& [key, w] : g_ws) {
        (void)key;
        if (w.ptr != nullptr) (void)hipFree(w.ptr);
    }
    g_ws.clear();
}

}  // namespace ccinfer
