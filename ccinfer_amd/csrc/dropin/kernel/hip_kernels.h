// The reference's hot-path kernel launchers (src/kernel/cuda_kernels.h:61-84) with their
// signatures unchanged except for the platform types: __hip_bfloat16 for __nv_bfloat16 and
// hipStream_t for cudaStream_t. Callers (Qwen3Model::forward, the kernel tests) switch the
// include and keep every argument.
//
// These wrappers call the C ABI (include/ccinfer_attn.h). The reference launchers take no
// workspace, so the split-KV partials and the prefill work list come from a buffer the
// library keeps per (device, stream), reserved once by reserve_launcher_workspace for the
// largest shapes the caller will launch (the reference sizes its KV cache the same way, at
// Worker::init_resources, src/worker/worker.cpp:223-294). The launchers themselves never
// allocate, free or synchronise: a launch on a stream with no reservation, or whose shape
// needs more than the reservation, returns ErrorCode::InvalidArgument. They are therefore
// safe under stream capture.
//
// Thread safety: the (device, stream) -> buffer map is guarded by a mutex; reserve and
// release modify it, launches only read it. Launches on different streams use different
// buffers and may run concurrently; launches on one stream are ordered by the stream.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "base/result.h"

namespace ccinfer {

// The largest shapes a caller will launch; a reservation covers every shape within them.
struct AttnWorkspaceLimits {
    int max_batch_size = 0;          // requests per launch
    int max_query_tokens = 0;        // prefill: query tokens per launch
    int max_blocks_per_req = 0;      // block-table row length
    int num_q_heads = 0;
    int num_kv_heads = 0;
    int head_dim = 0;
    int cache_block_size = 16;
};

// Bytes of device workspace that cover every decode and prefill launch within `lim` (0 when
// the limits are invalid).
size_t attn_workspace_bytes(const AttnWorkspaceLimits& lim);

// Reserves the workspace of (current device, stream) for launches within `lim`: allocates
// (after synchronising the stream, when a smaller buffer must be replaced) and keeps it until
// release_launcher_workspaces. Call at initialisation, outside stream capture.
Result<void> reserve_launcher_workspace(hipStream_t stream, const AttnWorkspaceLimits& lim);

Result<void> launch_prefill_attention(const __hip_bfloat16* q, const __hip_bfloat16* k_cache,
                                      const __hip_bfloat16* v_cache, const int32_t* block_table,
                                      const int32_t* query_start_loc, const int32_t* context_lens,
                                      __hip_bfloat16* output, int batch_size,
                                      int total_query_tokens, int max_blocks_per_req,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      int cache_block_size, hipStream_t stream);

Result<void> launch_decode_attention(const __hip_bfloat16* q, const __hip_bfloat16* k_cache,
                                     const __hip_bfloat16* v_cache, const int32_t* block_table,
                                     const int32_t* context_lens, __hip_bfloat16* output,
                                     int batch_size, int max_blocks_per_req, int num_q_heads,
                                     int num_kv_heads, int head_dim, int cache_block_size,
                                     hipStream_t stream);

Result<void> launch_write_kv_cache(const __hip_bfloat16* k_new, const __hip_bfloat16* v_new,
                                   __hip_bfloat16* k_cache, __hip_bfloat16* v_cache,
                                   const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                                   int head_dim, int max_slots, hipStream_t stream);

// Releases the per-stream workspaces the wrappers above keep (call before destroying a
// stream the wrappers were used on, or at shutdown). Synchronises the device.
void release_launcher_workspaces();

}  // namespace ccinfer
