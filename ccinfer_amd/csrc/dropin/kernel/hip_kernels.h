// The reference's hot-path kernel launchers (src/kernel/cuda_kernels.h:61-84) with their
// signatures unchanged except for the platform types: __hip_bfloat16 for __nv_bfloat16 and
// hipStream_t for cudaStream_t. Callers (Qwen3Model::forward, the kernel tests) switch the
// include and keep every argument.
//
// These wrappers call the C ABI (include/ccinfer_attn.h). The reference launchers take no
// workspace, so the split-KV partials and the prefill work list come from a buffer the
// library keeps per (device, stream); it is allocated on first use and grown when a larger
// batch shape arrives, never per call at steady state.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "base/result.h"

namespace ccinfer {

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
