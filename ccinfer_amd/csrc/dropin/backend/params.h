// Parameter structs of the three hot-path backend ops. Field names, types and meaning are
// the reference's interface (src/backend/params.h:148-211) so designated-initializer call
// sites compile unchanged.
#pragma once

#include <cstdint>

namespace ccinfer {

// Causal paged prefill. q/output: [num_tokens][num_q_heads][head_dim]; K/V read only from
// the cache (written beforehand by write_kv_cache). query_start_loc: [batch + 1];
// context_lens[i] = prefix_len_i + query_len_i; query j of request i sees [0, prefix_i + j];
// block_table: [batch][max_blocks_per_req], -1 for unused entries.
struct PrefillAttnParams {
    const void* q_ = nullptr;
    const void* k_cache_ = nullptr;
    const void* v_cache_ = nullptr;
    const int32_t* block_table_ = nullptr;
    const int32_t* query_start_loc_ = nullptr;
    const int32_t* context_lens_ = nullptr;
    void* output_ = nullptr;
    int num_tokens_ = 0;
    int batch_size_ = 0;
    int max_blocks_per_req_ = 0;
    int num_q_heads_ = 0;
    int num_kv_heads_ = 0;
    int head_dim_ = 0;
    int cache_block_size_ = 0;
};

// Paged decode, one query token per request. context_lens_ includes the current token.
struct DecodeAttnParams {
    const void* q_ = nullptr;
    const void* k_cache_ = nullptr;
    const void* v_cache_ = nullptr;
    const int32_t* block_table_ = nullptr;
    const int32_t* context_lens_ = nullptr;
    void* output_ = nullptr;
    int batch_size_ = 0;
    int max_blocks_per_req_ = 0;
    int num_q_heads_ = 0;
    int num_kv_heads_ = 0;
    int head_dim_ = 0;
    int cache_block_size_ = 0;
};

// Scatter new K/V rows: k_new/v_new [total_tokens][num_kv_heads][head_dim] into
// cache[slot_mapping[t]].
struct WriteKVCacheParams {
    const void* k_new_ = nullptr;
    const void* v_new_ = nullptr;
    void* k_cache_ = nullptr;
    void* v_cache_ = nullptr;
    const int32_t* slot_mapping_ = nullptr;
    int total_tokens_ = 0;
    int num_kv_heads_ = 0;
    int head_dim_ = 0;
    int max_slots_ = 0;
};

}  // namespace ccinfer
