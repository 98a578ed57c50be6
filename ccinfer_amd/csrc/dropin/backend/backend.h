// CRTP backend op layer for the hot path (the reference's DeviceBackend,
// src/backend/backend.h:172-223). The public methods validate their parameters exactly as
// the reference does -- null pointers, non-positive sizes and Hq % Hkv != 0 give
// ErrorCode::InvalidArgument -- and then call Derived::xxx_impl<DType>.
#pragma once

#include "backend/params.h"
#include "base/result.h"

namespace ccinfer {

template <typename Derived>
class DeviceBackend {
public:
    template <typename DType>
    Result<void> prefill_attention(const PrefillAttnParams& p) {
        if (p.q_ == nullptr || p.k_cache_ == nullptr || p.v_cache_ == nullptr ||
            p.block_table_ == nullptr || p.query_start_loc_ == nullptr ||
            p.context_lens_ == nullptr || p.output_ == nullptr) {
            return unexpected(ErrorCode::InvalidArgument);
        }
        if (p.batch_size_ <= 0 || p.num_tokens_ <= 0 || p.max_blocks_per_req_ <= 0 ||
            p.num_q_heads_ <= 0 || p.num_kv_heads_ <= 0 || p.head_dim_ <= 0 ||
            p.cache_block_size_ <= 0) {
            return unexpected(ErrorCode::InvalidArgument);
        }
        if (p.num_q_heads_ % p.num_kv_heads_ != 0) return unexpected(ErrorCode::InvalidArgument);
        return self().template prefill_attention_impl<DType>(p);
    }

    template <typename DType>
    Result<void> decode_attention(const DecodeAttnParams& p) {
        if (p.q_ == nullptr || p.k_cache_ == nullptr || p.v_cache_ == nullptr ||
            p.block_table_ == nullptr || p.context_lens_ == nullptr || p.output_ == nullptr) {
            return unexpected(ErrorCode::InvalidArgument);
        }
        if (p.batch_size_ <= 0 || p.max_blocks_per_req_ <= 0 || p.num_q_heads_ <= 0 ||
            p.num_kv_heads_ <= 0 || p.head_dim_ <= 0 || p.cache_block_size_ <= 0) {
            return unexpected(ErrorCode::InvalidArgument);
        }
        if (p.num_q_heads_ % p.num_kv_heads_ != 0) return unexpected(ErrorCode::InvalidArgument);
        return self().template decode_attention_impl<DType>(p);
    }

    template <typename DType>
    Result<void> write_kv_cache(const WriteKVCacheParams& p) {
        if (p.k_new_ == nullptr || p.v_new_ == nullptr || p.k_cache_ == nullptr ||
            p.v_cache_ == nullptr || p.slot_mapping_ == nullptr) {
            return unexpected(ErrorCode::InvalidArgument);
        }
        if (p.total_tokens_ <= 0 || p.num_kv_heads_ <= 0 || p.head_dim_ <= 0 ||
            p.max_slots_ <= 0) {
            return unexpected(ErrorCode::InvalidArgument);
        }
        return self().template write_kv_cache_impl<DType>(p);
    }

private:
    Derived& self() { return static_cast<Derived&>(*this); }
};

}  // namespace ccinfer
