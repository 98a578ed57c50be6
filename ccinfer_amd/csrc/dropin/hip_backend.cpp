// HipBackend implementation: forwards the three hot-path ops to the C ABI on the backend's
// own stream with its reserved workspace.
#include "backend/hip_backend.h"

#include "ccinfer_attn.h"

namespace ccinfer {

namespace {

ErrorCode from_status(int s) { return static_cast<ErrorCode>(s); }

Result<void> check(int s) {
    if (s != CCINFER_OK) return unexpected(from_status(s));
    return {};
}

Result<void> check_hip(hipError_t e) {
    switch (e) {
        case hipSuccess: return {};
        case hipErrorOutOfMemory: return unexpected(ErrorCode::CudaOutOfMemory);
        case hipErrorInvalidValue:
        case hipErrorInvalidDevice: return unexpected(ErrorCode::CudaInvalidValue);
        default: return unexpected(ErrorCode::CudaRuntimeError);
    }
}

}  // namespace

Result<std::unique_ptr<HipBackend>> HipBackend::create(int device_id) {
    std::unique_ptr<HipBackend> b(new HipBackend());
    b->device_id_ = device_id;
    if (auto r = check_hip(hipSetDevice(device_id)); !r) return unexpected(r.error());
    if (auto r = check_hip(hipStreamCreateWithFlags(&b->stream_, hipStreamNonBlocking)); !r)
        return unexpected(r.error());
    // The side stream a mixed prefill batch's decode items run on, and its fork / join events
    // (both streams at the default priority).
    if (auto r = check_hip(hipStreamCreateWithFlags(&b->side_stream_, hipStreamNonBlocking)); !r)
        return unexpected(r.error());
    if (auto r = check_hip(hipEventCreateWithFlags(&b->fork_event_, hipEventDisableTiming)); !r)
        return unexpected(r.error());
    if (auto r = check_hip(hipEventCreateWithFlags(&b->join_event_, hipEventDisableTiming)); !r)
        return unexpected(r.error());
    return b;
}

HipBackend::~HipBackend() {
    if (stream_ != nullptr) (void)hipStreamSynchronize(stream_);
    if (side_stream_ != nullptr) (void)hipStreamSynchronize(side_stream_);
    if (workspace_ != nullptr) (void)hipFree(workspace_);
    if (fork_event_ != nullptr) (void)hipEventDestroy(fork_event_);
    if (join_event_ != nullptr) (void)hipEventDestroy(join_event_);
    if (side_stream_ != nullptr) (void)hipStreamDestroy(side_stream_);
    if (stream_ != nullptr) (void)hipStreamDestroy(stream_);
}

Result<void> HipBackend::synchronize() { return check_hip(hipStreamSynchronize(stream_)); }

Result<void> HipBackend::reserve_workspace(const AttnWorkspaceLimits& lim) {
    const size_t bytes = attn_workspace_bytes(lim);
    if (bytes == 0) return unexpected(ErrorCode::InvalidArgument);
    if (bytes <= workspace_bytes_) return {};
    if (auto r = check_hip(hipSetDevice(device_id_)); !r) return r;
    if (workspace_ != nullptr) {
        // work queued on our streams may still read the old buffer
        if (auto r = check_hip(hipStreamSynchronize(stream_)); !r) return r;
        if (auto r = check_hip(hipStreamSynchronize(side_stream_)); !r) return r;
        (void)hipFree(workspace_);
        workspace_ = nullptr;
        workspace_bytes_ = 0;
    }
    if (auto r = check_hip(hipMalloc(&workspace_, bytes)); !r) return r;
    workspace_bytes_ = bytes;
    return {};
}

// The reserved workspace when it covers `bytes` (no allocation here).
Result<void*> HipBackend::workspace(size_t bytes) const {
    if (bytes == 0) return static_cast<void*>(nullptr);
    if (bytes > workspace_bytes_) return unexpected(ErrorCode::InvalidArgument);
    return workspace_;
}

template <>
Result<void> HipBackend::prefill_attention_impl<__hip_bfloat16>(const PrefillAttnParams& p) {
    const size_t need = ccinfer_prefill_workspace_size(p.batch_size_, p.num_tokens_,
                                                       p.max_blocks_per_req_, p.num_q_heads_,
                                                       p.num_kv_heads_, p.head_dim_,
                                                       p.cache_block_size_);
    auto ws = workspace(need);
    if (!ws) return unexpected(ws.error());
    return check(ccinfer_prefill_attention_overlap(
        p.q_, p.k_cache_, p.v_cache_, p.block_table_, p.query_start_loc_, p.context_lens_,
        p.output_, p.batch_size_, p.num_tokens_, p.max_blocks_per_req_, p.num_q_heads_,
        p.num_kv_heads_, p.head_dim_, p.cache_block_size_, *ws, need, stream_, side_stream_,
        fork_event_, join_event_));
}

template <>
Result<void> HipBackend::decode_attention_impl<__hip_bfloat16>(const DecodeAttnParams& p) {
    const size_t need = ccinfer_decode_workspace_size(p.batch_size_, p.max_blocks_per_req_,
                                                      p.num_q_heads_, p.num_kv_heads_,
                                                      p.head_dim_, p.cache_block_size_);
    auto ws = workspace(need);
    if (!ws) return unexpected(ws.error());
    return check(ccinfer_decode_attention(p.q_, p.k_cache_, p.v_cache_, p.block_table_,
                                          p.context_lens_, p.output_, p.batch_size_,
                                          p.max_blocks_per_req_, p.num_q_heads_,
                                          p.num_kv_heads_, p.head_dim_, p.cache_block_size_,
                                          *ws, need, stream_));
}

template <>
Result<void> HipBackend::write_kv_cache_impl<__hip_bfloat16>(const WriteKVCacheParams& p) {
    return check(ccinfer_write_kv_cache(p.k_new_, p.v_new_, p.k_cache_, p.v_cache_,
                                        p.slot_mapping_, p.total_tokens_, p.num_kv_heads_,
                                        p.head_dim_, p.max_slots_, stream_));
}

}  // namespace ccinfer
