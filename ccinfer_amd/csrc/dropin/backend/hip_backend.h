// HipBackend: the MI355X implementation of the hot-path backend ops (the reference's
// CudaBackend::{prefill,decode}_attention_impl / write_kv_cache_impl,
// src/backend/cuda/cuda_backend.cpp:162-187). It owns one HIP stream (default priority),
// a side stream plus fork/join events on which a mixed prefill batch's decode items run
// beside its prompt tiles, and one device workspace for the split-KV partials and the
// prefill work list. The workspace is reserved once, by reserve_workspace, for the largest
// shapes the caller will run (the reference's Worker::init_resources sizes its KV cache at
// the same point, src/worker/worker.cpp:223-294); the ops never allocate, free or
// synchronise, so they can be captured in a HIP graph. An op whose shape needs more
// workspace than was reserved returns ErrorCode::InvalidArgument.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <memory>

#include "backend/backend.h"
#include "kernel/hip_kernels.h"

namespace ccinfer {

class HipBackend : public DeviceBackend<HipBackend> {
public:
    // Creates a backend bound to `device_id` with its own stream.
    static Result<std::unique_ptr<HipBackend>> create(int device_id);
    ~HipBackend();
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;

    hipStream_t stream() const { return stream_; }
    int device_id() const { return device_id_; }
    Result<void> synchronize();

    // Reserves workspace for every decode / prefill op within `lim` (allocates; when a smaller
    // reservation exists, synchronises the backend's streams and replaces it). Call at
    // initialisation, outside stream capture.
    Result<void> reserve_workspace(const AttnWorkspaceLimits& lim);
    size_t reserved_workspace_bytes() const { return workspace_bytes_; }

    template <typename DType>
    Result<void> prefill_attention_impl(const PrefillAttnParams& p);
    template <typename DType>
    Result<void> decode_attention_impl(const DecodeAttnParams& p);
    template <typename DType>
    Result<void> write_kv_cache_impl(const WriteKVCacheParams& p);

private:
    HipBackend() = default;
    Result<void*> workspace(size_t bytes) const;

    int device_id_ = 0;
    hipStream_t stream_ = nullptr;
    hipStream_t side_stream_ = nullptr;
    hipEvent_t fork_event_ = nullptr;
    hipEvent_t join_event_ = nullptr;
    void* workspace_ = nullptr;
    size_t workspace_bytes_ = 0;
};

template <>
Result<void> HipBackend::prefill_attention_impl<__hip_bfloat16>(const PrefillAttnParams& p);
template <>
Result<void> HipBackend::decode_attention_impl<__hip_bfloat16>(const DecodeAttnParams& p);
template <>
Result<void> HipBackend::write_kv_cache_impl<__hip_bfloat16>(const WriteKVCacheParams& p);

// The reference's DefaultBackend alias (src/backend/default_backend.h).
using DefaultBackend = HipBackend;

}  // namespace ccinfer
