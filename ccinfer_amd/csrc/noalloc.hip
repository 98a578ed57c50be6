// Decode attention that allocates nothing and takes no workspace, for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). No counterpart in the reference.
//
// The split-KV partials and merge descriptors that ccinfer_decode_attention keeps in the
// caller's workspace live here in one file-scope device array, `scratch`, of
// kScratchBytes per GPU (each GPU the library runs on holds it until the process ends).
// Host code never passes the array's name to a kernel: on the first call on a device, with
// that device current, hipGetSymbolAddress resolves the device's own copy and the address
// is kept per device (that first call may itself be made under stream capture). Shapes whose plan needs more than kScratchBytes are rejected with
// CCINFER_ERR_INVALID_ARGUMENT. The partials need no clearing between calls (every launch
// rewrites what it reads). Calls that overlap on one GPU (concurrent streams) share the
// array and race.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include "ccinfer_attn.h"
#include "kernels.hpp"

namespace {

using namespace ccinfer::hipk;

constexpr size_t kScratchBytes = size_t{32} << 20;  // 32 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

// Device address of the current device's `scratch` (resolved once per device). A first
// call made while `stream` is being captured resolves the address with the thread in relaxed
// capture mode (the lookup enqueues no work, but the runtime's capture checks would
// otherwise reject or invalidate the capture).
hipError_t scratch_address(hipStream_t stream, void** out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
            err = hipStreamIsCapturing(stream, &status);
            if (err != hipSuccess) return err;
            const bool capturing = status != hipStreamCaptureStatusNone;
            hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
            if (capturing) {
                err = hipThreadExchangeStreamCaptureMode(&mode);
                if (err != hipSuccess) return err;
            }
            err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (capturing) {
                const hipError_t back = hipThreadExchangeStreamCaptureMode(&mode);
                if (err == hipSuccess) err = back;
            }
            if (err != hipSuccess) return err;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

}  // namespace

extern "C" int ccinfer_decode_attention_noalloc(const void* q, const void* k_cache,
                                                const void* v_cache, const int32_t* block_table,
                                                const int32_t* context_lens, void* output,
                                                int batch_size, int max_blocks_per_req,
                                                int num_q_heads, int num_kv_heads, int head_dim,
                                                int cache_block_size, void* stream) {
    size_t need = ccinfer_decode_workspace_size(batch_size, max_blocks_per_req, num_q_heads,
                                                num_kv_heads, head_dim, cache_block_size);
    // the q / output row copies are needed only for views that are not 16-byte aligned
    if (need > 0 && ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(output)) &
                     15u) == 0)
        need = ccinfer::hipk::decode_bytes_for(batch_size, max_blocks_per_req, num_q_heads,
                                               num_kv_heads, head_dim, cache_block_size, false);
    if (need > kScratchBytes) return CCINFER_ERR_INVALID_ARGUMENT;
    void* ws = nullptr;
    if (need > 0) {
        const hipError_t err = scratch_address(static_cast<hipStream_t>(stream), &ws);
        if (err != hipSuccess) return CCINFER_ERR_DEVICE_RUNTIME;
    }
    // The workspace path's validation, plan and kernels, on the static array.
    return ccinfer_decode_attention(q, k_cache, v_cache, block_table, context_lens, output,
                                    batch_size, max_blocks_per_req, num_q_heads, num_kv_heads,
                                    head_dim, cache_block_size, ws, need, stream);
}
