// Per-step attention metadata built on the device.
//
// The reference builds these arrays on the host every step (BatchTranslator::translate,
// src/worker/batch_translator.cpp:213-302), uploads them with seven synchronous copies
// (:305-420), and ModelRunner copies four of them back to validate them before the forward
// (src/model/model_runner.h:102-171). Here the host uploads only compact per-item records
// (tokens already in the cache, new tokens, flags, each item's block list) and two kernels
// write positions, slot_mapping, the -1-padded block table, query_start_loc, context_lens
// and logits_indices in HBM, together with the validation verdict as a device status word
// (0, or ErrorCode::InvalidArgument = 6). Entries that fail a check are written sanitised
// (slot -1, table entry -1), so the attention kernels that read them never leave the cache.
//
//   batch_scan_kernel  : one workgroup; prefix sum of the query lengths (query_start_loc),
//                        context_lens, logits_indices, the per-item checks, and the status
//                        word (written on every call, so it needs no clearing).
//   batch_fill_kernel  : one workgroup per item; positions and slot_mapping of its tokens
//                        and its block-table row; block-id checks (sets status on failure).
// The second kernel reads the first's query_start_loc; both run on one stream, in order.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

constexpr int kScanThreads = 1024;
constexpr int kFillThreads = 256;
constexpr int kInvalidArgument = 6;

struct MetaArgs {
    const int32_t* kv_written;
    const int32_t* new_tokens;
    const int32_t* flags;
    const int32_t* block_start;
    const int32_t* blocks;
    int B, T, total_blocks, mbpr, bs, num_cache_blocks;
    int32_t* positions;
    int32_t* slot_mapping;
    int32_t* block_table;
    int32_t* qsl;
    int32_t* context_lens;
    int32_t* logits_indices;
    int32_t* status;
};

// Offsets and lengths past INT_MAX (a batch that fails validation) are stored as INT_MAX,
// so no token index derived from them wraps into the arrays.
__device__ __forceinline__ int32_t clamp_int(int64_t v) {
    return static_cast<int32_t>(v < INT_MAX ? v : INT_MAX);
}

// Blocks of item i, or an empty range when its [start, end) does not lie inside `blocks`.
__device__ __forceinline__ bool item_blocks(const MetaArgs& a, int i, int& b0, int& nblk) {
    b0 = a.block_start[i];
    const int b1 = a.block_start[i + 1];
    if (b0 < 0 || b1 < b0 || b1 > a.total_blocks) {
        b0 = 0;
        nblk = 0;
        return false;
    }
    nblk = b1 - b0;
    return true;
}

__global__ __launch_bounds__(kScanThreads) void batch_scan_kernel(MetaArgs a) {
    __shared__ int64_t scan[kScanThreads];
    __shared__ int err;
    const int tid = threadIdx.x;
    if (tid == 0) err = a.mbpr > a.num_cache_blocks;  // model_runner.h:136
    int64_t carry = 0;
    for (int base = 0; base < a.B; base += kScanThreads) {
        const int i = base + tid;
        int n = 0;
        bool bad = false;
        int len = 0, kvw = 0, fl = 0;
        int64_t ctx = 0;
        if (i < a.B) {
            len = a.new_tokens[i];
            kvw = a.kv_written[i];
            fl = a.flags[i];
            ctx = static_cast<int64_t>(kvw) + len;
            int b0, nblk;
            bad = !item_blocks(a, i, b0, nblk);
            bad |= len <= 0;                                    // model_runner.h:112
            bad |= (fl & kItemDecode) != 0 && len != 1;         // :115
            bad |= kvw < 0;                                     // :126 (positions >= 0)
            bad |= ctx <= 0 || ctx > static_cast<int64_t>(a.mbpr) * a.bs;  // :140-145
            bad |= nblk > a.mbpr || (ctx > 0 && nblk < (ctx + a.bs - 1) / a.bs);
            n = len > 0 ? len : 0;
        }
        // inclusive scan of n over the workgroup (Hillis-Steele in LDS)
        scan[tid] = n;
        __syncthreads();
        for (int d = 1; d < kScanThreads; d <<= 1) {
            const int64_t add = tid >= d ? scan[tid - d] : 0;
            __syncthreads();
            scan[tid] += add;
            __syncthreads();
        }
        const int64_t excl = carry + scan[tid] - n;
        if (i < a.B) {
            a.qsl[i] = clamp_int(excl);
            a.context_lens[i] = clamp_int(ctx);
            a.logits_indices[i] = (fl & (kItemDecode | kItemSample)) ? clamp_int(excl + n - 1) : -1;
            if (bad) err = 1;
        }
        carry += scan[kScanThreads - 1];
        __syncthreads();
    }
    if (tid == 0) {
        a.qsl[a.B] = clamp_int(carry);
        const bool bad = err != 0 || carry != a.T;  // model_runner.h:109
        a.status[0] = bad ? kInvalidArgument : 0;
    }
}

__global__ __launch_bounds__(kFillThreads) void batch_fill_kernel(MetaArgs a) {
    const int i = blockIdx.x;
    const int tid = threadIdx.x;
    const int off = a.qsl[i];
    const int len = a.new_tokens[i];
    const int kvw = a.kv_written[i];
    const int n = len > 0 ? len : 0;
    int b0, nblk;
    item_blocks(a, i, b0, nblk);
    bool bad = false;
    for (int t = tid; t < n; t += kFillThreads) {
        const int64_t tok = static_cast<int64_t>(off) + t;
        if (tok >= a.T) break;
        const int64_t pos = static_cast<int64_t>(kvw) + t;
        a.positions[tok] = static_cast<int32_t>(pos);
        int32_t slot = -1;
        if (pos >= 0) {
            const int64_t bidx = pos / a.bs;
            if (bidx < nblk) {
                const int blk = a.blocks[b0 + bidx];
                if (blk >= 0 && blk < a.num_cache_blocks)
                    slot = static_cast<int32_t>(static_cast<int64_t>(blk) * a.bs + pos % a.bs);
                else
                    bad = true;
            }
        }
        a.slot_mapping[tok] = slot;
    }
    for (int b = tid; b < a.mbpr; b += kFillThreads) {
        int32_t v = -1;
        if (b < nblk) {
            const int blk = a.blocks[b0 + b];
            if (blk >= 0 && blk < a.num_cache_blocks)
                v = blk;
            else
                bad = true;
        }
        a.block_table[static_cast<int64_t>(i) * a.mbpr + b] = v;
    }
    if (bad) a.status[0] = kInvalidArgument;  // every writer stores the same value
}

}  // namespace

hipError_t build_batch_metadata(const int32_t* item_kv_written, const int32_t* item_new_tokens,
                                const int32_t* item_flags, const int32_t* item_block_start,
                                const int32_t* blocks, int batch_size, int num_tokens,
                                int total_blocks, int max_blocks_per_req, int block_size,
                                int num_cache_blocks, int32_t* positions, int32_t* slot_mapping,
                                int32_t* block_table, int32_t* query_start_loc,
                                int32_t* context_lens, int32_t* logits_indices, int32_t* status,
                                hipStream_t stream) {
    MetaArgs a{item_kv_written, item_new_tokens, item_flags, item_block_start, blocks,
               batch_size,      num_tokens,      total_blocks, max_blocks_per_req, block_size,
               num_cache_blocks, positions,      slot_mapping, block_table, query_start_loc,
               context_lens,    logits_indices,  status};
    batch_scan_kernel<<<1, kScanThreads, 0, stream>>>(a);
    batch_fill_kernel<<<static_cast<unsigned>(batch_size), kFillThreads, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace ccinfer::hipk
