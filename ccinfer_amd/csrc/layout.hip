// Layout helpers around the MFMA paths: row copies that put q / output views which are
// only 2-byte aligned on 16-byte-aligned workspace rows, and the expansion of a table of
// 16k-token blocks into the equivalent table of 16-token blocks.
#include <algorithm>

#include "attn_common.hpp"
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

// Row copies between a caller's 2-byte-aligned bf16 view and a 16-byte-aligned workspace
// copy, 8 elements per thread (n is a multiple of 8). The unaligned side moves 2-byte
// elements (neighbouring lanes' elements are contiguous, so a wavefront still reads and
// writes whole cache lines); the aligned side moves 16 bytes per lane.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* __restrict__ src,
                                                          uint4* __restrict__ dst,
                                                          int64_t chunks) {
    for (int64_t i = blockIdx.x * int64_t{256} + threadIdx.x; i < chunks;
         i += int64_t{gridDim.x} * 256) {
        const uint16_t* s = src + i * 8;
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = s[2 * j] | (static_cast<uint32_t>(s[2 * j + 1]) << 16);
        dst[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

__global__ __launch_bounds__(256) void scatter_rows_kernel(const uint4* __restrict__ src,
                                                           uint16_t* __restrict__ dst,
                                                           int64_t chunks) {
    for (int64_t i = blockIdx.x * int64_t{256} + threadIdx.x; i < chunks;
         i += int64_t{gridDim.x} * 256) {
        const uint4 v = src[i];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint16_t* d = dst + i * 8;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            d[2 * j] = static_cast<uint16_t>(w[j]);
            d[2 * j + 1] = static_cast<uint16_t>(w[j] >> 16);
        }
    }
}

// Table of `bs`-token blocks -> table of 16-token blocks: entry j of a row is sub-block
// j % k of block j / k (k = bs / 16), i.e. the same cache rows. Negative entries stay.
__global__ __launch_bounds__(256) void expand_table_kernel(const int32_t* __restrict__ bt,
                                                           int32_t* __restrict__ out,
                                                           int64_t entries, int k) {
    for (int64_t i = blockIdx.x * int64_t{256} + threadIdx.x; i < entries;
         i += int64_t{gridDim.x} * 256) {
        const int32_t id = bt[i / k];
        // unsigned: entries past a row's context may hold any value and are never read
        out[i] = id < 0 ? id
                        : static_cast<int32_t>(static_cast<uint32_t>(id) * static_cast<uint32_t>(k) +
                                               static_cast<uint32_t>(i % k));
    }
}

unsigned copy_grid(int64_t items) {
    return static_cast<unsigned>(std::min<int64_t>((items + 255) / 256, 4096));
}

}  // namespace

hipError_t gather_rows(const void* src, void* dst, int64_t elems, hipStream_t stream) {
    const int64_t chunks = elems / 8;
    if (chunks <= 0) return hipSuccess;
    gather_rows_kernel<<<copy_grid(chunks), 256, 0, stream>>>(
        static_cast<const uint16_t*>(src), static_cast<uint4*>(dst), chunks);
    return hipGetLastError();
}

hipError_t scatter_rows(const void* src, void* dst, int64_t elems, hipStream_t stream) {
    const int64_t chunks = elems / 8;
    if (chunks <= 0) return hipSuccess;
    scatter_rows_kernel<<<copy_grid(chunks), 256, 0, stream>>>(
        static_cast<const uint4*>(src), static_cast<uint16_t*>(dst), chunks);
    return hipGetLastError();
}

hipError_t expand_block_table(const int32_t* block_table, int32_t* out, int rows,
                              int max_blocks_per_req, int k, hipStream_t stream) {
    const int64_t entries = static_cast<int64_t>(rows) * max_blocks_per_req * k;
    expand_table_kernel<<<copy_grid(entries), 256, 0, stream>>>(block_table, out, entries, k);
    return hipGetLastError();
}

}  // namespace ccinfer::hipk
