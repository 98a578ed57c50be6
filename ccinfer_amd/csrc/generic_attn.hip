// Generic paged prefill attention (any head_dim <= 256, any GQA ratio, any cache block
// size, any 2-byte-aligned view).
//
// Coverage path for the prefill shapes the MFMA kernels do not take (head dims that are not
// a multiple of 8, block sizes that are not a multiple of 16, caches that are only 2-byte
// aligned, head_dim 256 past 4096 table blocks). Same semantics as the reference launcher
// (prefill_attn.cu:43-242): one wavefront per (query row, q_head); 64 positions per step,
// one per lane, scores reduced with cross-lane max/sum; each lane accumulates up to 4
// output dims over the step's positions with an online softmax. Scalar fp32, not tuned.
// Also the row copies and the table expansion that put unaligned q / output views and
// blocks of 16k tokens on the MFMA paths.
#include <algorithm>

#include "attn_common.hpp"
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

constexpr int kMaxDims = 256;
constexpr int kDimsPerLane = kMaxDims / kWave;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Attends q_vec over positions [0, visible) of one block-table row. Writes bf16 output.
__device__ void attend_row(const __bf16* __restrict__ q_vec, const __bf16* __restrict__ k_cache,
                           const __bf16* __restrict__ v_cache,
                           const int32_t* __restrict__ req_blocks, int visible, int kv_head,
                           int head_dim, int hkv, int block_size, int mbpr, float scale_log2,
                           float eps, __bf16* __restrict__ out_vec) {
    const int lane = threadIdx.x & 63;
    float m = kNegInf, l = 0.f;
    float acc[kDimsPerLane];
#pragma unroll
    for (int x = 0; x < kDimsPerLane; ++x) acc[x] = 0.f;
    for (int base = 0; base < visible; base += kWave) {
        const int pos = base + lane;
        int64_t off = -1;
        float s = kNegInf;
        if (pos < visible) {
            off = kv_row_offset(pos, kv_head, head_dim, hkv, block_size, mbpr, req_blocks);
            if (off >= 0) {
                float dot = 0.f;
                for (int d = 0; d < head_dim; ++d)
                    dot += static_cast<float>(q_vec[d]) * static_cast<float>(k_cache[off + d]);
                s = dot * scale_log2;
            }
        }
        const float m_new = fmaxf(m, wave_max(s));
        const float m_use = m_new == kNegInf ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m - m_use);
        const float p = off >= 0 ? __builtin_amdgcn_exp2f(s - m_use) : 0.f;
        l = l * alpha + wave_sum(p);
        m = m_new;
#pragma unroll
        for (int x = 0; x < kDimsPerLane; ++x) acc[x] *= alpha;
        const int n = min(kWave, visible - base);
        for (int t = 0; t < n; ++t) {
            const float pt = __shfl(p, t);
            const int64_t ot = __shfl(off, t);
            if (ot < 0) continue;
#pragma unroll
            for (int x = 0; x < kDimsPerLane; ++x) {
                const int d = lane + x * kWave;
                if (d < head_dim) acc[x] += pt * static_cast<float>(v_cache[ot + d]);
            }
        }
    }
    const float inv = l > 0.f ? 1.f / (l + eps) : 0.f;
#pragma unroll
    for (int x = 0; x < kDimsPerLane; ++x) {
        const int d = lane + x * kWave;
        if (d < head_dim) out_vec[d] = static_cast<__bf16>(acc[x] * inv);
    }
}

__global__ __launch_bounds__(64) void generic_prefill_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k_cache,
    const __bf16* __restrict__ v_cache, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ context_lens,
    __bf16* __restrict__ out, int batch_size, int mbpr, int hq, int hkv, int head_dim,
    int block_size, float scale_log2) {
    const int gq = blockIdx.x / hq;
    const int qh = blockIdx.x % hq;
    int req = 0;
    while (req + 1 < batch_size && qsl[req + 1] <= gq) ++req;
    const int qb = qsl[req];
    const int qlen = qsl[req + 1] - qb;
    const int local = gq - qb;
    if (qlen <= 0 || local < 0 || local >= qlen) return;
    const int ctx = context_lens[req];
    const int prefix = ctx - qlen;
    if (prefix < 0) return;
    const int visible = prefix + local + 1;
    const int kvh = qh / (hq / hkv);
    attend_row(q + (static_cast<int64_t>(gq) * hq + qh) * head_dim, k_cache, v_cache,
               block_table + static_cast<int64_t>(req) * mbpr, visible, kvh, head_dim, hkv,
               block_size, mbpr, scale_log2, 0.f,
               out + (static_cast<int64_t>(gq) * hq + qh) * head_dim);
}

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

hipError_t generic_prefill_attention(const void* q, const void* k_cache, const void* v_cache,
                                     const int32_t* block_table,
                                     const int32_t* query_start_loc,
                                     const int32_t* context_lens, void* output, int batch_size,
                                     int total_query_tokens, int max_blocks_per_req,
                                     int num_q_heads, int num_kv_heads, int head_dim,
                                     int block_size, hipStream_t stream) {
    const float scale_log2 = kLog2e / sqrtf(static_cast<float>(head_dim));
    const int64_t grid = static_cast<int64_t>(total_query_tokens) * num_q_heads;
    generic_prefill_kernel<<<static_cast<unsigned>(grid), kWave, 0, stream>>>(
        static_cast<const __bf16*>(q), static_cast<const __bf16*>(k_cache),
        static_cast<const __bf16*>(v_cache), block_table, query_start_loc, context_lens,
        static_cast<__bf16*>(output), batch_size, max_blocks_per_req, num_q_heads,
        num_kv_heads, head_dim, block_size, scale_log2);
    return hipGetLastError();
}

}  // namespace ccinfer::hipk
