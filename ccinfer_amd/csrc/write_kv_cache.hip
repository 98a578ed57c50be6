// KV-cache write: scatter each new token's K and V rows into its cache slot.
//
// Semantics follow src/kernel/attention/write_kv_cache.cu:12-34 of the reference:
//   cache[slot_mapping[t]][h][d] = new[t][h][d] for K and V, tokens whose slot lies
//   outside [0, max_slots) are skipped. The copy is bit-exact.
//
// Design: the [n_kv_heads][head_dim] row of one token is contiguous in both the
// source and the cache, so the write is a row copy. One workgroup per token moves
// the K row and the V row with 16-byte loads/stores (128-bit, fully coalesced: a
// 2 KiB row is 128 lanes x 16 B). Rows whose byte size is not a multiple of 16 (or
// misaligned buffers) use a 2-byte path.
#include "attn_common.hpp"
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void write_kv_rows16(
    const u32x4* __restrict__ k_new, const u32x4* __restrict__ v_new, u32x4* __restrict__ k_cache,
    u32x4* __restrict__ v_cache, const int32_t* __restrict__ slot_mapping, int chunks_per_row,
    int max_slots) {
    const int t = blockIdx.x;
    const int slot = slot_mapping[t];
    if (slot < 0 || slot >= max_slots) return;
    const int64_t src = static_cast<int64_t>(t) * chunks_per_row;
    const int64_t dst = static_cast<int64_t>(slot) * chunks_per_row;
    for (int c = threadIdx.x; c < 2 * chunks_per_row; c += kThreads) {
        if (c < chunks_per_row) {
            k_cache[dst + c] = k_new[src + c];
        } else {
            v_cache[dst + c - chunks_per_row] = v_new[src + c - chunks_per_row];
        }
    }
}

__global__ __launch_bounds__(kThreads) void write_kv_rows2(
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int row_elems, int max_slots) {
    const int t = blockIdx.x;
    const int slot = slot_mapping[t];
    if (slot < 0 || slot >= max_slots) return;
    const int64_t src = static_cast<int64_t>(t) * row_elems;
    const int64_t dst = static_cast<int64_t>(slot) * row_elems;
    for (int e = threadIdx.x; e < row_elems; e += kThreads) {
        k_cache[dst + e] = k_new[src + e];
        v_cache[dst + e] = v_new[src + e];
    }
}

// Request b's new token into the slot of its last position ctx_b - 1 (through its table
// row); rows with ctx outside [1, mbpr * 16], a negative block id or a slot past max_slots
// are skipped.
__global__ __launch_bounds__(kThreads) void write_last_tokens_kernel(
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ context_lens, int mbpr,
    int row_elems, int max_slots) {
    const int b = blockIdx.x;
    const int ctx = context_lens[b];
    if (ctx < 1 || ctx > mbpr * 16) return;
    const int pos = ctx - 1;
    const int pb = block_table[static_cast<int64_t>(b) * mbpr + pos / 16];
    if (pb < 0) return;
    const int64_t slot = static_cast<int64_t>(pb) * 16 + pos % 16;
    if (slot >= max_slots) return;
    const int64_t src = static_cast<int64_t>(b) * row_elems;
    const int64_t dst = slot * row_elems;
    for (int e = threadIdx.x; e < row_elems; e += kThreads) {
        k_cache[dst + e] = k_new[src + e];
        v_cache[dst + e] = v_new[src + e];
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t write_kv_cache(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                          const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                          int head_dim, int max_slots, hipStream_t stream) {
    const int row_elems = n_kv_heads * head_dim;
    const int row_bytes = row_elems * 2;
    if (row_bytes % 16 == 0 && aligned16(k_new) && aligned16(v_new) && aligned16(k_cache) &&
        aligned16(v_cache)) {
        write_kv_rows16<<<total_tokens, kThreads, 0, stream>>>(
            static_cast<const u32x4*>(k_new), static_cast<const u32x4*>(v_new),
            static_cast<u32x4*>(k_cache), static_cast<u32x4*>(v_cache), slot_mapping,
            row_bytes / 16, max_slots);
    } else {
        write_kv_rows2<<<total_tokens, kThreads, 0, stream>>>(
            static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new),
            static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), slot_mapping,
            row_elems, max_slots);
    }
    return hipGetLastError();
}

hipError_t write_last_tokens(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                             const int32_t* block_table, const int32_t* context_lens,
                             int batch_size, int max_blocks_per_req, int n_kv_heads, int head_dim,
                             int max_slots, hipStream_t stream) {
    write_last_tokens_kernel<<<batch_size, kThreads, 0, stream>>>(
        static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new),
        static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), block_table,
        context_lens, max_blocks_per_req, n_kv_heads * head_dim, max_slots);
    return hipGetLastError();
}

}  // namespace ccinfer::hipk
