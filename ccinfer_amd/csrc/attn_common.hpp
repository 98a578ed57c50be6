// Device-side helpers shared by the paged-attention kernels (gfx950 / CDNA4 only).
//
// KV cache layout (kept identical to the reference so callers need no change):
//   k_cache, v_cache : [num_slots][num_kv_heads][head_dim] bf16, one buffer per layer,
//   slot = physical_block * cache_block_size + offset_in_block
//   (reference: src/cache/kv_cache_storage.cpp:75-136, src/kernel/attention/attn_common.cuh:7-27).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ccinfer::hipk {

using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using f32x2 = float __attribute__((ext_vector_type(2)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using f32x16 = float __attribute__((ext_vector_type(16)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using u32x1 = uint32_t __attribute__((ext_vector_type(1)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
using u32x3 = uint32_t __attribute__((ext_vector_type(3)));
// A 12-byte piece at 4-byte alignment: loads through this type claim only that alignment,
// so the compiler may not widen them to 16 bytes past the piece.
typedef u32x3 u32x3_a4 __attribute__((aligned(4)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// Token-to-cache-row mapping of the reference (attn_common.cuh:7-27): position p of a
// request lives in slot table[p / block_size] * block_size + p % block_size, at element
// (slot * num_kv_heads + kv_head) * head_dim; a negative table entry, or a block past the
// table row, holds no position. Every kernel computes it inline in the form its staging
// needs (a wave-uniform block base plus a per-lane row offset in the pipelined prefill,
// a readlane of the split's block ids in decode, a per-lane block lookup in the
// any-layout staging).

// Round-to-nearest-even fp32 -> bf16 pair (gfx950 has a native packed convert).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    using bf16x2 = __bf16 __attribute__((ext_vector_type(2)));
    bf16x2 v;
    v[0] = static_cast<__bf16>(lo);
    v[1] = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

// Select the 16-bit half `half` of a and b and pack {a.half, b.half}.
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, uint32_t b, int half) {
    // v_perm_b32: bytes 0-3 of the selector index src1 (a), 4-7 index src0 (b).
    return __builtin_amdgcn_perm(b, a, half ? 0x07060302u : 0x05040100u);
}

__device__ __forceinline__ float wave_max_xor16_32(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

// Max over lanes l and l^32 (one permlane32_swap).
__device__ __forceinline__ float wave_max_swap32(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}

__device__ __forceinline__ float wave_sum_xor16_32(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b,
                                               const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Two OCP E4M3 bytes (the low or high half of `w`) -> a bf16 pair, times 2^e where e is
// the exponent of `pow2` (the conversion uses only the scale's exponent field); exact
// (every E4M3 value times a power of two in bf16's range is a bf16 value).
template <bool kHi>
__device__ __forceinline__ uint32_t e4m3x2_to_bf16x2(uint32_t w, float pow2 = 1.0f) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(
                                            static_cast<int>(w), pow2, kHi));
}

// The N (2 or 4) 32-bit words at p, a 2-byte-aligned address `a` bytes past a 16-byte
// boundary (a per lane): the aligned 16-byte granules that hold those bytes are loaded --
// the second one only by lanes whose piece reaches into it, so no granule without one of
// the piece's bytes is touched (nothing outside the pages the data occupies) -- and the
// words are shifted into place. Two 16-byte loads per piece instead of eight 2-byte ones.
template <int N, typename T>
__device__ __forceinline__ T load_shifted(const void* p) {
    const uintptr_t u = reinterpret_cast<uintptr_t>(p);
    const int a = static_cast<int>(u & 15u);
    const u32x4* g = reinterpret_cast<const u32x4*>(u - static_cast<uintptr_t>(a));
    T out;
    const u32x4 lo = g[0];
    const bool two = a + 4 * N > 16;  // the piece reaches into the next granule
    const u32x4 hi = two ? g[1] : u32x4{0u, 0u, 0u, 0u};
    const uint32_t w[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const int q = a >> 2;          // whole words
    const bool half = (a & 2) != 0;  // plus one 16-bit half
    auto word = [&](int j) -> uint32_t {
        uint32_t x0 = 0, x1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (q == k) {
                x0 = w[(j + k) & 7];
                x1 = w[(j + k + 1) & 7];
            }
        }
        return half ? __builtin_amdgcn_alignbyte(x1, x0, 2) : x0;
    };
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = word(j);
    return out;
}

__device__ __forceinline__ u32x4 load16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

}  // namespace ccinfer::hipk
