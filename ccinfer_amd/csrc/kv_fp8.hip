// KV-cache write into an fp8 (OCP E4M3) cache with one fp32 scale per cache row.
//
// There is no counterpart in the reference, whose cache is bf16 only (its KV profile list,
// src/base/traits.h:117-124, anticipates other element types). The layout keeps the
// reference's contract -- [slot][kv_head][head_dim], slot = block * 16 + offset -- with one
// byte per element, plus two fp32 scale arrays (K and V) indexed
//   ((slot / 16) * Hkv + kv_head) * 16 + slot % 16,
// so the 16 scales of one block's rows for one head are contiguous (a 64-byte line the
// decode kernel reads with two 16-byte loads per chunk).
//
// Quantisation of one row x[0..D): amax = max |x|; scale = the smallest power of two P
// (at least 2^-126) with amax <= 448 P; q = e4m3(clamp(x / P, +-448)) rounded to nearest
// even (an all-zero row stores zeros and scale 0). Dequantised value = q * scale. Per-row
// scales make appends exact: a decode step writes one new row and never has to requantise
// earlier rows of the block. A power-of-two scale (as in the OCP microscaling formats'
// E8M0 scales) loses no relative precision -- x / P is exact and E4M3 has the same
// relative spacing at every exponent -- and lets a consumer apply it inside the hardware's
// scaled fp8 -> bf16 conversion, which uses only the exponent of its scale operand.
//
// Head dims 64/128/256/512 (aligned buffers): D/8 lanes per row, 8 elements per lane.
// Other even head dims: one wavefront per (token, kv_head, K or V) row, lane l holding
// elements 2l, 2l+1 (+128 per step for rows longer than 128).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "attn_common.hpp"
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

constexpr int kWaves = 4;

// The row scale: the smallest power of two P >= 2^-126 with amax <= 448 P (448 = 0.875 *
// 2^9), 0 for an all-zero row, and 2^126 for a row holding an infinity (its infinities
// store as +-448 and dequantise to +-inf again; its finite elements store as zeros).
__device__ __forceinline__ float fp8_row_scale(float amax) {
    if (!(amax > 0.f)) return 0.f;
    if (__builtin_isinf(amax)) return 0x1p126f;
    int e;
    const float f = frexpf(amax, &e);  // amax = f * 2^e, f in [0.5, 1)
    int p = e - 9 + (f > 0.875f ? 1 : 0);
    p = p < -126 ? -126 : p;
    return ldexpf(1.0f, p);
}

__device__ __forceinline__ float wave_max_all(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

template <int kSteps>  // kSteps * 128 elements per row at most
__global__ __launch_bounds__(256) void write_kv_fp8_kernel(
    const __bf16* __restrict__ k_new, const __bf16* __restrict__ v_new, uint8_t* __restrict__ k_cache,
    uint8_t* __restrict__ v_cache, float* __restrict__ k_scale, float* __restrict__ v_scale,
    const int32_t* __restrict__ slot_mapping, int total_tokens, int hkv, int d, int max_slots) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;  // (t, h, kv)
    if (row >= static_cast<int64_t>(total_tokens) * hkv * 2) return;
    const bool is_v = row & 1;
    const int64_t th = row >> 1;
    const int t = static_cast<int>(th / hkv);
    const int h = static_cast<int>(th - static_cast<int64_t>(t) * hkv);
    const int slot = slot_mapping[t];
    if (slot < 0 || slot >= max_slots) return;
    const __bf16* src = (is_v ? v_new : k_new) + th * d;
    uint8_t* dst = (is_v ? v_cache : k_cache) + (static_cast<int64_t>(slot) * hkv + h) * d;

    float x[kSteps][2];
    float amax = 0.f;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        const int e = s * 128 + 2 * lane;
        x[s][0] = e < d ? static_cast<float>(src[e]) : 0.f;
        x[s][1] = e + 1 < d ? static_cast<float>(src[e + 1]) : 0.f;
        amax = fmaxf(amax, fmaxf(fabsf(x[s][0]), fabsf(x[s][1])));
    }
    amax = wave_max_all(amax);
    const float scale = fp8_row_scale(amax);
    const float inv = amax > 0.f ? 1.0f / scale : 0.f;  // exact: a power of two
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        const int e = s * 128 + 2 * lane;
        if (e >= d) break;
        const float a = fminf(fmaxf(x[s][0] * inv, -448.0f), 448.0f);
        const float b = fminf(fmaxf(x[s][1] * inv, -448.0f), 448.0f);
        const uint32_t pk = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false));
        *reinterpret_cast<uint16_t*>(dst + e) = static_cast<uint16_t>(pk & 0xffffu);
    }
    if (lane == 0) {
        const int64_t si = (static_cast<int64_t>(slot / kFp8Block) * hkv + h) * kFp8Block +
                           slot % kFp8Block;
        (is_v ? v_scale : k_scale)[si] = scale;
    }
}

// Head dims that are multiples of 8: LPR = D / 8 lanes per row, 8 elements (one 16-byte
// load, one 8-byte store) per lane, 64 / LPR rows per wavefront. Same arithmetic as above.
template <int LPR>
__global__ __launch_bounds__(256) void write_kv_fp8_vec_kernel(
    const __bf16* __restrict__ k_new, const __bf16* __restrict__ v_new, uint8_t* __restrict__ k_cache,
    uint8_t* __restrict__ v_cache, float* __restrict__ k_scale, float* __restrict__ v_scale,
    const int32_t* __restrict__ slot_mapping, int total_tokens, int hkv, int max_slots) {
    constexpr int D = LPR * 8;
    constexpr int kRowsPerWave = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane % LPR;                 // lane within its row
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) *
                            kRowsPerWave + lane / LPR;  // (t, h, K/V)
    const bool live = row < static_cast<int64_t>(total_tokens) * hkv * 2;
    const bool is_v = row & 1;
    const int64_t th = row >> 1;
    const int t = live ? static_cast<int>(th / hkv) : 0;
    const int h = static_cast<int>(th - static_cast<int64_t>(t) * hkv);
    const int slot = live ? slot_mapping[t] : -1;
    const bool write = live && slot >= 0 && slot < max_slots;

    u32x4 w = u32x4{0, 0, 0, 0};
    if (live) w = load16((is_v ? v_new : k_new) + th * D + sub * 8);
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(w[i] << 16);
        x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float scale = fp8_row_scale(amax);
    const float inv = amax > 0.f ? 1.0f / scale : 0.f;  // exact: a power of two
    uint32_t q[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        float a[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = fminf(fmaxf(x[4 * i + e] * inv, -448.0f), 448.0f);
        const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a[0], a[1], 0, false);
        q[i] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a[2], a[3], lo, true));
    }
    if (!write) return;
    uint8_t* dst = (is_v ? v_cache : k_cache) + (static_cast<int64_t>(slot) * hkv + h) * D;
    *reinterpret_cast<u32x2*>(dst + sub * 8) = u32x2{q[0], q[1]};
    if (sub == 0) {
        const int64_t si = (static_cast<int64_t>(slot / kFp8Block) * hkv + h) * kFp8Block +
                           slot % kFp8Block;
        (is_v ? v_scale : k_scale)[si] = scale;
    }
}

}  // namespace

hipError_t write_kv_cache_fp8(const void* k_new, const void* v_new, void* k_cache,
                              void* v_cache, float* k_scale, float* v_scale,
                              const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                              int head_dim, int max_slots, hipStream_t stream) {
    const int64_t rows = static_cast<int64_t>(total_tokens) * n_kv_heads * 2;
    const unsigned grid = static_cast<unsigned>((rows + kWaves - 1) / kWaves);
    auto* kn = static_cast<const __bf16*>(k_new);
    auto* vn = static_cast<const __bf16*>(v_new);
    auto* kc = static_cast<uint8_t*>(k_cache);
    auto* vc = static_cast<uint8_t*>(v_cache);
    const bool aligned = reinterpret_cast<uintptr_t>(k_new) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(v_new) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(k_cache) % 8 == 0 &&
                         reinterpret_cast<uintptr_t>(v_cache) % 8 == 0;
    auto vec = [&](auto lpr_tag) {
        constexpr int LPR = decltype(lpr_tag)::value;
        const int64_t waves = (rows + 64 / LPR - 1) / (64 / LPR);
        write_kv_fp8_vec_kernel<LPR><<<static_cast<unsigned>((waves + kWaves - 1) / kWaves), 256,
                                       0, stream>>>(kn, vn, kc, vc, k_scale, v_scale,
                                                    slot_mapping, total_tokens, n_kv_heads,
                                                    max_slots);
        return hipGetLastError();
    };
    if (aligned && head_dim == 64) return vec(std::integral_constant<int, 8>{});
    if (aligned && head_dim == 128) return vec(std::integral_constant<int, 16>{});
    if (aligned && head_dim == 256) return vec(std::integral_constant<int, 32>{});
    if (aligned && head_dim == 512) return vec(std::integral_constant<int, 64>{});
    if (head_dim <= 128)
        write_kv_fp8_kernel<1><<<grid, 256, 0, stream>>>(kn, vn, kc, vc, k_scale, v_scale,
                                                         slot_mapping, total_tokens, n_kv_heads,
                                                         head_dim, max_slots);
    else if (head_dim <= 256)
        write_kv_fp8_kernel<2><<<grid, 256, 0, stream>>>(kn, vn, kc, vc, k_scale, v_scale,
                                                         slot_mapping, total_tokens, n_kv_heads,
                                                         head_dim, max_slots);
    else
        write_kv_fp8_kernel<4><<<grid, 256, 0, stream>>>(kn, vn, kc, vc, k_scale, v_scale,
                                                         slot_mapping, total_tokens, n_kv_heads,
                                                         head_dim, max_slots);
    return hipGetLastError();
}

}  // namespace ccinfer::hipk
