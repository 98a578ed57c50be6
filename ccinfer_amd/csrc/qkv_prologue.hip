// Decode-side attention prologue for gfx950, fused into one launch: split the packed QKV
// projection, RMS-normalise q and k per head, rotate them with split-half RoPE, store q and
// write the new K/V rows into the paged cache.
//
// The reference runs this as five launches per layer (src/model/qwen3/qwen3_model.cpp:174-244):
//   split_qkv  (src/kernel/elementwise/elementwise.cu:34-64)
//   rms_norm q, rms_norm k (src/kernel/norm/rms_norm.cu:22-88, reduction order of
//                           src/kernel/cuda_common.cuh:14-62)
//   rope       (src/kernel/pos/rope.cu:14-43)
//   write_kv_cache (src/kernel/attention/write_kv_cache.cu:12-34)
// and each reads and writes the rows it touches from HBM; here every row is read once and
// written once.
//
// Numerics follow the reference step by step: the sum of squares adds (x[2i]^2 + x[2i+1]^2)
// per pair, rounds the partial sum to bf16 after every addition, reduces the partials with
// the reference's 32-lane trees and rounds the total to bf16; normalised values are rounded
// to bf16 before RoPE (as the reference stores them between its kernels); RoPE uses the
// caller's (cos, sin) table.
//
// head_dim 128 (the fast path): a wavefront holds one (token, head) row at a time (R rows per
// wavefront, their loads issued together). Lane l holds elements
// 2l and 2l+1 -- exactly the pair thread l of the reference kernel sums, so lanes 0..31 and
// 32..63 are the reference's two warps and the same trees apply. The RoPE partner of element
// j is j + 64, held by lane l ^ 32, and is fetched with v_permlane32_swap. A wavefront that
// handles a K row also copies the matching V row into the cache.
// Other head dims: one workgroup of 256 threads per row, laid out as the reference kernel.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "attn_common.hpp"
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

__device__ __forceinline__ float bf16_round(float x) {
    return static_cast<float>(static_cast<__bf16>(x));
}

__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Sum over one 32-lane half with the reference's shfl_down tree (offsets 16..1); lane 0 of
// the half ends with the total.
__device__ __forceinline__ float half_tree_sum(float v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v += __shfl_down(v, off, 32);
    return v;
}

struct PrologueArgs {
    const __bf16* qkv;
    const __bf16* q_norm_w;
    const __bf16* k_norm_w;
    const int32_t* positions;
    const float2* rope_cache;
    const int32_t* slot_mapping;
    __bf16* q_out;
    __bf16* k_cache;
    __bf16* v_cache;
    int T, nq, nkv, hd, rope_max, max_slots;
    float eps;
};

constexpr int kWavesPerGroup = 4;  // fast path: wavefronts per workgroup

template <int Ctrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xf, 0xf, true));
}

// The reference's sum of squares of one D = 128 row held as lane pairs: thread l's term
// x[2l]^2 + x[2l+1]^2 rounded to bf16 (one term per thread at this size), a shfl_down tree
// with offsets 16, 8, 4, 2, 1 inside each 32-lane warp, then warp 0's sum + warp 1's sum.
// The tree runs on cross-lane moves without LDS: v_permlane16_swap brings lane l + 16 to
// lanes 0..15 (and 32..47), DPP row_shl:n brings lane l + n within a row of 16 lanes, and
// v_permlane32_swap brings lane 32's sum to lane 0. Lane 0 ends with the total (unrounded),
// added in exactly the reference's order.
__device__ __forceinline__ float row_sum_squares(float x0, float x1) {
    float v = bf16_round(x0 * x0 + x1 * x1);
    const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                      false, false);
    v += __uint_as_float(s16[1]);  // lanes 0..15: v[l] + v[l + 16]
    v += dpp_f<0x108>(v);          // row_shl:8
    v += dpp_f<0x104>(v);          // row_shl:4
    v += dpp_f<0x102>(v);          // row_shl:2
    v += dpp_f<0x101>(v);          // row_shl:1 -> lane 0: warp 0's sum, lane 32: warp 1's
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                      false, false);
    return v + __uint_as_float(s32[1]);
}

// R rows per wavefront, interleaved across the workgroup's waves so that each step of the
// four waves covers four consecutive rows. kNorm: both norm weights given (else neither).
//
// Phases: (1) positions and slots (scalar loads); (2) every vector load of the R rows (QKV
// row, V row, (cos, sin) pairs), unconditional -- a q row "loads V" from its own row, an
// out-of-table position reads row 0 -- and fenced from the math; (3) sums of squares, the
// totals of the R rows gathered into lanes 0..R-1 of one register so that the correctly
// rounded sqrt and division run once for all rows; (4) normalise and rotate; (5) stores.
template <int R, bool kNorm>
__global__ __launch_bounds__(256) void qkv_prologue_d128_kernel(PrologueArgs a) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int heads = a.nq + a.nkv;
    const int total = a.T * heads;  // fits in int (checked by the caller)
    const int64_t qkv_row = static_cast<int64_t>(a.nq + 2 * a.nkv) * D;
    const int p0 = 2 * (lane & 31);  // pair index of element 2*lane (mod D/2)
    const bool lo_half = lane < 32;
    const uint32_t sin_sign = lo_half ? 0x80000000u : 0u;  // lo element: x0 c - x1 s

    float qw0 = 0.f, qw1 = 0.f, kw0 = 0.f, kw1 = 0.f;
    if constexpr (kNorm) {
        const uint32_t qnw = reinterpret_cast<const uint32_t*>(a.q_norm_w)[lane];
        const uint32_t knw = reinterpret_cast<const uint32_t*>(a.k_norm_w)[lane];
        qw0 = lo_f(qnw), qw1 = hi_f(qnw), kw0 = lo_f(knw), kw1 = hi_f(knw);
    }

    // Row of step r: (blockIdx.x * R + r) * waves + wave. The (token, head) pair of the first
    // row takes one division; later rows advance by `waves` heads. Rows past the end are
    // clamped to the last row for loading and skipped when storing.
    const int row0 = (blockIdx.x * R) * kWavesPerGroup + wave;
    const int last_t = a.T - 1;
    int t = row0 / heads;
    int h = row0 - t * heads;
    int tok[R], tl[R], lh[R], pos_r[R], slot_r[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r > 0) {
            h += kWavesPerGroup;
            while (h >= heads) { h -= heads; ++t; }
        }
        const bool valid = row0 + r * kWavesPerGroup < total;
        tl[r] = valid ? t : last_t;
        lh[r] = valid ? h : heads - 1;
        tok[r] = valid ? t : -1;
        slot_r[r] = a.slot_mapping[tl[r]];
        pos_r[r] = a.positions[tl[r]];
    }

    uint32_t w[R], v[R];
    float4 cs[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int hl = lh[r];
        const __bf16* src = a.qkv + tl[r] * qkv_row + static_cast<int64_t>(hl) * D;
        const __bf16* vsrc = hl >= a.nq ? src + static_cast<int64_t>(a.nkv) * D : src;
        w[r] = reinterpret_cast<const uint32_t*>(src)[lane];
        v[r] = reinterpret_cast<const uint32_t*>(vsrc)[lane];
        const int pos = pos_r[r];
        const int pos_c = (pos >= 0 && pos < a.rope_max) ? pos : 0;
        cs[r] = *reinterpret_cast<const float4*>(a.rope_cache +
                                                 static_cast<int64_t>(pos_c) * (D / 2) + p0);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any math below

    float inv_rms_lanes = 0.f;  // lane r: 1 / rms of row r
    if constexpr (kNorm) {
        float totals = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float sum = row_sum_squares(lo_f(w[r]), hi_f(w[r]));
            const float sum0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), 0));
            totals = lane == r ? sum0 : totals;
        }
        inv_rms_lanes = 1.0f / sqrtf(bf16_round(totals) / static_cast<float>(D) + a.eps);
    }

    uint32_t out[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const bool is_q = lh[r] < a.nq;
        uint32_t x = w[r];
        if constexpr (kNorm) {
            const float inv = __int_as_float(
                __builtin_amdgcn_readlane(__float_as_int(inv_rms_lanes), r));
            x = pack_bf16x2((lo_f(x) * inv) * (is_q ? qw0 : kw0),
                            (hi_f(x) * inv) * (is_q ? qw1 : kw1));
        }
        // Partner elements 2l+64, 2l+65 (lane l < 32) or 2l-64, 2l-63 (lane l >= 32).
        // v_permlane32_swap moves VSRC's lanes 0..31 into VDST's lanes 32..63 and VDST's
        // lanes 32..63 into VSRC's lanes 0..31; with both operands x, the returned VSRC
        // (element 1) holds x[l + 32] in lanes 0..31 and the returned VDST (element 0) holds
        // x[l - 32] in lanes 32..63.
        const auto sw = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        const uint32_t partner = lo_half ? sw[1] : sw[0];
        const float s0 = __uint_as_float(__float_as_uint(cs[r].y) ^ sin_sign);
        const float s1 = __uint_as_float(__float_as_uint(cs[r].w) ^ sin_sign);
        const uint32_t rotated = pack_bf16x2(lo_f(x) * cs[r].x + lo_f(partner) * s0,
                                             hi_f(x) * cs[r].z + hi_f(partner) * s1);
        const int pos = pos_r[r];
        out[r] = (pos >= 0 && pos < a.rope_max) ? rotated : x;
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int tt = tok[r];
        if (tt < 0) break;
        if (lh[r] < a.nq) {
            reinterpret_cast<uint32_t*>(a.q_out + (static_cast<int64_t>(tt) * a.nq + lh[r]) * D)
                [lane] = out[r];
            continue;
        }
        const int slot = slot_r[r];
        if (slot < 0 || slot >= a.max_slots) continue;
        const int64_t dst = (static_cast<int64_t>(slot) * a.nkv + (lh[r] - a.nq)) * D;
        reinterpret_cast<uint32_t*>(a.k_cache + dst)[lane] = out[r];
        reinterpret_cast<uint32_t*>(a.v_cache + dst)[lane] = v[r];
    }
}

// Any head_dim: one 256-thread workgroup per (token, head) row, the reference's layout.
__global__ __launch_bounds__(256) void qkv_prologue_generic_kernel(PrologueArgs a) {
    constexpr int kBlock = 256;
    __shared__ float warp_sums[kBlock / 32];
    __shared__ float s_total;
    extern __shared__ float row_buf[];  // hd floats: the normalised, bf16-rounded row
    const int tid = threadIdx.x;
    const int heads = a.nq + a.nkv;
    const int64_t row = blockIdx.x;
    const int t = static_cast<int>(row / heads);
    const int lh = static_cast<int>(row % heads);
    const bool is_q = lh < a.nq;
    const int hd = a.hd;
    const int64_t qkv_row = static_cast<int64_t>(a.nq + 2 * a.nkv) * hd;
    const __bf16* src = a.qkv + t * qkv_row + static_cast<int64_t>(lh) * hd;
    const __bf16* nw = is_q ? a.q_norm_w : a.k_norm_w;

    float inv_rms = 1.0f;
    if (nw != nullptr) {
        float s = 0.0f;
        if (hd % 2 == 0) {
            for (int i = tid; i < hd / 2; i += kBlock) {
                const float x0 = static_cast<float>(src[2 * i]);
                const float x1 = static_cast<float>(src[2 * i + 1]);
                s = bf16_round(s + (x0 * x0 + x1 * x1));
            }
        } else {
            for (int i = tid; i < hd; i += kBlock) {
                const float x = static_cast<float>(src[i]);
                s = bf16_round(s + x * x);
            }
        }
        s = half_tree_sum(s);  // 32-lane groups = the reference's warps
        if ((tid & 31) == 0) warp_sums[tid >> 5] = s;
        __syncthreads();
        if (tid < 32) {
            float b = tid < kBlock / 32 ? warp_sums[tid] : 0.0f;
            b = half_tree_sum(b);
            if (tid == 0) s_total = bf16_round(b);
        }
        __syncthreads();
        inv_rms = 1.0f / sqrtf(s_total / static_cast<float>(hd) + a.eps);
    }
    for (int i = tid; i < hd; i += kBlock) {
        const float x = static_cast<float>(src[i]);
        row_buf[i] = nw != nullptr ? bf16_round((x * inv_rms) * static_cast<float>(nw[i]))
                                   : x;
    }
    __syncthreads();
    const int pos = a.positions[t];
    const int half = hd / 2;
    if (pos >= 0 && pos < a.rope_max) {
        for (int p = tid; p < half; p += kBlock) {
            const float2 cs = a.rope_cache[static_cast<int64_t>(pos) * half + p];
            const float x0 = row_buf[p], x1 = row_buf[p + half];
            row_buf[p] = x0 * cs.x - x1 * cs.y;
            row_buf[p + half] = x1 * cs.x + x0 * cs.y;
        }
        __syncthreads();
    }
    __bf16* dst;
    if (is_q) {
        dst = a.q_out + (static_cast<int64_t>(t) * a.nq + lh) * hd;
    } else {
        const int slot = a.slot_mapping[t];
        if (slot < 0 || slot >= a.max_slots) return;
        const int h = lh - a.nq;
        const int64_t off = (static_cast<int64_t>(slot) * a.nkv + h) * hd;
        dst = a.k_cache + off;
        const __bf16* vsrc = a.qkv + t * qkv_row + static_cast<int64_t>(a.nq + a.nkv + h) * hd;
        for (int i = tid; i < hd; i += kBlock) a.v_cache[off + i] = vsrc[i];
    }
    for (int i = tid; i < hd; i += kBlock) dst[i] = static_cast<__bf16>(row_buf[i]);
}

}  // namespace

bool qkv_prologue_fast_supported(int head_dim) { return head_dim == 128; }

hipError_t qkv_prologue(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                        const int32_t* positions, const void* rope_cache,
                        const int32_t* slot_mapping, void* q_out, void* k_cache, void* v_cache,
                        int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                        int rope_cache_max_position, int max_slots, float eps,
                        hipStream_t stream) {
    PrologueArgs a{static_cast<const __bf16*>(qkv),
                   static_cast<const __bf16*>(q_norm_w),
                   static_cast<const __bf16*>(k_norm_w),
                   positions,
                   static_cast<const float2*>(rope_cache),
                   slot_mapping,
                   static_cast<__bf16*>(q_out),
                   static_cast<__bf16*>(k_cache),
                   static_cast<__bf16*>(v_cache),
                   num_tokens,
                   num_q_heads,
                   num_kv_heads,
                   head_dim,
                   rope_cache_max_position,
                   max_slots,
                   eps};
    const int64_t rows = static_cast<int64_t>(num_tokens) * (num_q_heads + num_kv_heads);
    // The fast path loads qkv/weights as 32-bit pairs and (cos, sin) pairs as float4.
    const bool aligned = (reinterpret_cast<uintptr_t>(qkv) % 4 == 0) &&
                         (reinterpret_cast<uintptr_t>(q_norm_w) % 4 == 0) &&
                         (reinterpret_cast<uintptr_t>(k_norm_w) % 4 == 0) &&
                         (reinterpret_cast<uintptr_t>(rope_cache) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(q_out) % 4 == 0) &&
                         (reinterpret_cast<uintptr_t>(k_cache) % 4 == 0) &&
                         (reinterpret_cast<uintptr_t>(v_cache) % 4 == 0);
    // The fast path takes both norm weights or neither (one alone goes to the generic kernel).
    const bool norm_pair = (q_norm_w == nullptr) == (k_norm_w == nullptr);
    if (qkv_prologue_fast_supported(head_dim) && aligned && norm_pair) {
        // Eight rows per wave once the grid still has a few thousand workgroups; small
        // (decode-batch) launches keep one row per wave for the shortest latency.
        constexpr int kBig = 8;
        const int64_t big_groups = (rows + kBig * kWavesPerGroup - 1) / (kBig * kWavesPerGroup);
        const int64_t small_groups = (rows + kWavesPerGroup - 1) / kWavesPerGroup;
        const bool norm = q_norm_w != nullptr;
        if (big_groups >= 2048) {
            if (norm)
                qkv_prologue_d128_kernel<kBig, true>
                    <<<static_cast<unsigned>(big_groups), 256, 0, stream>>>(a);
            else
                qkv_prologue_d128_kernel<kBig, false>
                    <<<static_cast<unsigned>(big_groups), 256, 0, stream>>>(a);
        } else if (norm) {
            qkv_prologue_d128_kernel<1, true>
                <<<static_cast<unsigned>(small_groups), 256, 0, stream>>>(a);
        } else {
            qkv_prologue_d128_kernel<1, false>
                <<<static_cast<unsigned>(small_groups), 256, 0, stream>>>(a);
        }
    } else {
        qkv_prologue_generic_kernel<<<static_cast<unsigned>(rows), 256,
                                      static_cast<size_t>(head_dim) * sizeof(float), stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace ccinfer::hipk
