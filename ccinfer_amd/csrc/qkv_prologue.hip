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
// head_dim 128 (the fast path): a wavefront takes up to eight consecutive (token, head) rows
// of one section of the packed QKV row and holds each as lane pairs: lane l holds elements 2l and 2l+1 -- exactly
// the pair thread l of the reference kernel sums, so lanes 0..31 and 32..63 are the
// reference's two warps and the same trees apply. The RoPE partner of element j is j + 64,
// held by lane l ^ 32, and is fetched with v_permlane32_swap. V rows are copied through.
// Other head dims: one workgroup of 256 threads per row, laid out as the reference kernel.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

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
    // A swap leaves the receiving lanes' own values in the other returned register (VDST
    // keeps its even rows / low half), so each step adds the two results and the input
    // register is not needed afterwards.
    const float v = bf16_round(x0 * x0 + x1 * x1);
    const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                      false, false);
    float u = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);  // lanes 0..15: v[l] + v[l+16]
    u += dpp_f<0x108>(u);  // row_shl:8
    u += dpp_f<0x104>(u);  // row_shl:4
    u += dpp_f<0x102>(u);  // row_shl:2
    u += dpp_f<0x101>(u);  // row_shl:1 -> lane 0: warp 0's sum, lane 32: warp 1's
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(u), __float_as_uint(u),
                                                      false, false);
    return __uint_as_float(s32[0]) + __uint_as_float(s32[1]);  // lane 0: warp 0 + warp 1
}

// Raw buffer descriptor over `base` (dword 3: 32-bit data format, the gfx9-family raw-buffer
// setting). Loads past `num_records` bytes (lane offset + immediate) return 0. Descriptors
// are built once per wavefront on the scalar unit; a lane's address is then its 32-bit byte
// offset plus an immediate, with no per-row address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                            uint32_t num_records) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                             static_cast<int>(num_records), 0x00020000);
}

// One wavefront = up to kRowsPerWave (8, or 2 for small launches) consecutive rows of one section (q heads, k heads or v heads)
// of one token's packed QKV row; each section is split into groups of that size. kNorm: both
// norm weights given (else neither). A v wavefront copies its rows into the cache. A q or
// k wavefront: (1) issues every load (rows past the section's end read as 0), the token's
// (cos, sin) pairs and the weight row, fenced from the math; (2) sums of squares, the eight
// totals gathered into lanes 0..kRowsPerWave-1 of one register so that the correctly rounded sqrt and
// division run once; (3) normalise and rotate; (4) stores the section's rows.
template <int kRowsPerWave, bool kNorm>
__global__ __launch_bounds__(256) void qkv_prologue_d128_kernel(PrologueArgs a) {
    constexpr int D = 128;
    constexpr int kRowBytes = D * 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gq = (a.nq + kRowsPerWave - 1) / kRowsPerWave;
    const int gkv = (a.nkv + kRowsPerWave - 1) / kRowsPerWave;
    const int groups = gq + 2 * gkv;
    const int wave_id = blockIdx.x * kWavesPerGroup + wave;
    if (wave_id >= a.T * groups) return;  // whole wavefronts only; no barriers below
    const int t = wave_id / groups;
    const int g = wave_id - t * groups;
    // section 0: q heads, 1: k heads, 2: v heads
    const int section = g < gq ? 0 : (g < gq + gkv ? 1 : 2);
    const int h0 = (section == 0 ? g : (section == 1 ? g - gq : g - gq - gkv)) * kRowsPerWave;
    const int sec_rows = section == 0 ? a.nq : a.nkv;
    const int sec_start = section == 0 ? 0 : (section == 1 ? a.nq : a.nq + a.nkv);
    const int n = min(kRowsPerWave, sec_rows - h0);  // rows of this wavefront
    const int lane_off = lane * 4;                   // byte offset of the lane's pair in a row
    const int row_all = a.nq + 2 * a.nkv;

    const auto src = make_rsrc(a.qkv + (static_cast<int64_t>(t) * row_all + sec_start + h0) * D,
                               static_cast<uint32_t>(n) * kRowBytes);
    uint32_t w[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
        w[r] = __builtin_amdgcn_raw_buffer_load_b32(src, lane_off + r * kRowBytes, 0, 0);

    const int slot = a.slot_mapping[t];
    const bool slot_ok = slot >= 0 && slot < a.max_slots;
    const int64_t kv_row = (static_cast<int64_t>(slot) * a.nkv + h0) * D;

    if (section == 2) {  // v rows: copy into the cache
        if (!slot_ok) return;
        const auto dst = make_rsrc(a.v_cache + kv_row, static_cast<uint32_t>(n) * kRowBytes);
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r)  // rows past n fall outside the descriptor
            __builtin_amdgcn_raw_buffer_store_b32(w[r], dst, lane_off + r * kRowBytes, 0, 0);
        return;
    }

    const bool lo_half = lane < 32;
    // lo element of a pair: x0 c - x1 s, so lanes 0..31 negate the partner (both halves)
    const uint32_t partner_sign = lo_half ? 0x80008000u : 0u;
    const int pos = a.positions[t];
    const bool rotate = pos >= 0 && pos < a.rope_max;
    const float4 cs = __builtin_bit_cast(
        float4, __builtin_amdgcn_raw_buffer_load_b128(
                    make_rsrc(a.rope_cache + static_cast<int64_t>(rotate ? pos : 0) * (D / 2),
                              D * 4),
                    (lane & 31) * 16, 0, 0));  // pairs 2 * (lane & 31) and +1
    uint32_t nw = 0;
    if constexpr (kNorm)
        nw = __builtin_amdgcn_raw_buffer_load_b32(
            make_rsrc(section == 0 ? a.q_norm_w : a.k_norm_w, kRowBytes), lane_off, 0, 0);
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any math below
    const float nw0 = lo_f(nw), nw1 = hi_f(nw);
    // Rows keep x where the position is outside the table. The select runs as a bit select
    // on a mask the compiler cannot see is uniform (a vector copy it does not look
    // through); a select on a uniform condition would become a branch, with the (cos, sin)
    // load moved into it and waited for late.
    uint32_t rot_mask;
    asm("v_mov_b32 %0, %1" : "=v"(rot_mask) : "s"(rotate ? ~0u : 0u));

    float inv_rms_lanes = 0.f;  // lane r: 1 / rms of row h0 + r
    if constexpr (kNorm) {
        float totals = 0.f;
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
            const float sum = row_sum_squares(lo_f(w[r]), hi_f(w[r]));
            const float sum0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), 0));
            totals = lane == r ? sum0 : totals;
        }
        inv_rms_lanes = 1.0f / sqrtf(bf16_round(totals) / static_cast<float>(D) + a.eps);
    }

    uint32_t out[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        uint32_t x = w[r];
        if constexpr (kNorm) {
            const float inv = __int_as_float(
                __builtin_amdgcn_readlane(__float_as_int(inv_rms_lanes), r));
            x = pack_bf16x2((lo_f(x) * inv) * nw0, (hi_f(x) * inv) * nw1);
        }
        // Partner elements 2l+64, 2l+65 (lane l < 32) or 2l-64, 2l-63 (lane l >= 32).
        // v_permlane32_swap moves VSRC's lanes 0..31 into VDST's lanes 32..63 and VDST's
        // lanes 32..63 into VSRC's lanes 0..31; with both operands x, the returned VSRC
        // (element 1) holds x[l + 32] in lanes 0..31 and the returned VDST (element 0)
        // holds x[l - 32] in lanes 32..63, while the lane's own x survives in the other
        // register (VDST keeps lanes 0..31, VSRC keeps lanes 32..63).
        const auto sw = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        const uint32_t partner = (lo_half ? sw[1] : sw[0]) ^ partner_sign;
        x = lo_half ? sw[0] : sw[1];
        const uint32_t rotated = pack_bf16x2(lo_f(x) * cs.x + lo_f(partner) * cs.y,
                                             hi_f(x) * cs.z + hi_f(partner) * cs.w);
        out[r] = x ^ ((x ^ rotated) & rot_mask);
    }

    // A skipped slot gets an empty descriptor (its stores are dropped) rather than an early
    // return, which would let the compiler move the math and the (cos, sin) load behind it.
    const uint32_t dst_bytes = section == 1 && !slot_ok ? 0u : static_cast<uint32_t>(n) * kRowBytes;
    // both candidate addresses are computed and one selected: no branch between the loads
    // and the stores, which would again invite the compiler to sink the loads
    __bf16* const q_row = a.q_out + (static_cast<int64_t>(t) * a.nq + h0) * D;
    __bf16* const k_row = a.k_cache + kv_row;
    const auto dst = make_rsrc(section == 0 ? q_row : k_row, dst_bytes);
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)  // rows past n fall outside the descriptor
        __builtin_amdgcn_raw_buffer_store_b32(out[r], dst, lane_off + r * kRowBytes, 0, 0);
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
        auto launch = [&](auto rows_tag) {
            constexpr int kRows = decltype(rows_tag)::value;
            const int64_t groups = (num_q_heads + kRows - 1) / kRows +
                                   2 * ((num_kv_heads + kRows - 1) / kRows);
            const int64_t waves = static_cast<int64_t>(num_tokens) * groups;
            const unsigned grid =
                static_cast<unsigned>((waves + kWavesPerGroup - 1) / kWavesPerGroup);
            if (q_norm_w != nullptr)
                qkv_prologue_d128_kernel<kRows, true><<<grid, 256, 0, stream>>>(a);
            else
                qkv_prologue_d128_kernel<kRows, false><<<grid, 256, 0, stream>>>(a);
        };
        // Eight rows per wavefront keep enough loads in flight to stream HBM once there are
        // thousands of wavefronts; decode-size launches take two rows per wavefront, which
        // spreads them over more CUs and shortens each wavefront's dependent chain.
        if (static_cast<int64_t>(num_tokens) * (num_q_heads + 2 * num_kv_heads) >= 16384 * 8)
            launch(std::integral_constant<int, 8>{});
        else
            launch(std::integral_constant<int, 2>{});
    } else {
        qkv_prologue_generic_kernel<<<static_cast<unsigned>(rows), 256,
                                      static_cast<size_t>(head_dim) * sizeof(float), stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace ccinfer::hipk
