// Device-side building blocks of the split-KV decode (decode_attn.hip), shared with the
// prefill tile launch, which runs the single-token requests of a small prefill batch as
// extra workgroups of its own grid (prefill_attn.hip). Everything here is inline device
// code in namespace dcore; the kernels and host code that use it stay in those files.
#pragma once

#include <type_traits>

#include "attn_common.hpp"

namespace ccinfer::hipk::dcore {

constexpr int kBlock = 16;        // tokens per KV block (the reference's kKVBlockSize)
constexpr int kChunk = 32;        // tokens per PV MFMA
constexpr int kWavesPerGroup = 4;
constexpr int kMaxSplitTokens = 2048;  // 128 blocks: two table entries per lane

struct ItemArgs {
    int num_items;
    const int32_t* item_count;
    const int32_t* item_req;
    const int32_t* qsl;
    float eps;
    int zero_invalid;
    // Optional new token per request (bf16 [B][Hkv][dr]), written to the cache slot of the
    // request's last position before it is read (nullptr: none).
    const __bf16* new_k;
    const __bf16* new_v;
    int max_slots;
    // Shared-prefix decode (decode_attention_shared): the first position each item attends
    // to here (a multiple of kChunk; nullptr: 0), and the number of partials of the item's
    // rows that the shared-prefix kernel wrote for positions before it (nullptr: none). Such
    // rows always go through the merge, which adds those partials.
    const int32_t* begin;
    const int32_t* sh_splits;
    // >= 0: item i is request i of a prefill batch of this many query rows, attended only
    // when it is a single-token request (single_token_request); -1: items as listed above.
    int singles_total = -1;
};

__device__ __forceinline__ int item_first(const ItemArgs& it, int item) {
    return it.begin != nullptr ? it.begin[item] : 0;
}
__device__ __forceinline__ int item_shared(const ItemArgs& it, int item) {
    return it.sh_splits != nullptr ? it.sh_splits[item] : 0;
}

// Per (item, q_head) row: how many splits its partials span and where they start. Written
// by split 0 of the row's kv_head group on every launch; the merge reads it instead of
// re-deriving the plan (ns <= 1: nothing to merge).
struct MergeDesc {
    int64_t base;
    int64_t ns;
};

template <int D>
struct DecodeShape {
    static constexpr int kSteps = D / 32;  // QK MFMA k-steps per 16-token block
    static constexpr int kNV = D / 16;     // V dims per lane per token == number of PV MFMAs
    static constexpr int kVWords = kNV / 2;
};

// Resolves an item to (request, query row). Returns false for items past the live count.
__device__ __forceinline__ bool resolve_item(const ItemArgs& it, int item, int* req, int* qrow) {
    if (item >= it.num_items) return false;
    if (it.item_count != nullptr && item >= *it.item_count) return false;
    const int r = it.item_req != nullptr ? it.item_req[item] : item;
    *req = r;
    *qrow = it.qsl != nullptr ? it.qsl[r] : r;
    return true;
}

// Number of context positions to visit for a request, or -1 when the output must be zero
// (decode mode) / left untouched (prefill mode).
// The wavefront whose split holds position ctx - 1 of request req writes that position's K
// and V rows for its cache head from the new token of the request (block id checked against
// the cache's slot count), and waits for the stores before any load of the split. No other
// wavefront reads that slot (one split holds each position; other requests do not see a
// request's newest position).
template <bool kPad>
__device__ __forceinline__ void write_new_token(__bf16* k_cache, __bf16* v_cache,
                                                const ItemArgs& items,
                                                const int32_t* __restrict__ req_blocks, int req,
                                                int ctx, int hkv_c, int kvh, int ds, int lane) {
    const int pos = ctx - 1;
    const int pb = req_blocks[pos / kBlock];
    const int64_t slot = static_cast<int64_t>(pb) * kBlock + pos % kBlock;
    if (pb >= 0 && slot < items.max_slots) {
        // Stores through the same cache pointers the split's loads use, so the compiler
        // keeps the loads after them.
        uint32_t* kd = reinterpret_cast<uint32_t*>(k_cache + (slot * hkv_c + kvh) * ds);
        uint32_t* vd = reinterpret_cast<uint32_t*>(v_cache + (slot * hkv_c + kvh) * ds);
        const int64_t src = (static_cast<int64_t>(req) * hkv_c + kvh) * ds;
        const uint32_t* ks = reinterpret_cast<const uint32_t*>(items.new_k + src);
        const uint32_t* vs = reinterpret_cast<const uint32_t*>(items.new_v + src);
        for (int x = lane; x < ds / 2; x += 64) {
            kd[x] = ks[x];
            vd[x] = vs[x];
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the rows are in L2 before any load
    asm volatile("" ::: "memory");
}

// Whether request b of a prefill batch (total_tokens query rows) is a single-token
// request: the rows the prefill planner hands to the decode kernels instead of a tile
// (prefill_plan_kernel applies the same test).
__device__ __forceinline__ bool single_token_request(const int32_t* __restrict__ qsl,
                                                     const int32_t* __restrict__ context_lens,
                                                     int b, int total_tokens) {
    const int qb = qsl[b];
    const int qe_raw = qsl[b + 1];
    const int qlen = qe_raw - qb;
    const int rows = (qe_raw < total_tokens ? qe_raw : total_tokens) - (qb > 0 ? qb : 0);
    return qlen == 1 && context_lens[b] - qlen >= 0 && qb >= 0 && rows > 0;
}

__device__ __forceinline__ int effective_ctx(int ctx, int mbpr, int zero_invalid) {
    if (ctx <= 0) return -1;
    const int cap = mbpr * kBlock;
    if (zero_invalid) {
        // decode_attn.cu:406-412: more blocks than the table row holds -> zeros.
        return (ctx + kBlock - 1) / kBlock > mbpr ? -1 : ctx;
    }
    // Prefill semantics: positions past the table row are invalid, not an error.
    return ctx < cap ? ctx : cap;
}

// K/V bytes are read once per (request, kv_head) and never again in the launch: streaming
// (nontemporal) loads keep them from displacing reused lines in the caches. Measured on the
// box: configs[1] 119 -> 108 us, configs[4] 715 -> 658 us.
template <typename T>
__device__ __forceinline__ T nt_load(const T* p) {
    return __builtin_nontemporal_load(p);
}

// K/V chunk loads: nontemporal (each byte is read once per launch) unless kTL, where the same
// lines are read again soon (padded rows re-read a piece of their own row; virtual kv heads
// read their cache head's blocks once per virtual head) and should stay in L2.
template <bool kTL, typename T>
__device__ __forceinline__ T kv_load(const T* p) {
    if constexpr (kTL)
        return *p;
    else
        return __builtin_nontemporal_load(p);
}

// kU: the alignment of cache rows that are not 16-byte aligned (a cache pointer offset by a
// number of elements that is not a multiple of 8; the reference kernels read bf16 scalars,
// so they accept one): 4 or 2 bytes, 0 for aligned rows. Each piece is then assembled from
// 4-byte or 2-byte loads -- neighbouring lanes read neighbouring elements, so a wavefront
// still touches whole lines -- and the rest of the kernel is unchanged. (The choice is per
// kernel: a branch per piece keeps both paths' registers live.) (Two
// aligned 16-byte loads shifted into place, as the prefill staging does, hold twice the
// registers per piece in flight: 48-1198 spilled VGPRs here, 7.6x instead of 1.7x. The
// whole dwords around a 2-byte-aligned piece, one more than the piece, shifted with
// v_alignbyte: 8 spilled VGPRs at head dim 128 and 37 at 96 / 192, where the 2-byte loads,
// which fill both halves of one register each, spill none.)
template <bool kTL, int kU, typename T>
__device__ __forceinline__ T kv_piece(const __bf16* p) {
    constexpr int kWords = std::is_same_v<T, u32x3> ? 3 : sizeof(T) / 4;
    if constexpr (kU == 0 && std::is_same_v<T, u32x3>) {
        return kv_load<kTL>(reinterpret_cast<const u32x3_a4*>(p));
    } else if constexpr (kU == 0) {
        return kv_load<kTL>(reinterpret_cast<const T*>(p));
    } else if constexpr (kU == 4) {
        const uint32_t* e = reinterpret_cast<const uint32_t*>(p);
        T w;
#pragma unroll
        for (int i = 0; i < kWords; ++i) w[i] = e[i];
        return w;
    } else {
        const uint16_t* e = reinterpret_cast<const uint16_t*>(p);
        T w;
#pragma unroll
        for (int i = 0; i < kWords; ++i)
            w[i] = static_cast<uint32_t>(e[2 * i]) | (static_cast<uint32_t>(e[2 * i + 1]) << 16);
        return w;
    }
}

// KS: the K steps a row needs (fewer than D / 32 when the padded dims leave whole steps
// empty; those steps are neither loaded nor multiplied).
template <int D, int KS = DecodeShape<D>::kSteps>
struct ChunkRegs {
    u32x4 k[2][KS];
    uint32_t v[8][DecodeShape<D>::kVWords];
};

// kPad: the cache rows hold dr < D dims (dr a multiple of D/16); the kernel runs at the
// MFMA size D with dims [dr, D) zero. At D = 128 (head dims 80-120) the lanes of missing
// dims load nothing (exec-masked loads): the L2 re-reads they would make cost 4-11 % of
// the batch (d=80 151.5 -> 139.7 us, d=120 191.4 -> 183.4 us at 64 x 4096). At D = 64 and
// 256 such loads read a valid piece of the row instead and are replaced by zeros: masking
// measured 11-23 % slower at d=32, and spills 137 VGPRs at D = 256.
template <int D, bool kPad = false, bool kTL = false, int KS = DecodeShape<D>::kSteps,
          int kU = 0>
__device__ __forceinline__ void load_chunk(ChunkRegs<D, KS>& c,
                                           const __bf16* __restrict__ k_cache,
                                           const __bf16* __restrict__ v_cache, int pb0, int pb1,
                                           int kv_head, int hkv, int lane, int dr = D) {
    constexpr int S = KS;
    constexpr int NV = DecodeShape<D>::kNV;
    const int rs = kPad ? dr : D;  // row stride (elements)
    constexpr bool kMasked = kPad && D == 128;
    const int i = lane & 15;
    const int g = lane >> 4;
    const int pbs[2] = {pb0 < 0 ? 0 : pb0, pb1 < 0 ? 0 : pb1};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        const __bf16* row =
            k_cache + ((static_cast<int64_t>(pbs[kb]) * kBlock + i) * hkv + kv_head) * rs;
#pragma unroll
        for (int kk = 0; kk < S; ++kk) {
            const int dim0 = (kk * 4 + g) * 8;
            const bool ok = !kPad || dim0 < dr;
            if constexpr (kMasked) {
                c.k[kb][kk] = u32x4{0, 0, 0, 0};
                if (ok) c.k[kb][kk] = kv_piece<kTL, kU, u32x4>(row + dim0);
            } else {
                c.k[kb][kk] = kv_piece<kTL, kU, u32x4>(row + (ok ? dim0 : 0));
                if (!ok) c.k[kb][kk] = u32x4{0, 0, 0, 0};
            }
        }
    }
    const bool vok = !kPad || i * NV < dr;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int kb = e >> 2;
        const int off = g * 4 + (e & 3);
        const __bf16* row =
            v_cache + ((static_cast<int64_t>(pbs[kb]) * kBlock + off) * hkv + kv_head) * rs +
            (vok ? i * NV : 0);
        if constexpr (NV == 8) {
            u32x4 w = u32x4{0, 0, 0, 0};
            if (!kMasked || vok) w = kv_piece<kTL, kU, u32x4>(row);
#pragma unroll
            for (int x = 0; x < 4; ++x) c.v[e][x] = vok ? w[x] : 0u;
        } else if constexpr (NV == 6) {  // D = 96: a 12-byte piece per lane
            const u32x3 w = kv_piece<kTL, kU, u32x3>(row);
#pragma unroll
            for (int x = 0; x < 3; ++x) c.v[e][x] = w[x];
        } else if constexpr (NV == 2) {  // D = 32: a 4-byte piece per lane
            c.v[e][0] = kv_piece<kTL, kU, u32x1>(row)[0];
        } else if constexpr (NV == 12) {  // D = 192: a 24-byte piece per lane
            const u32x4 w0 = kv_piece<kTL, kU, u32x4>(row);
            const u32x2 w1 = kv_piece<kTL, kU, u32x2>(row + 8);
#pragma unroll
            for (int x = 0; x < 4; ++x) c.v[e][x] = w0[x];
            c.v[e][4] = w1[0];
            c.v[e][5] = w1[1];
        } else if constexpr (NV == 4) {
            u32x2 w = u32x2{0, 0};
            if (!kMasked || vok) w = kv_piece<kTL, kU, u32x2>(row);
            c.v[e][0] = vok ? w[0] : 0u;
            c.v[e][1] = vok ? w[1] : 0u;
        } else {
            const u32x4 w0 = kv_piece<kTL, kU, u32x4>(row);
            const u32x4 w1 = kv_piece<kTL, kU, u32x4>(row + 8);
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                c.v[e][x] = vok ? w0[x] : 0u;
                c.v[e][4 + x] = vok ? w1[x] : 0u;
            }
        }
    }
}

// fp8 cache: one byte per element plus the row scales of the chunk's tokens T(g, e) =
// 16 * (e / 4) + 4 * g + e % 4 (tokens 4g..4g+3 of each block: 16 contiguous bytes of the
// block's scale line). K is read 16 bytes per lane: lane (row i, group g) takes bytes
// 64 k2 + 16 g .. +16 of its row, i.e. dims 64 (kk / 2) + 16 g + 8 (kk % 2) .. +8 for k-step
// kk; the dot product only needs Q's operand to use the same dim order (it does, F8 only),
// and the row is covered by half as many, twice as wide loads as the bf16 order would give.
// V keeps the bf16 layout (NV bytes per token piece; a 16-lane group reads whole rows) and
// is read nontemporally; K stays cached (measured: configs[1] batch 73 -> 62 us).
template <int D>
struct ChunkRegsF8 {
    u32x2 k[2][DecodeShape<D>::kSteps];
    uint32_t v[8][(DecodeShape<D>::kNV + 3) / 4];
    u32x4 ks[2];
    u32x4 vs[2];
};

template <int D, bool kTL = false>
__device__ __forceinline__ void load_chunk(ChunkRegsF8<D>& c, const uint8_t* __restrict__ k_cache,
                                           const uint8_t* __restrict__ v_cache,
                                           const float* __restrict__ k_scale,
                                           const float* __restrict__ v_scale, int pb0, int pb1,
                                           int kv_head, int hkv, int lane) {
    constexpr int S = DecodeShape<D>::kSteps;
    constexpr int NV = DecodeShape<D>::kNV;
    const int i = lane & 15;
    const int g = lane >> 4;
    const int pbs[2] = {pb0 < 0 ? 0 : pb0, pb1 < 0 ? 0 : pb1};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        const uint8_t* row =
            k_cache + ((static_cast<int64_t>(pbs[kb]) * kBlock + i) * hkv + kv_head) * D;
#pragma unroll
        for (int k2 = 0; k2 < S / 2; ++k2) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(row + k2 * 64 + g * 16);
            c.k[kb][2 * k2] = u32x2{w[0], w[1]};
            c.k[kb][2 * k2 + 1] = u32x2{w[2], w[3]};
        }
        const int64_t sl = (static_cast<int64_t>(pbs[kb]) * hkv + kv_head) * kBlock + 4 * g;
        c.ks[kb] = *reinterpret_cast<const u32x4*>(k_scale + sl);
        c.vs[kb] = *reinterpret_cast<const u32x4*>(v_scale + sl);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int kb = e >> 2;
        const int off = g * 4 + (e & 3);
        const uint8_t* row =
            v_cache + ((static_cast<int64_t>(pbs[kb]) * kBlock + off) * hkv + kv_head) * D +
            i * NV;
        if constexpr (NV == 4) {
            c.v[e][0] = kv_load<kTL>(reinterpret_cast<const uint32_t*>(row));
        } else if constexpr (NV == 8) {
            const u32x2 w = kv_load<kTL>(reinterpret_cast<const u32x2*>(row));
            c.v[e][0] = w[0];
            c.v[e][1] = w[1];
        } else {
            const u32x4 w = kv_load<kTL>(reinterpret_cast<const u32x4*>(row));
#pragma unroll
            for (int x = 0; x < 4; ++x) c.v[e][x] = w[x];
        }
    }
}

// Online-softmax state of one wavefront: lane (head j, grp g) holds O[j][NV*(4g+r)+n] in
// acc[n][r], the running max m (base-2 domain, per head, replicated over the 4 grp lanes)
// and a per-lane partial sum l.
template <int D>
struct SoftmaxState {
    f32x4 acc[DecodeShape<D>::kNV];
    float m;
    float l;
};

// kScaled: K/V came from the fp8 cache; ks[e] / vs[e] are the row scales of token T(g, e),
// applied to its score (K) and to its probability in the PV product (V).
template <int D, bool kScaled = false, int KS = DecodeShape<D>::kSteps>
__device__ __forceinline__ void consume_chunk(SoftmaxState<D>& st, ChunkRegs<D, KS>& c,
                                              const bf16x8 (&qop)[DecodeShape<D>::kSteps],
                                              int cb, int end, int pb0, int pb1,
                                              float scale_log2, int g,
                                              const float* ks = nullptr,
                                              const float* vs = nullptr) {
    constexpr int S = KS;
    constexpr int NV = DecodeShape<D>::kNV;
    float sc[8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < S; ++kk)
            s4 = mfma16x16x32(__builtin_bit_cast(bf16x8, c.k[kb][kk]), qop[kk], s4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (kScaled)
                sc[kb * 4 + r] = s4[r] * (scale_log2 * ks[kb * 4 + r]);
            else
                sc[kb * 4 + r] = s4[r] * scale_log2;
        }
    }
    // Masking (context end, negative block ids) is branch-free: the selects are cheap in
    // this memory-bound loop, and a wave-uniform branch around them would merge every V
    // register through a phi (which the gfx950 backend of this toolchain has been seen to
    // miscompile). Masked V rows are zeroed so NaN/Inf garbage in unwritten slots cannot
    // reach the PV product.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int kb = e >> 2;
        const int pos = cb + kb * kBlock + g * 4 + (e & 3);
        const bool ok = pos < end && (kb == 0 ? pb0 : pb1) >= 0;
        sc[e] = ok ? sc[e] : kNegInf;
#pragma unroll
        for (int x = 0; x < DecodeShape<D>::kVWords; ++x) c.v[e][x] = ok ? c.v[e][x] : 0u;
    }
    float mloc = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                       fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
    mloc = wave_max_xor16_32(mloc);
    const float m_new = fmaxf(st.m, mloc);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_use);
    float p[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        p[e] = __builtin_amdgcn_exp2f(sc[e] - m_use);
        psum += p[e];
    }
    st.l = st.l * alpha + psum;
    st.m = m_new;
    u32x4 pw;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        if constexpr (kScaled)
            pw[x] = pack_bf16x2(p[2 * x] * vs[2 * x], p[2 * x + 1] * vs[2 * x + 1]);
        else
            pw[x] = pack_bf16x2(p[2 * x], p[2 * x + 1]);
    }
    const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        u32x4 vw;
#pragma unroll
        for (int x = 0; x < 4; ++x)
            vw[x] = pick_halves(c.v[2 * x][n >> 1], c.v[2 * x + 1][n >> 1], n & 1);
        st.acc[n] = st.acc[n] * alpha;
        st.acc[n] = mfma16x16x32(__builtin_bit_cast(bf16x8, vw), pop, st.acc[n]);
    }
}

template <int D>
__device__ __forceinline__ void consume_chunk(SoftmaxState<D>& st, ChunkRegsF8<D>& r,
                                              const bf16x8 (&qop)[DecodeShape<D>::kSteps],
                                              int cb, int end, int pb0, int pb1,
                                              float scale_log2, int g) {
    constexpr int S = DecodeShape<D>::kSteps;
    ChunkRegs<D> c;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int kk = 0; kk < S; ++kk)
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                c.k[kb][kk][2 * w] = e4m3x2_to_bf16x2<false>(r.k[kb][kk][w]);
                c.k[kb][kk][2 * w + 1] = e4m3x2_to_bf16x2<true>(r.k[kb][kk][w]);
            }
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int x = 0; x < DecodeShape<D>::kVWords; x += 2) {
            c.v[e][x] = e4m3x2_to_bf16x2<false>(r.v[e][x >> 1]);
            c.v[e][x + 1] = e4m3x2_to_bf16x2<true>(r.v[e][x >> 1]);
        }
    float ks[8], vs[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        ks[e] = __uint_as_float(r.ks[e >> 2][e & 3]);
        vs[e] = __uint_as_float(r.vs[e >> 2][e & 3]);
    }
    consume_chunk<D, true>(st, c, qop, cb, end, pb0, pb1, scale_log2, g, ks, vs);
}

// The columns of a row the merges give lane `lane`: kPer consecutive ones, lanes past the
// row (D = 96: lanes 48-63) re-reading its last column and storing nothing.
template <int D>
struct MergeCols {
    static constexpr int kPer = (D + 63) / 64;
    static __device__ __forceinline__ int col(int lane, int x) {
        if constexpr (D % 64 == 0)
            return lane * kPer + x;
        else
            return min(lane * kPer + x, D - 1);
    }
};

// Per-split inputs: the split's block ids, one per lane (two registers cover 128 blocks),
// and the Q^T operand: lane (head j, grp g) holds dims (kk*4+g)*8 .. +8 of head j (fp8:
// the permuted order of the fp8 K loads).
template <int D>
struct SplitInputs {
    int bt_lo;
    int bt_hi;
    bf16x8 qop[DecodeShape<D>::kSteps];
};

// Loads the inputs of a split starting at position `begin` whose table entries end at
// position tbl_end (no more than 2048 positions).
template <int D, bool F8, bool kPad = false>
__device__ __forceinline__ void load_split_inputs(const __bf16* __restrict__ q,
                                                  const int32_t* __restrict__ req_blocks,
                                                  int mbpr, int qrow, int hq, int h, int G,
                                                  int begin, int tbl_end, int lane,
                                                  SplitInputs<D>& in, int dr = D) {
    constexpr int S = DecodeShape<D>::kSteps;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int lb0 = begin / kBlock;
    const int nblk = (tbl_end - begin + kBlock - 1) / kBlock;
    in.bt_lo = (lane < nblk && lb0 + lane < mbpr) ? req_blocks[lb0 + lane] : -1;
    in.bt_hi = (lane + 64 < nblk && lb0 + lane + 64 < mbpr) ? req_blocks[lb0 + lane + 64] : -1;
    const bool live = j < G;
    const __bf16* qv =
        q + (static_cast<int64_t>(qrow) * hq + h * G + (live ? j : 0)) * (kPad ? dr : D);
#pragma unroll
    for (int kk = 0; kk < S; ++kk) {
        const int dim0 = F8 ? 64 * (kk >> 1) + 16 * g + 8 * (kk & 1) : (kk * 4 + g) * 8;
        const bool ok = !kPad || dim0 < dr;
        u32x4 w = load16(qv + (ok ? dim0 : 0));
        if (!live || !ok) w = u32x4{0, 0, 0, 0};
        in.qop[kk] = __builtin_bit_cast(bf16x8, w);
    }
}

// Attention of the G query heads of kv_head h over context positions [begin, end) (at most
// 2048) with the split's inputs: the online-softmax state of one wavefront.
// KS: K steps per row (bf16); NBUF: chunks in flight (two, or three, which the kernels
// have the registers for at no head dim today: three padded chunks at head dim 80 / 192
// spill 521 / 619 VGPRs).
template <int D, bool F8, bool kPad = false, bool kTL = false,
          int KS = DecodeShape<D>::kSteps, int NBUF = 2, int kU = 0>
__device__ __forceinline__ void run_split(
    const std::conditional_t<F8, uint8_t, __bf16>* __restrict__ k_cache,
    const std::conditional_t<F8, uint8_t, __bf16>* __restrict__ v_cache,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale,
    const SplitInputs<D>& in, int hkv, int h, int begin, int end, float scale_log2, int lane,
    SoftmaxState<D>& st, int dr = D) {
    static_assert(NBUF == 2 || NBUF == 3, "two or three chunks in flight");
    static_assert(!F8 || (KS == DecodeShape<D>::kSteps && NBUF == 2 && kU == 0),
                  "fp8: the full chunk, 16-byte aligned");
    constexpr int NV = DecodeShape<D>::kNV;
    using Regs = std::conditional_t<F8, ChunkRegsF8<D>, ChunkRegs<D, KS>>;
    const int g = lane >> 4;
    const int nblk = (end - begin + kBlock - 1) / kBlock;
    auto block_id = [&](int jb) -> int {  // jb: wave-uniform block index within the split
        return __builtin_amdgcn_readlane(jb < 64 ? in.bt_lo : in.bt_hi, jb & 63);
    };
#pragma unroll
    for (int n = 0; n < NV; ++n) st.acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = kNegInf;
    st.l = 0.f;

    const int nchunks = (end - begin + kChunk - 1) / kChunk;
    // Block ids of chunk c (clamped to the last chunk so prefetches are unconditional).
    auto chunk_blocks = [&](int c, int* p0, int* p1) {
        c = c < nchunks ? c : nchunks - 1;
        *p0 = block_id(2 * c);
        *p1 = (2 * c + 1 < nblk) ? block_id(2 * c + 1) : -1;
    };
    auto load = [&](Regs& r, int p0, int p1) {
        if constexpr (F8)
            load_chunk<D, kTL>(r, k_cache, v_cache, k_scale, v_scale, p0, p1, h, hkv, lane);
        else
            load_chunk<D, kPad, kTL, KS, kU>(r, k_cache, v_cache, p0, p1, h, hkv, lane, dr);
    };
    auto consume = [&](Regs& r, int c, int p0, int p1) {
        if constexpr (F8)
            consume_chunk<D>(st, r, in.qop, begin + c * kChunk, end, p0, p1, scale_log2, g);
        else
            consume_chunk<D, false, KS>(st, r, in.qop, begin + c * kChunk, end, p0, p1,
                                        scale_log2, g);
    };
    Regs ra, rb;
    int a0, a1, b0, b1;
    chunk_blocks(0, &a0, &a1);
    load(ra, a0, a1);
    if constexpr (NBUF == 2) {
        for (int c = 0; c < nchunks; c += 2) {
            chunk_blocks(c + 1, &b0, &b1);
            load(rb, b0, b1);
            consume(ra, c, a0, a1);
            if (c + 1 >= nchunks) break;
            chunk_blocks(c + 2, &a0, &a1);
            load(ra, a0, a1);
            consume(rb, c + 1, b0, b1);
        }
    } else {
        Regs rc;
        int c0, c1;
        chunk_blocks(1, &b0, &b1);
        load(rb, b0, b1);
        for (int c = 0; c < nchunks; c += 3) {
            chunk_blocks(c + 2, &c0, &c1);
            load(rc, c0, c1);
            consume(ra, c, a0, a1);
            if (c + 1 >= nchunks) break;
            chunk_blocks(c + 3, &a0, &a1);
            load(ra, a0, a1);
            consume(rb, c + 1, b0, b1);
            if (c + 2 >= nchunks) break;
            chunk_blocks(c + 4, &b0, &b1);
            load(rb, b0, b1);
            consume(rc, c + 2, c0, c1);
        }
    }
}


// Query groups larger than one MFMA N-tile run as virtual kv heads: the smallest r with
// G % r == 0 and G / r <= 16 (host code).
inline int decode_head_rep(int G) {
    int r = (G + 15) / 16;
    while (G % r != 0) ++r;
    return r;
}

// Single-launch decode for batches with few (item, kv_head) groups: one workgroup of W
// wavefronts per group, wavefront w attending over the w-th of W equal parts of the
// context; the parts are merged through LDS with the same log-sum-exp weighting as the
// merge kernel's, so no second kernel and no workspace. (For many groups the flat split
// plan spreads ragged contexts better.)
template <int D>
struct GroupShape {
    static constexpr int kWaves = D <= 128 ? 8 : 4;  // two wavefronts per SIMD at <= 256 VGPRs
    static constexpr int kMaxG = 16;                 // LDS: kWaves * 16 * D floats = 64 KiB
};

// The body of one group's workgroup (group = item * hkv + virtual kv head). LDS: part(w)
// gives wavefront w's kMaxG x D floats of partial rows, lds_m / lds_l kWaves x kMaxG floats
// each (the caller's arrays: the group kernel's own, or a prefill tile kernel's K/V buffers
// when the decode items of a prefill batch run inside the tile launch).
template <int D, bool F8, bool kPad, bool kTL, int kU, typename Part>
__device__ __forceinline__ void decode_group_body(
    const __bf16* __restrict__ q, void* k_cache_v, void* v_cache_v,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ context_lens,
    __bf16* __restrict__ out, const ItemArgs& items, int mbpr, int hq, int hkv,
    float scale_log2, int dr, int rep, int group, Part part, float* lds_m, float* lds_l) {
    const int ds = kPad ? dr : D;  // q / output row stride
    constexpr int W = GroupShape<D>::kWaves;
    constexpr int NV = DecodeShape<D>::kNV;
    constexpr int kMaxG = GroupShape<D>::kMaxG;
    using Cache = std::conditional_t<F8, uint8_t, __bf16>;
    // Neither const nor restrict: the fused new-token write (write_new_token) stores
    // through these pointers before the split's loads read the same rows.
    Cache* k_cache = static_cast<Cache*>(k_cache_v);
    Cache* v_cache = static_cast<Cache*>(v_cache_v);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = group % hkv;
    const int item = group / hkv;
    int req, qrow;
    if (!resolve_item(items, item, &req, &qrow)) return;  // workgroup-uniform
    if (items.singles_total >= 0 &&
        !single_token_request(items.qsl, context_lens, req, items.singles_total))
        return;  // workgroup-uniform: a tile of the prefill launch owns this request
    const int G = hq / hkv;
    // Parts are cut from the table row (mbpr blocks) in whole 32-token chunks, so every
    // wavefront's block ids and Q are loaded together with the context length.
    const int ctx_raw = context_lens[req];
    const int per = ((mbpr + 1) / 2 + W - 1) / W;  // chunks per part
    const int begin = wave * per * kChunk;
    const int tbl_end = min(mbpr * kBlock, begin + per * kChunk);
    SplitInputs<D> in;
    load_split_inputs<D, F8, kPad>(q, block_table + static_cast<int64_t>(req) * mbpr, mbpr, qrow,
                                   hq, h, G, begin, max(begin, tbl_end), lane, in, dr);
    const int ctx = effective_ctx(ctx_raw, mbpr, items.zero_invalid);
    if (ctx < 0) {
        // Decode semantics: invalid context -> zeros; prefill semantics: row untouched.
        if (items.zero_invalid) {
            for (int x = threadIdx.x; x < G * ds; x += 64 * W)
                out[(static_cast<int64_t>(qrow) * hq + h * G) * ds + x] = static_cast<__bf16>(0.0f);
        }
        return;
    }
    const int end = min(ctx, tbl_end);
    if constexpr (!F8) {
        if (items.new_k != nullptr && begin < end && end == ctx)
            write_new_token<kPad>(k_cache, v_cache, items, block_table + static_cast<int64_t>(req) * mbpr,
                                  req, ctx, hkv / rep, h / rep, ds, lane);
    }
    SoftmaxState<D> st;
    if (begin < end) {
        run_split<D, F8, kPad, kTL, DecodeShape<D>::kSteps, 2, kU>(
            k_cache, v_cache, k_scale, v_scale, in, hkv / rep, h / rep, begin, end, scale_log2,
            lane, st, dr);
    } else {
#pragma unroll
        for (int n = 0; n < NV; ++n) st.acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
        st.m = kNegInf;
        st.l = 0.f;
    }
    const float l_tot = wave_sum_xor16_32(st.l);
    const int j = lane & 15;
    const int g = lane >> 4;
    if (j < G) {
        float* po = part(wave) + j * D;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int n = 0; n < NV; ++n) po[NV * (4 * g + r) + n] = st.acc[n][r];
        if (g == 0) {
            lds_m[wave * kMaxG + j] = st.m;
            lds_l[wave * kMaxG + j] = l_tot;
        }
    }
    __syncthreads();
    constexpr int kPer = MergeCols<D>::kPer;
    for (int jj = wave; jj < G; jj += W) {
        float mmax = kNegInf;
#pragma unroll
        for (int w = 0; w < W; ++w) mmax = fmaxf(mmax, lds_m[w * kMaxG + jj]);
        float acc[kPer];
#pragma unroll
        for (int x = 0; x < kPer; ++x) acc[x] = 0.f;
        float lsum = 0.f;
        if (mmax != kNegInf) {
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float wt = __builtin_amdgcn_exp2f(lds_m[w * kMaxG + jj] - mmax);
                lsum += lds_l[w * kMaxG + jj] * wt;
                const float* pw = part(w) + jj * D;
#pragma unroll
                for (int x = 0; x < kPer; ++x) acc[x] += pw[MergeCols<D>::col(lane, x)] * wt;
            }
        }
        const float inv = lsum > 0.f ? 1.f / (lsum + items.eps) : 0.f;
        __bf16* o = out + (static_cast<int64_t>(qrow) * hq + h * G + jj) * ds;
#pragma unroll
        for (int x = 0; x < kPer; ++x)
            if (lane * kPer + x < dr) o[lane * kPer + x] = static_cast<__bf16>(acc[x] * inv);
    }
}

}  // namespace ccinfer::hipk::dcore
