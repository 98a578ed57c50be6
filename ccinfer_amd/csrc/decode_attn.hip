// Paged decode attention for gfx950: split-KV (flash-decoding) on bf16 MFMA tiles.
//
// Semantics follow the reference decode (src/kernel/attention/decode_attn.cu:364-473):
//   out[b, hq, :] = softmax(q . K_ctx^T / sqrt(D)) . V_ctx  with kv_head = hq / (Hq/Hkv),
//   positions addressed through block_table (16-token blocks), negative block ids skipped,
//   ctx <= 0 or ceil(ctx/16) > max_blocks_per_req -> zeros, denominator sum + 1e-6.
//
// Work decomposition (one wavefront = one work item):
//   item = (query row, kv_head, split). A split covers `split_tokens` consecutive context
//   positions (a multiple of 32). All Hq/Hkv query heads of the GQA group are handled by the
//   same wavefront, so every K/V byte of a (request, kv_head) is read from HBM exactly once.
//
// Per 32-token chunk (two 16-token cache blocks) the wavefront computes
//   S^T[token][head] = K[token][:] . Q^T           (v_mfma_f32_16x16x32_bf16, D/32 steps/block)
//   O^T[dim][head]  += V^T[dim][token] . P^T        (D/16 MFMAs over the 32 tokens)
// MFMA lane layout (16x16x32): lane = col + 16*grp; the A/B operands hold 8 consecutive
// k-values of row/col (lane%16) for k-group grp; the result holds rows 4*grp..4*grp+3.
// With S^T's rows = tokens and cols = heads, lane (head j, grp g) ends up with the scores of
// tokens T(g,e) = 16*(e/4) + 4*g + e%4, e = 0..7 -- exactly the 8 k-values the P^T operand of
// the PV MFMA needs in that lane, so P never moves between lanes. The V^T operand needs, per
// lane (dim row i, grp g), 8 tokens of one dim: each lane loads the 8 token rows T(g,e) at
// dims [NV*i, NV*i+NV) with 16-byte loads (a 256-byte row is covered by 16 lanes) and
// transposes in registers with v_perm_b32. O^T lands with every accumulator of a lane
// belonging to one head, so the online-softmax rescale is lane-local.
//
// Partial results (unnormalised O, running max m, sum l) go to a workspace and a second
// kernel merges the splits with a log-sum-exp weighting. With a single split the first
// kernel writes the output directly.
#include "attn_common.hpp"
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

constexpr int kBlock = 16;        // tokens per KV block (the reference's kKVBlockSize)
constexpr int kChunk = 32;        // tokens per PV MFMA
constexpr int kWavesPerGroup = 4;

struct ItemArgs {
    int num_items;
    const int32_t* item_count;
    const int32_t* item_req;
    const int32_t* qsl;
    float eps;
    int zero_invalid;
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

template <int D>
struct ChunkRegs {
    u32x4 k[2][DecodeShape<D>::kSteps];
    uint32_t v[8][DecodeShape<D>::kVWords];
};

template <int D>
__device__ __forceinline__ void load_chunk(ChunkRegs<D>& c, const __bf16* __restrict__ k_cache,
                                           const __bf16* __restrict__ v_cache, int pb0, int pb1,
                                           int kv_head, int hkv, int lane) {
    constexpr int S = DecodeShape<D>::kSteps;
    constexpr int NV = DecodeShape<D>::kNV;
    const int i = lane & 15;
    const int g = lane >> 4;
    const int pbs[2] = {pb0 < 0 ? 0 : pb0, pb1 < 0 ? 0 : pb1};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        const __bf16* row =
            k_cache + ((static_cast<int64_t>(pbs[kb]) * kBlock + i) * hkv + kv_head) * D;
#pragma unroll
        for (int kk = 0; kk < S; ++kk) c.k[kb][kk] = load16(row + (kk * 4 + g) * 8);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int kb = e >> 2;
        const int off = g * 4 + (e & 3);
        const __bf16* row =
            v_cache + ((static_cast<int64_t>(pbs[kb]) * kBlock + off) * hkv + kv_head) * D +
            i * NV;
        if constexpr (NV == 8) {
            const u32x4 w = load16(row);
#pragma unroll
            for (int x = 0; x < 4; ++x) c.v[e][x] = w[x];
        } else if constexpr (NV == 4) {
            const u32x2 w = *reinterpret_cast<const u32x2*>(row);
            c.v[e][0] = w[0];
            c.v[e][1] = w[1];
        } else {
            const u32x4 w0 = load16(row);
            const u32x4 w1 = load16(row + 8);
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                c.v[e][x] = w0[x];
                c.v[e][4 + x] = w1[x];
            }
        }
    }
}

template <int D>
__global__ __launch_bounds__(256) void decode_split_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k_cache,
    const __bf16* __restrict__ v_cache, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ context_lens, __bf16* __restrict__ out, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, ItemArgs items, int mbpr, int hq, int hkv, int splits,
    int split_tokens, float scale_log2, int direct_out) {
    constexpr int S = DecodeShape<D>::kSteps;
    constexpr int NV = DecodeShape<D>::kNV;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wi = blockIdx.x * kWavesPerGroup + wave;
    const int s = wi % splits;
    const int rest = wi / splits;
    const int h = rest % hkv;
    const int item = rest / hkv;

    int req, qrow;
    if (!resolve_item(items, item, &req, &qrow)) return;
    const int ctx = effective_ctx(context_lens[req], mbpr, items.zero_invalid);
    const int G = hq / hkv;
    const int j = lane & 15;
    const int g = lane >> 4;

    if (ctx < 0) {
        // Decode semantics: invalid context -> zeros (written once, by split 0).
        if (direct_out && items.zero_invalid && s == 0 && j < G && g == 0) {
            __bf16* o = out + (static_cast<int64_t>(qrow) * hq + h * G + j) * D;
            for (int d = 0; d < D; ++d) o[d] = static_cast<__bf16>(0.0f);
        }
        return;
    }
    const int begin = s * split_tokens;
    if (begin >= ctx) return;
    const int end = min(ctx, begin + split_tokens);
    const int32_t* req_blocks = block_table + static_cast<int64_t>(req) * mbpr;

    // Q^T operand: lane (head j, grp g) holds dims (kk*4+g)*8 .. +8 of head j.
    bf16x8 qop[S];
    {
        const bool live = j < G;
        const __bf16* qv = q + (static_cast<int64_t>(qrow) * hq + h * G + (live ? j : 0)) * D;
#pragma unroll
        for (int kk = 0; kk < S; ++kk) {
            u32x4 w = load16(qv + (kk * 4 + g) * 8);
            if (!live) w = u32x4{0, 0, 0, 0};
            qop[kk] = __builtin_bit_cast(bf16x8, w);
        }
    }

    f32x4 acc[NV];
#pragma unroll
    for (int n = 0; n < NV; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = kNegInf;
    float l = 0.f;

    auto table = [&](int lb) -> int { return lb < mbpr ? req_blocks[lb] : -1; };

    int cb = begin;
    int pb0 = table(cb / kBlock);
    int pb1 = (cb + kBlock < end) ? table(cb / kBlock + 1) : -1;
    ChunkRegs<D> cur;
    load_chunk<D>(cur, k_cache, v_cache, pb0, pb1, h, hkv, lane);

    for (; cb < end; cb += kChunk) {
        // Prefetch the next chunk while this one is consumed.
        const int nb = cb + kChunk;
        int npb0 = -1, npb1 = -1;
        ChunkRegs<D> nxt;
        if (nb < end) {
            npb0 = table(nb / kBlock);
            npb1 = (nb + kBlock < end) ? table(nb / kBlock + 1) : -1;
            load_chunk<D>(nxt, k_cache, v_cache, npb0, npb1, h, hkv, lane);
        }

        // S^T = K . Q^T for the two 16-token blocks.
        float sc[8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < S; ++kk)
                st = mfma16x16x32(__builtin_bit_cast(bf16x8, cur.k[kb][kk]), qop[kk], st);
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[kb * 4 + r] = st[r] * scale_log2;
        }

        const bool full = (cb + kChunk <= end) && pb0 >= 0 && pb1 >= 0;
        if (!full) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int kb = e >> 2;
                const int pos = cb + kb * kBlock + g * 4 + (e & 3);
                const bool ok = pos < end && (kb == 0 ? pb0 : pb1) >= 0;
                if (!ok) {
                    sc[e] = kNegInf;
#pragma unroll
                    for (int x = 0; x < DecodeShape<D>::kVWords; ++x) cur.v[e][x] = 0u;
                }
            }
        }

        // Online softmax (base-2 domain); rows of a head live in lanes j, j+16, j+32, j+48.
        float mloc = sc[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) mloc = fmaxf(mloc, sc[e]);
        mloc = wave_max_xor16_32(mloc);
        const float m_new = fmaxf(m, mloc);
        const float m_use = (m_new == kNegInf) ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m - m_use);
        float p[8];
        float psum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            p[e] = __builtin_amdgcn_exp2f(sc[e] - m_use);
            psum += p[e];
        }
        l = l * alpha + psum;
        m = m_new;
        u32x4 pw;
#pragma unroll
        for (int x = 0; x < 4; ++x) pw[x] = pack_bf16x2(p[2 * x], p[2 * x + 1]);
        const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);

#pragma unroll
        for (int n = 0; n < NV; ++n) {
            u32x4 vw;
#pragma unroll
            for (int x = 0; x < 4; ++x)
                vw[x] = pick_halves(cur.v[2 * x][n >> 1], cur.v[2 * x + 1][n >> 1], n & 1);
            acc[n] = acc[n] * alpha;
            acc[n] = mfma16x16x32(__builtin_bit_cast(bf16x8, vw), pop, acc[n]);
        }

        if (nb < end) {
            cur = nxt;
            pb0 = npb0;
            pb1 = npb1;
        }
    }

    const float l_tot = wave_sum_xor16_32(l);
    if (j >= G) return;
    const int head = h * G + j;
    // Lane (j, g) holds O[head][NV*(4g+r) + n] = acc[n][r].
    if (direct_out) {
        const float inv = l_tot > 0.f ? 1.f / (l_tot + items.eps) : 0.f;
        __bf16* o = out + (static_cast<int64_t>(qrow) * hq + head) * D;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint32_t w[NV / 2];
#pragma unroll
            for (int x = 0; x < NV / 2; ++x)
                w[x] = pack_bf16x2(acc[2 * x][r] * inv, acc[2 * x + 1][r] * inv);
            uint32_t* dst = reinterpret_cast<uint32_t*>(o + NV * (4 * g + r));
#pragma unroll
            for (int x = 0; x < NV / 2; ++x) dst[x] = w[x];
        }
    } else {
        const int64_t slot = (static_cast<int64_t>(item) * hq + head) * splits + s;
        float* po = ws_o + slot * D;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int n = 0; n < NV; ++n) po[NV * (4 * g + r) + n] = acc[n][r];
        }
        if (g == 0) {
            ws_ml[slot * 2 + 0] = m;
            ws_ml[slot * 2 + 1] = l_tot;
        }
    }
}

// One wavefront per (item, q_head): log-sum-exp merge of the valid splits.
template <int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(
    const int32_t* __restrict__ context_lens, __bf16* __restrict__ out,
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, ItemArgs items, int mbpr,
    int hq, int splits, int split_tokens) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wi = blockIdx.x * kWavesPerGroup + wave;
    const int head = wi % hq;
    const int item = wi / hq;
    int req, qrow;
    if (!resolve_item(items, item, &req, &qrow)) return;
    const int ctx = effective_ctx(context_lens[req], mbpr, items.zero_invalid);
    constexpr int kPer = D / 64;
    __bf16* o = out + (static_cast<int64_t>(qrow) * hq + head) * D;
    if (ctx < 0) {
        if (items.zero_invalid) {
#pragma unroll
            for (int x = 0; x < kPer; ++x) o[lane * kPer + x] = static_cast<__bf16>(0.0f);
        }
        return;
    }
    const int ns = (ctx + split_tokens - 1) / split_tokens;
    const int64_t base = (static_cast<int64_t>(item) * hq + head) * splits;
    float mmax = kNegInf;
    for (int s = lane; s < ns; s += 64) mmax = fmaxf(mmax, ws_ml[(base + s) * 2]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, off));
    float acc[kPer];
#pragma unroll
    for (int x = 0; x < kPer; ++x) acc[x] = 0.f;
    float lsum = 0.f;
    if (mmax != kNegInf) {
        for (int s = 0; s < ns; ++s) {
            const float ms = ws_ml[(base + s) * 2];
            const float w = __builtin_amdgcn_exp2f(ms - mmax);
            lsum += ws_ml[(base + s) * 2 + 1] * w;
            const float* po = ws_o + (base + s) * D + lane * kPer;
#pragma unroll
            for (int x = 0; x < kPer; ++x) acc[x] += po[x] * w;
        }
    }
    const float inv = lsum > 0.f ? 1.f / (lsum + items.eps) : 0.f;
#pragma unroll
    for (int x = 0; x < kPer; ++x) o[lane * kPer + x] = static_cast<__bf16>(acc[x] * inv);
}

template <int D>
hipError_t launch_decode(const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* block_table, const int32_t* context_lens, void* output,
                         const ItemArgs& it, int mbpr, int hq, int hkv, const DecodePlan& plan,
                         void* workspace, hipStream_t stream) {
    const float scale_log2 = kLog2e / sqrtf(static_cast<float>(D));
    const int64_t waves = static_cast<int64_t>(it.num_items) * hkv * plan.splits;
    const int grid = static_cast<int>((waves + kWavesPerGroup - 1) / kWavesPerGroup);
    const bool direct = plan.splits == 1;
    float* ws_o = static_cast<float*>(workspace);
    float* ws_ml = direct ? nullptr
                          : ws_o + static_cast<int64_t>(it.num_items) * hq * plan.splits * D;
    decode_split_kernel<D><<<grid, 256, 0, stream>>>(
        static_cast<const __bf16*>(q), static_cast<const __bf16*>(k_cache),
        static_cast<const __bf16*>(v_cache), block_table, context_lens,
        static_cast<__bf16*>(output), ws_o, ws_ml, it, mbpr, hq, hkv, plan.splits,
        plan.split_tokens, scale_log2, direct ? 1 : 0);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || direct) return err;
    const int64_t mw = static_cast<int64_t>(it.num_items) * hq;
    const int mgrid = static_cast<int>((mw + kWavesPerGroup - 1) / kWavesPerGroup);
    decode_merge_kernel<D><<<mgrid, 256, 0, stream>>>(context_lens,
                                                      static_cast<__bf16*>(output), ws_o, ws_ml,
                                                      it, mbpr, hq, plan.splits,
                                                      plan.split_tokens);
    return hipGetLastError();
}

}  // namespace

DecodePlan plan_decode(int num_items, int num_kv_heads, int max_ctx) {
    DecodePlan p;
    const int chunks = max_ctx > 0 ? (max_ctx + kChunk - 1) / kChunk : 1;
    // Aim for ~16 wavefronts per CU (256 CUs) of work so ragged batches still balance.
    const int64_t target_waves = 4096;
    const int64_t total = static_cast<int64_t>(num_items) * num_kv_heads * chunks;
    int64_t cpw = (total + target_waves - 1) / target_waves;
    if (cpw < 1) cpw = 1;
    if (cpw > chunks) cpw = chunks;
    p.split_tokens = static_cast<int>(cpw) * kChunk;
    p.splits = (chunks + static_cast<int>(cpw) - 1) / static_cast<int>(cpw);
    return p;
}

size_t decode_workspace_bytes(int num_items, int num_q_heads, int head_dim,
                              const DecodePlan& plan) {
    if (plan.splits <= 1) return 0;
    return static_cast<size_t>(num_items) * num_q_heads * plan.splits * (head_dim + 2) *
           sizeof(float);
}

bool decode_fast_supported(int num_q_heads, int num_kv_heads, int head_dim, int block_size) {
    if (block_size != kBlock || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0)
        return false;
    const int G = num_q_heads / num_kv_heads;
    return G >= 1 && G <= 16 && (head_dim == 64 || head_dim == 128 || head_dim == 256);
}

hipError_t decode_attention(const void* q, const void* k_cache, const void* v_cache,
                            const int32_t* block_table, const int32_t* context_lens, void* output,
                            const DecodeItems& items, int max_blocks_per_req, int num_q_heads,
                            int num_kv_heads, int head_dim, int block_size,
                            const DecodePlan& plan, void* workspace, hipStream_t stream) {
    (void)block_size;
    ItemArgs it{items.num_items, items.item_count, items.item_req, items.query_start_loc,
                items.denom_eps, items.zero_invalid ? 1 : 0};
    switch (head_dim) {
        case 64:
            return launch_decode<64>(q, k_cache, v_cache, block_table, context_lens, output, it,
                                     max_blocks_per_req, num_q_heads, num_kv_heads, plan,
                                     workspace, stream);
        case 128:
            return launch_decode<128>(q, k_cache, v_cache, block_table, context_lens, output, it,
                                      max_blocks_per_req, num_q_heads, num_kv_heads, plan,
                                      workspace, stream);
        case 256:
            return launch_decode<256>(q, k_cache, v_cache, block_table, context_lens, output, it,
                                      max_blocks_per_req, num_q_heads, num_kv_heads, plan,
                                      workspace, stream);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace ccinfer::hipk
