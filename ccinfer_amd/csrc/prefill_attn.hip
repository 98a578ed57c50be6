// Paged causal prefill attention for gfx950 (bf16 MFMA, fp32 accumulation).
//
// Semantics follow the reference prefill (src/kernel/attention/prefill_attn.cu:80-241 and
// the contract in src/backend/params.h:140-146):
//   request r owns query rows [query_start_loc[r], query_start_loc[r+1]); prefix =
//   context_lens[r] - qlen; local query i attends to cache positions [0, prefix + i]
//   through the block table (negative ids / positions past the table are skipped);
//   rows of requests with prefix < 0 are left unwritten; out = sum(p v) / sum(p) (0 if
//   nothing is visible).
//
// Launch plan (all on the caller's stream, no host sync, no allocation):
//   1. plan kernel (one workgroup): reads query_start_loc / context_lens, emits the list of
//      query tiles sorted longest-first (counting sort on the number of visible keys), and
//      the list of single-token requests (decode items of a mixed batch).
//   2. tile kernel: one workgroup (4 wavefronts) per (query tile, kv_head, head group).
//      Each wavefront owns QW = 64 query rows of one q-head (32 for head_dim 256); the
//      workgroup covers Hq/Hkv heads that share one KV head so every K/V tile staged in LDS
//      serves all of them. K/V tiles of 64 positions are gathered through the block table
//      into LDS (double-buffered: the next tile's global loads are in flight while MFMAs run
//      on the current one). Scores are formed transposed, S^T = K . Q^T, so the softmax'd
//      probabilities are already in the lane layout of the P^T operand of O^T = V^T . P^T,
//      and every O accumulator of a lane belongs to one query row (lane-local rescale).
//      Tiles entirely above the causal diagonal are skipped; masking only runs on the
//      diagonal / ragged tiles.
//   3. single-token requests go through the split-KV decode kernel (decode_attn.hip) with
//      prefill semantics (no 1e-6 in the denominator, bad rows left untouched).
#include <type_traits>

#include "attn_common.hpp"
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

constexpr int kKeysPerTile = 64;
constexpr int kThreads = 512;     // tile kernel: 8 wavefronts, 2 per SIMD
constexpr int kWaves = kThreads / 64;
constexpr int kBlock = 16;        // cache block size of the fast path
constexpr int kMaxTableLds = 4096;  // block-table entries staged in LDS (64K-token context)
constexpr int kBuckets = 1024;
constexpr int kMaxPlanRequests = 4096;

template <int D>
struct PrefillShape {
    static constexpr int kQT = D <= 128 ? 2 : 1;     // 16-row query tiles per wavefront
    static constexpr int kQW = 16 * kQT;             // query rows per wavefront
    static constexpr int kSteps = D / 32;            // QK k-steps
    static constexpr int kNV = D / 16;               // PV MFMAs per query tile
    static constexpr int kCPR = D / 8;               // 16-byte chunks per K/V row
    static constexpr int kLoadsPerThread = kKeysPerTile * kCPR / kThreads;  // per K or V
};

// Heads per workgroup: the 8 wavefronts split as HPW heads x (8/HPW) row groups.
__host__ __device__ inline int heads_per_wg(int G) {
    return (G % 4 == 0) ? 4 : ((G % 2 == 0) ? 2 : 1);
}

struct TileEntry {
    int req;
    int t0;
};

// In-place inclusive prefix sum of a[0..n) (n <= 4 * blockDim.x) by a 1024-thread block.
// Each thread scans up to 4 consecutive entries, then a Hillis-Steele pass over the
// per-thread totals adds the carries. Must be called by every thread of the block.
__device__ void block_inclusive_scan(int* a, int n, int* part) {
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    const int per = (n + nt - 1) / nt;
    const int lo = tid * per;
    const int hi = min(n, lo + per);
    int run = 0;
    for (int x = lo; x < hi; ++x) {
        run += a[x];
        a[x] = run;
    }
    part[tid] = run;
    __syncthreads();
    for (int off = 1; off < nt; off <<= 1) {
        const int v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    const int carry = tid > 0 ? part[tid - 1] : 0;
    for (int x = lo; x < hi; ++x) a[x] += carry;
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Planner: one workgroup of 1024 threads.
// ws layout: counts[0] = #tiles, counts[1] = #decode items; tiles[max_tiles]; dec[B].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void prefill_plan_kernel(
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ context_lens, int batch_size,
    int total_tokens, int tile_tokens, int32_t* __restrict__ counts,
    TileEntry* __restrict__ tiles, int32_t* __restrict__ dec_req, uint32_t* __restrict__ zero_row,
    int zero_words) {
    __shared__ int s_ntiles[kMaxPlanRequests];
    __shared__ int s_scan[kMaxPlanRequests];
    __shared__ int s_hist[kBuckets];
    __shared__ int s_hscan[kBuckets];
    __shared__ int s_part[1024];
    __shared__ int s_ndec;
    __shared__ int s_total;
    const int tid = threadIdx.x;
    for (int i = tid; i < zero_words; i += blockDim.x) zero_row[i] = 0u;  // staging's zero row
    for (int i = tid; i < kBuckets; i += blockDim.x) s_hist[i] = 0;
    if (tid == 0) s_ndec = 0;
    __syncthreads();

    // Per-request tile counts; single-token requests become decode items.
    for (int b = tid; b < batch_size; b += blockDim.x) {
        const int qb = qsl[b];
        const int qe_raw = qsl[b + 1];
        const int qlen = qe_raw - qb;
        const int qe = qe_raw < total_tokens ? qe_raw : total_tokens;
        const int rows = qe - (qb > 0 ? qb : 0);
        const int prefix = context_lens[b] - qlen;
        int n = 0;
        if (qlen > 0 && prefix >= 0 && qb >= 0 && rows > 0) {
            if (qlen == 1) {
                const int slot = atomicAdd(&s_ndec, 1);
                dec_req[slot] = b;
            } else {
                n = (rows + tile_tokens - 1) / tile_tokens;
            }
        }
        s_ntiles[b] = n;
    }
    __syncthreads();
    for (int b = tid; b < batch_size; b += blockDim.x) s_scan[b] = s_ntiles[b];
    __syncthreads();
    block_inclusive_scan(s_scan, batch_size, s_part);
    if (tid == 0) s_total = batch_size > 0 ? s_scan[batch_size - 1] : 0;
    __syncthreads();
    const int total = s_total;
    auto locate = [&](int t, int* b_out, int* r_out) {
        int lo = 0, hi = batch_size - 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (s_scan[mid] > t) hi = mid; else lo = mid + 1;
        }
        *b_out = lo;
        *r_out = t - (s_scan[lo] - s_ntiles[lo]);
    };
    auto bucket_of = [&](int b, int r) {
        const int qlen = qsl[b + 1] - qsl[b];
        const int prefix = context_lens[b] - qlen;
        int last = (r + 1) * tile_tokens;
        if (last > qlen) last = qlen;
        const int cost = (prefix + last) >> 6;
        return kBuckets - 1 - (cost < kBuckets - 1 ? cost : kBuckets - 1);
    };
    for (int t = tid; t < total; t += blockDim.x) {
        int b, r;
        locate(t, &b, &r);
        atomicAdd(&s_hist[bucket_of(b, r)], 1);
    }
    __syncthreads();
    // Exclusive scan of the histogram -> first slot of each bucket.
    for (int i = tid; i < kBuckets; i += blockDim.x) s_hscan[i] = s_hist[i];
    __syncthreads();
    block_inclusive_scan(s_hscan, kBuckets, s_part);
    for (int i = tid; i < kBuckets; i += blockDim.x) s_hist[i] = s_hscan[i] - s_hist[i];
    __syncthreads();
    for (int t = tid; t < total; t += blockDim.x) {
        int b, r;
        locate(t, &b, &r);
        const int pos = atomicAdd(&s_hist[bucket_of(b, r)], 1);
        tiles[pos] = TileEntry{b, r * tile_tokens};
    }
    if (tid == 0) {
        counts[0] = total;
        counts[1] = s_ndec;
    }
}

// ---------------------------------------------------------------------------
// Tile kernel.
// ---------------------------------------------------------------------------

// Swizzle of the 16-byte chunk index of K/V row `row` in LDS. f is a permutation of 0..15
// over any 16 consecutive rows, so the K operand read (16 rows, one logical chunk) hits 16
// distinct chunk positions, and for any 4 rows 4g..4g+3 and chunk pair {2n, 2n+1} -- one
// transposing V read -- the 8 (row, chunk) pieces land on 8 distinct positions.
__device__ __forceinline__ int chunk_swizzle(int row) {
    const int i = row & 15;
    return ((i & 3) << 1) | ((i & 4) << 1) | ((i >> 3) & 1);
}

template <int D>
__device__ __forceinline__ int lds_off(int row, int chunk) {
    // Element offset of logical 16-byte chunk `chunk` of key row `row`.
    constexpr int kMask = PrefillShape<D>::kCPR - 1;
    return row * D + ((chunk ^ (chunk_swizzle(row) & kMask)) << 3);
}

// Direct global->LDS staging of one 64-key K/V tile (gfx950 global_load_lds_dwordx4): an
// instruction moves 16 bytes per lane straight into LDS at base + 16*lane, so the chunk
// swizzle is applied on the source side: LDS slot p holds row p/CPR, logical chunk
// (p%CPR) ^ swizzle(row). Rows outside the visible range (past the context, negative block
// ids, past the table row) are fetched from `zero_row` so the tile never holds garbage that
// a masked probability of 0 could turn into NaN. Validity flags go to lvalid[row].
template <int D>
__device__ __forceinline__ void stage_issue(__bf16* lk, __bf16* lv, uint8_t* lvalid,
                                            const __bf16* __restrict__ k_cache,
                                            const __bf16* __restrict__ v_cache,
                                            const __bf16* __restrict__ zero_row,
                                            const int32_t* lbt, int key_base, int ctx, int nblk,
                                            int kv_head, int hkv) {
    constexpr int CPR = PrefillShape<D>::kCPR;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int x = 0; x < PrefillShape<D>::kLoadsPerThread; ++x) {
        const int slot0 = (x * kWaves + wave) * 64;  // first 16-byte LDS slot of this load
        const int p = slot0 + lane;
        const int row = p / CPR;
        const int lchunk = (p % CPR) ^ (chunk_swizzle(row) & (CPR - 1));
        const int key = key_base + row;
        const int lb = key >> 4;
        int pb = -1;
        if (key < ctx && lb < nblk) pb = lbt[lb];
        const __bf16* ks = zero_row;
        const __bf16* vs = zero_row;
        if (pb >= 0) {
            const int64_t base =
                ((static_cast<int64_t>(pb) * kBlock + (key & (kBlock - 1))) * hkv + kv_head) * D;
            ks = k_cache + base;
            vs = v_cache + base;
        }
        __builtin_amdgcn_global_load_lds(
            ks + lchunk * 8, (__attribute__((address_space(3))) void*)(lk + slot0 * 8), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(
            vs + lchunk * 8, (__attribute__((address_space(3))) void*)(lv + slot0 * 8), 16, 0, 0);
        if ((p % CPR) == 0) lvalid[row] = static_cast<uint8_t>(pb >= 0);
    }
}

// V^T MFMA operand for dim tile n of a 32-key half, read transposed straight out of the
// row-major [key][dim] LDS tile with ds_read_b64_tr_b16 (gfx950). Within a 16-lane group g,
// result lane i gets element e from the lane (4e + i/4) of the group, 16-bit word i%4.
// Pointing source lane s at V[key 4g + s/4][dims 16n + 4(s%4) ..+3] therefore hands lane
// (dim i, group g) the 4 consecutive keys 4g..4g+3 of dim 16n+i; a second read covers keys
// 16+4g..16+4g+3. Those 8 keys are exactly T(g, e) = 16*(e/4) + 4g + e%4, the keys the
// P^T operand of the same lane carries, so no register transpose is needed.
template <int D>
__device__ __forceinline__ bf16x8 load_vt(const __bf16* lv, int h2, int n, int lane) {
    using v4s = short __attribute__((ext_vector_type(4)));
    const int s = lane & 15;
    const int g = lane >> 4;
    const int row = h2 * 32 + 4 * g + (s >> 2);
    const int dim = 16 * n + 4 * (s & 3);
    const int chunk = dim >> 3;
    const int within = dim & 7;
    const __bf16* p0 = lv + lds_off<D>(row, chunk) + within;
    const __bf16* p1 = lv + lds_off<D>(row + 16, chunk) + within;
    const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4s*)(p0));
    const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4s*)(p1));
    using v8s = short __attribute__((ext_vector_type(8)));
    const v8s ab = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(bf16x8, ab);
}

// Max growth (log2 units) tolerated before the accumulators are rescaled. Probabilities
// stay <= 2^8 and sums of them fit fp32 comfortably; acc and l always share one reference
// max, so the final acc / l is exact whatever the reference.
constexpr float kRescaleSlack = 8.0f;

template <int D>
__global__ __launch_bounds__(kThreads) void prefill_tile_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k_cache,
    const __bf16* __restrict__ v_cache, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ context_lens,
    __bf16* __restrict__ out, const int32_t* __restrict__ counts,
    const TileEntry* __restrict__ tiles, const __bf16* __restrict__ zero_row, int total_tokens,
    int mbpr, int hq, int hkv, int block_size, float scale_log2) {
    (void)block_size;  // the fast path is specialised for 16-token blocks
    using Sh = PrefillShape<D>;
    constexpr int QT = Sh::kQT;
    constexpr int QW = Sh::kQW;
    constexpr int S = Sh::kSteps;
    constexpr int NT = D / 16;  // PV dim tiles
    // Two K/V buffers as distinct arrays: every access names its buffer statically, so the
    // compiler can see that the direct-to-LDS loads filling one buffer never alias reads of
    // the other and does not drain them before the attention math.
    __shared__ __attribute__((aligned(16))) __bf16 lds_k0[kKeysPerTile * D];
    __shared__ __attribute__((aligned(16))) __bf16 lds_k1[kKeysPerTile * D];
    __shared__ __attribute__((aligned(16))) __bf16 lds_v0[kKeysPerTile * D];
    __shared__ __attribute__((aligned(16))) __bf16 lds_v1[kKeysPerTile * D];
    __shared__ uint8_t lds_valid0[kKeysPerTile];
    __shared__ uint8_t lds_valid1[kKeysPerTile];
    // The request's block-table entries for the visible range (-1 past the table row).
    __shared__ int32_t lds_bt[kMaxTableLds];

    const int G = hq / hkv;
    const int HPW = heads_per_wg(G);
    const int WPH = kWaves / HPW;
    const int U = hkv * (G / HPW);
    const int tile_idx = blockIdx.x / U;
    if (tile_idx >= counts[0]) return;
    const int u = blockIdx.x % U;
    const int kvh = u / (G / HPW);
    const int hg = u % (G / HPW);
    const TileEntry te = tiles[tile_idx];
    const int req = te.req;
    const int t0 = te.t0;

    const int qb = qsl[req];
    const int qlen = qsl[req + 1] - qb;
    const int ctx = context_lens[req];
    const int prefix = ctx - qlen;
    const int qe = min(qb + qlen, total_tokens);
    const int rows = qe - qb;  // rows of this request that exist in q/out
    const int TT = WPH * QW;
    const int kv_end = prefix + min(t0 + TT, rows);
    const int ntiles = (kv_end + kKeysPerTile - 1) / kKeysPerTile;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int head_local = wave / WPH;
    const int tw = t0 + (wave % WPH) * QW;  // first local token of this wavefront
    const int q_head = kvh * G + hg * HPW + head_local;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int wave_rows = max(0, min(QW, rows - tw));
    const int wave_max_key = prefix + tw + wave_rows - 1;  // last key any row here sees
    const int32_t* req_blocks = block_table + static_cast<int64_t>(req) * mbpr;

    // Q^T operands: lane (query j, grp g) holds dims (kk*4+g)*8.. of row tw + qt*16 + j.
    bf16x8 qop[QT][S];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int tq = tw + qt * 16 + j;
        const bool live = tq < rows;
        const __bf16* qv = q + (static_cast<int64_t>(qb + (live ? tq : 0)) * hq + q_head) * D;
#pragma unroll
        for (int kk = 0; kk < S; ++kk) {
            u32x4 w = load16(qv + (kk * 4 + g) * 8);
            if (!live) w = u32x4{0, 0, 0, 0};
            qop[qt][kk] = __builtin_bit_cast(bf16x8, w);
        }
    }

    // O^T accumulators: acc[qt][n] lane (query j, grp g) = O[row][16n + 4g + r].
    // Row sums of P ride on the MFMA unit: ones(16x32) . P^T gives every lane of query
    // column j the full sum over the 32 keys (and sums the same bf16-rounded P that the PV
    // product uses).
    f32x4 acc[QT][NT];
    f32x4 lsum[QT];
    float m[QT];
    const bf16x8 ones = __builtin_bit_cast(
        bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m[qt] = kNegInf;  // reference max (log2 units, already scaled)
        lsum[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[qt][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // Stage the visible block-table slice in LDS (so tile staging never waits on a global
    // load) and note whether it has holes (negative or missing entries).
    __shared__ int s_holes;
    if (threadIdx.x == 0) s_holes = 0;
    __syncthreads();
    // Positions past the table row are invalid, so only min(visible, mbpr) entries matter;
    // the host routes tables longer than kMaxTableLds to the generic kernel.
    const int nblk_vis = (kv_end + kBlock - 1) / kBlock;
    const int nblk = min(nblk_vis, mbpr);
    for (int lb = threadIdx.x; lb < nblk; lb += kThreads) {
        const int pb = req_blocks[lb];
        lds_bt[lb] = pb;
        if (pb < 0) s_holes = 1;
    }
    __syncthreads();
    const bool holes = s_holes != 0 || nblk_vis > mbpr;

    stage_issue<D>(lds_k0, lds_v0, lds_valid0, k_cache, v_cache, zero_row, lds_bt, 0, ctx, nblk,
                   kvh, hkv);
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's direct-to-LDS loads have landed
    __syncthreads();

    // Attention over one staged 64-key tile, straight-line so the scheduler can overlap the
    // LDS reads, MFMAs and softmax VALU work of both 32-key halves. kMask selects the variant
    // with the causal / validity mask (diagonal, ragged-end and hole tiles only).
    auto attend_tile = [&](const __bf16* lk, const __bf16* lv, const uint64_t vmask, int key0,
                           auto mask_tag) __attribute__((always_inline)) {
        constexpr bool kMask = decltype(mask_tag)::value;
        // S^T: st[kb][qt] lane (query j, g) holds keys key0 + 16kb + 4g + r.
        f32x4 st[4][QT];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            if (kb == 2) __builtin_amdgcn_sched_barrier(0);  // bound K operands in flight
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) st[kb][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < S; ++kk) {
                const bf16x8 kop = __builtin_bit_cast(
                    bf16x8,
                    *reinterpret_cast<const u32x4*>(lk + lds_off<D>(kb * 16 + j, kk * 4 + g)));
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
                    st[kb][qt] = mfma16x16x32(kop, qop[qt][kk], st[kb][qt]);
            }
        }
        if constexpr (kMask) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const int limit = prefix + tw + qt * 16 + j;  // last visible key of the row
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int kt = kb * 16 + g * 4 + r;
                        const bool ok = key0 + kt <= limit && ((vmask >> kt) & 1ull);
                        st[kb][qt][r] = ok ? st[kb][qt][r] : kNegInf;
                    }
                }
            }
        }
        // Row max of the tile; rescale only when some row's max grew past the slack.
        float mt[QT];
        bool grow = false;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            float x = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                x = fmaxf(x, fmaxf(fmaxf(st[kb][qt][0], st[kb][qt][1]),
                                   fmaxf(st[kb][qt][2], st[kb][qt][3])));
            x = wave_max_xor16_32(x) * scale_log2;
            mt[qt] = x;
            grow |= x > m[qt] + kRescaleSlack;
        }
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const float m_new = fmaxf(m[qt], mt[qt]);
                const float alpha =
                    m_new == kNegInf ? 1.f : __builtin_amdgcn_exp2f(m[qt] - m_new);
                lsum[qt] = lsum[qt] * alpha;
#pragma unroll
                for (int n = 0; n < NT; ++n) acc[qt][n] = acc[qt][n] * alpha;
                m[qt] = m_new;
            }
        }
        // P = exp2(s * scale - m) as bf16 P^T operands; O^T += V^T . P^T; row sums.
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            // Keep each half's V reads and exp work in its own scheduling window (bounds the
            // registers in flight at two wavefronts per SIMD).
            __builtin_amdgcn_sched_barrier(0);
            bf16x8 pop[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const float mneg = m[qt] == kNegInf ? 0.f : -m[qt];
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    p[e] = __builtin_amdgcn_exp2f(
                        __builtin_fmaf(st[2 * h2 + (e >> 2)][qt][e & 3], scale_log2, mneg));
                }
                u32x4 pw;
#pragma unroll
                for (int x = 0; x < 4; ++x) pw[x] = pack_bf16x2(p[2 * x], p[2 * x + 1]);
                pop[qt] = __builtin_bit_cast(bf16x8, pw);
                lsum[qt] = mfma16x16x32(ones, pop[qt], lsum[qt]);
            }
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const bf16x8 vop = load_vt<D>(lv, h2, n, lane);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
                    acc[qt][n] = mfma16x16x32(vop, pop[qt], acc[qt][n]);
            }
        }
    };

    // One K/V tile from buffer B (0/1, a compile-time constant), with the next tile's loads
    // in flight into the other buffer. Every wavefront stages every tile and meets one barrier
    // per tile; the attention work is skipped for tiles entirely above its diagonal.
    auto process_tile = [&](int t, auto buf_tag, auto mask_tag) __attribute__((always_inline)) {
        constexpr int B = decltype(buf_tag)::value;
        __bf16* ck = B == 0 ? lds_k0 : lds_k1;
        __bf16* cv = B == 0 ? lds_v0 : lds_v1;
        uint8_t* cvalid = B == 0 ? lds_valid0 : lds_valid1;
        __bf16* nk = B == 0 ? lds_k1 : lds_k0;
        __bf16* nv = B == 0 ? lds_v1 : lds_v0;
        uint8_t* nvalid = B == 0 ? lds_valid1 : lds_valid0;
        const bool more = t + 1 < ntiles;
        if (more) {
            stage_issue<D>(nk, nv, nvalid, k_cache, v_cache, zero_row, lds_bt,
                           (t + 1) * kKeysPerTile, ctx, nblk, kvh, hkv);
        }
        const int key0 = t * kKeysPerTile;
        if (key0 <= wave_max_key) {
            const uint64_t vmask = decltype(mask_tag)::value
                                       ? __builtin_amdgcn_ballot_w64(cvalid[lane] != 0)
                                       : ~0ull;
            attend_tile(ck, cv, vmask, key0, mask_tag);
        }
        if (more) __builtin_amdgcn_s_waitcnt(0);  // next tile resident before the barrier
        __syncthreads();
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;

    // Tiles wholly below this wavefront's diagonal need no mask unless the block table has
    // holes inside the visible range (then every tile takes the masked path). Tiles go in
    // pairs (buffer 0 then 1); the mask-free count is rounded down to a pair.
    int mask_free = 0;
    if (!holes) mask_free = min(ntiles, (prefix + tw + 1) / kKeysPerTile) & ~1;
    int t = 0;
    for (; t < mask_free; t += 2) {
        process_tile(t, B0{}, std::false_type{});
        process_tile(t + 1, B1{}, std::false_type{});
    }
    for (; t + 1 < ntiles; t += 2) {
        process_tile(t, B0{}, std::true_type{});
        process_tile(t + 1, B1{}, std::true_type{});
    }
    if (t < ntiles) process_tile(t, B0{}, std::true_type{});

    // Epilogue: lane (j, g) holds O[row][16n + 4g + r] = acc[qt][n][r].
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float l_tot = lsum[qt][0];
        const int tq = tw + qt * 16 + j;
        if (tq >= rows) continue;
        const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
        __bf16* o = out + (static_cast<int64_t>(qb + tq) * hq + q_head) * D;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            u32x2 w;
            w[0] = pack_bf16x2(acc[qt][n][0] * inv, acc[qt][n][1] * inv);
            w[1] = pack_bf16x2(acc[qt][n][2] * inv, acc[qt][n][3] * inv);
            *reinterpret_cast<u32x2*>(o + 16 * n + 4 * g) = w;
        }
    }
}

struct PrefillLayout {
    size_t counts_off, zero_off, tiles_off, dec_off, decode_ws_off, total;
    int max_tiles;
    int tile_tokens;
    DecodePlan plan;
};

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int tile_tokens_for(int head_dim, int G) {
    const int qw = head_dim <= 128 ? 32 : 16;
    return (kWaves / heads_per_wg(G)) * qw;
}

PrefillLayout prefill_layout(int batch_size, int total_query_tokens, int max_blocks_per_req,
                             int num_q_heads, int num_kv_heads, int head_dim, int block_size) {
    PrefillLayout L{};
    const int G = num_q_heads / num_kv_heads;
    L.tile_tokens = tile_tokens_for(head_dim, G);
    L.max_tiles = total_query_tokens / L.tile_tokens + batch_size;
    L.plan = plan_decode(batch_size, num_kv_heads, max_blocks_per_req * block_size);
    size_t off = 0;
    L.counts_off = off;
    off = align256(off + 2 * sizeof(int32_t));
    L.zero_off = off;  // one all-zero K/V row (head_dim bf16), rewritten by the planner
    off = align256(off + static_cast<size_t>(head_dim) * 2);
    L.tiles_off = off;
    off = align256(off + static_cast<size_t>(L.max_tiles) * sizeof(TileEntry));
    L.dec_off = off;
    off = align256(off + static_cast<size_t>(batch_size) * sizeof(int32_t));
    L.decode_ws_off = off;
    off = align256(off + decode_workspace_bytes(batch_size, num_q_heads, head_dim, L.plan));
    L.total = off;
    return L;
}

template <int D>
hipError_t launch_tiles(const void* q, const void* k_cache, const void* v_cache,
                        const int32_t* block_table, const int32_t* qsl,
                        const int32_t* context_lens, void* output, int total_query_tokens,
                        int mbpr, int hq, int hkv, int block_size, const int32_t* counts,
                        const TileEntry* tiles, const void* zero_row, int max_tiles,
                        hipStream_t stream) {
    const int G = hq / hkv;
    const int U = hkv * (G / heads_per_wg(G));
    const int64_t grid = static_cast<int64_t>(max_tiles) * U;
    const float scale_log2 = kLog2e / sqrtf(static_cast<float>(D));
    prefill_tile_kernel<D><<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(
        static_cast<const __bf16*>(q), static_cast<const __bf16*>(k_cache),
        static_cast<const __bf16*>(v_cache), block_table, qsl, context_lens,
        static_cast<__bf16*>(output), counts, tiles, static_cast<const __bf16*>(zero_row),
        total_query_tokens, mbpr, hq, hkv, block_size, scale_log2);
    return hipGetLastError();
}

}  // namespace

bool prefill_fast_supported(int num_q_heads, int num_kv_heads, int head_dim,
                            int max_blocks_per_req) {
    if (num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0) return false;
    if (max_blocks_per_req > kMaxTableLds) return false;
    const int G = num_q_heads / num_kv_heads;
    return G <= 16 && (head_dim == 64 || head_dim == 128 || head_dim == 256);
}

size_t prefill_workspace_bytes(int batch_size, int total_query_tokens, int max_blocks_per_req,
                               int num_q_heads, int num_kv_heads, int head_dim,
                               int block_size) {
    return prefill_layout(batch_size, total_query_tokens, max_blocks_per_req, num_q_heads,
                          num_kv_heads, head_dim, block_size)
        .total;
}

hipError_t prefill_attention(const void* q, const void* k_cache, const void* v_cache,
                             const int32_t* block_table, const int32_t* query_start_loc,
                             const int32_t* context_lens, void* output, int batch_size,
                             int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                             int num_kv_heads, int head_dim, int block_size, void* workspace,
                             hipStream_t stream) {
    if (batch_size > kMaxPlanRequests) return hipErrorInvalidValue;
    const PrefillLayout L = prefill_layout(batch_size, total_query_tokens, max_blocks_per_req,
                                           num_q_heads, num_kv_heads, head_dim, block_size);
    char* ws = static_cast<char*>(workspace);
    int32_t* counts = reinterpret_cast<int32_t*>(ws + L.counts_off);
    TileEntry* tiles = reinterpret_cast<TileEntry*>(ws + L.tiles_off);
    int32_t* dec = reinterpret_cast<int32_t*>(ws + L.dec_off);
    uint32_t* zero_row = reinterpret_cast<uint32_t*>(ws + L.zero_off);
    prefill_plan_kernel<<<1, 1024, 0, stream>>>(query_start_loc, context_lens, batch_size,
                                                total_query_tokens, L.tile_tokens, counts, tiles,
                                                dec, zero_row, head_dim / 2);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    switch (head_dim) {
        case 64:
            err = launch_tiles<64>(q, k_cache, v_cache, block_table, query_start_loc,
                                   context_lens, output, total_query_tokens, max_blocks_per_req,
                                   num_q_heads, num_kv_heads, block_size, counts, tiles,
                                   zero_row, L.max_tiles, stream);
            break;
        case 128:
            err = launch_tiles<128>(q, k_cache, v_cache, block_table, query_start_loc,
                                    context_lens, output, total_query_tokens, max_blocks_per_req,
                                    num_q_heads, num_kv_heads, block_size, counts, tiles,
                                    zero_row, L.max_tiles, stream);
            break;
        case 256:
            err = launch_tiles<256>(q, k_cache, v_cache, block_table, query_start_loc,
                                    context_lens, output, total_query_tokens, max_blocks_per_req,
                                    num_q_heads, num_kv_heads, block_size, counts, tiles,
                                    zero_row, L.max_tiles, stream);
            break;
        default:
            return hipErrorInvalidValue;
    }
    if (err != hipSuccess) return err;
    // Single-token requests of a mixed batch: split-KV decode with prefill semantics.
    DecodeItems items;
    items.num_items = batch_size;
    items.item_count = counts + 1;
    items.item_req = dec;
    items.query_start_loc = query_start_loc;
    items.denom_eps = 0.0f;
    items.zero_invalid = false;
    return decode_attention(q, k_cache, v_cache, block_table, context_lens, output, items,
                            max_blocks_per_req, num_q_heads, num_kv_heads, head_dim, block_size,
                            L.plan, ws + L.decode_ws_off, stream);
}

}  // namespace ccinfer::hipk
