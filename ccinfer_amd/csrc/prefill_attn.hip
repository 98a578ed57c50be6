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
//   3. single-token requests run with prefill semantics (no 1e-6 in the denominator, bad
//      rows left untouched). Batches (bf16 or fp8) of at most 1024 (request, virtual kv head) groups with
//      table rows of at most 2048 positions run them in extra workgroups at the front of the
//      tile launch (the decode kernels' group body, decode_core.hpp): no further launch.
//      Others go through the split-KV decode kernels (decode_attn.hip): for batches of 32+
//      requests on the caller's side stream (when given) forked after the planner and
//      joined back at the end, so the memory-bound decode items run beside the MFMA-bound
//      tiles.
#include <type_traits>

#include "attn_common.hpp"
#include "decode_core.hpp"
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

// Inclusive prefix sum over the 64 lanes of a wavefront (shuffles, no LDS).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(v, off, 64);
        if (lane >= off) v += t;
    }
    return v;
}

// In-place inclusive prefix sum of a[0..n) (n <= 4 * blockDim.x) by a 1024-thread block.
// Each thread scans up to 4 consecutive entries; the per-thread totals are scanned within
// each wavefront by shuffles and across the 16 wavefronts through `part` (>= 16 ints).
// Must be called by every thread of the block.
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
    const int incl = wave_inclusive_scan(run);
    const int wave = tid >> 6;
    if ((tid & 63) == 63) part[wave] = incl;
    __syncthreads();
    if (tid < 64) {
        const int nw = nt >> 6;
        const int w = tid < nw ? part[tid] : 0;
        const int wi = wave_inclusive_scan(w);
        if (tid < nw) part[tid] = wi - w;  // exclusive offset of wavefront tid
    }
    __syncthreads();
    const int carry = part[wave] + incl - run;
    for (int x = lo; x < hi; ++x) a[x] += carry;
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Planner: one workgroup of 1024 threads.
// ws layout: counts[0] = #tiles, counts[1] = #decode items; tiles[max_tiles]; dec[B].
// split_dec: single-token requests become decode items (else one-row tiles).
// kBig: more than kMaxPlanRequests requests; the per-request arrays then live in the
// workspace (big_ntiles / big_scan, B ints each) instead of LDS.
// ---------------------------------------------------------------------------
template <bool kBig>
__global__ __launch_bounds__(1024) void prefill_plan_kernel(
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ context_lens, int batch_size,
    int total_tokens, int tile_tokens, int32_t* __restrict__ counts,
    TileEntry* __restrict__ tiles, int32_t* __restrict__ dec_req, uint32_t* __restrict__ zero_row,
    int zero_words, int* __restrict__ big_ntiles, int* __restrict__ big_scan, int split_dec) {
    __shared__ int lds_ntiles[kBig ? 1 : kMaxPlanRequests];
    __shared__ int lds_scan[kBig ? 1 : kMaxPlanRequests];
    // Each request's query length and cached prefix, read once (the bucket pass and the
    // scatter pass need them again).
    __shared__ int lds_qlen[kBig ? 1 : kMaxPlanRequests];
    __shared__ int lds_prefix[kBig ? 1 : kMaxPlanRequests];
    int* s_ntiles = kBig ? big_ntiles : lds_ntiles;
    int* s_scan = kBig ? big_scan : lds_scan;
    __shared__ int s_hist[kBuckets];
    __shared__ int s_hscan[kBuckets];
    __shared__ int s_part[16];
    __shared__ int s_ndec;
    __shared__ int s_total;
    const int tid = threadIdx.x;
    for (int i = tid; i < zero_words; i += blockDim.x) zero_row[i] = 0u;  // staging's zero row
    for (int i = tid; i < kBuckets; i += blockDim.x) s_hist[i] = 0;
    if (tid == 0) s_ndec = 0;
    __syncthreads();

    // Per-request tile counts; single-token requests become decode items, listed in request
    // order (a block-wide compaction per round of blockDim.x requests), so the decode plan
    // built from the list -- and with it the output bits -- is the same on every run.
    for (int b0 = 0; b0 < batch_size; b0 += blockDim.x) {
        const int b = b0 + tid;
        int isdec = 0;
        if (b < batch_size) {
        const int qb = qsl[b];
        const int qe_raw = qsl[b + 1];
        const int qlen = qe_raw - qb;
        const int qe = qe_raw < total_tokens ? qe_raw : total_tokens;
        const int rows = qe - (qb > 0 ? qb : 0);
        const int prefix = context_lens[b] - qlen;
        if constexpr (!kBig) {
            lds_qlen[b] = qlen;
            lds_prefix[b] = prefix;
        }
        int n = 0;
        if (qlen > 0 && prefix >= 0 && qb >= 0 && rows > 0) {
            if (qlen == 1 && split_dec)
                isdec = 1;
            else
                n = (rows + tile_tokens - 1) / tile_tokens;
        }
        s_ntiles[b] = n;
        }
        const int wave = tid >> 6;
        const int incl = wave_inclusive_scan(isdec);
        if ((tid & 63) == 63) s_part[wave] = incl;
        __syncthreads();
        int base = s_ndec;
        int round = 0;
        for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) {
            const int pw = s_part[w];
            if (w < wave) base += pw;
            round += pw;
        }
        if (isdec) dec_req[base + incl - 1] = b;
        __syncthreads();  // every thread has read s_ndec and s_part
        if (tid == 0) s_ndec += round;
        __syncthreads();
    }
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
        const int qlen = kBig ? qsl[b + 1] - qsl[b] : lds_qlen[b];
        const int prefix = kBig ? context_lens[b] - qlen : lds_prefix[b];
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
template <int D>
__device__ __forceinline__ int chunk_swizzle(int row) {
    if constexpr (D == 128)
        return 4 * (row & 3) + 2 * ((row >> 2) & 1) + ((row >> 3) & 1);
    else
        return row & 15;
}

template <int D>
__device__ __forceinline__ int lds_off(int row, int chunk) {
    // Element offset of logical 16-byte chunk `chunk` of key row `row`.
    constexpr int kMask = PrefillShape<D>::kCPR - 1;
    return row * D + ((chunk ^ (chunk_swizzle<D>(row) & kMask)) << 3);
}

// Direct global->LDS staging of one 64-key K/V tile (gfx950 global_load_lds_dwordx4): an
// instruction moves 16 bytes per lane straight into LDS at base + 16*lane, so the chunk
// swizzle is applied on the source side: LDS slot p holds row p/CPR, logical chunk
// (p%CPR) ^ swizzle(row). Rows outside the visible range (past the context, negative block
// ids, past the table row) are fetched from `zero_row` so the tile never holds garbage that
// a masked probability of 0 could turn into NaN. Validity flags go to lvalid[row].
// kPad: cache rows hold dr < D dims (a multiple of 8); chunks past dr come from zero_row.
template <int D, bool kPad = false>
__device__ __forceinline__ void stage_issue(__bf16* lk, __bf16* lv, uint8_t* lvalid,
                                            const __bf16* __restrict__ k_cache,
                                            const __bf16* __restrict__ v_cache,
                                            const __bf16* __restrict__ zero_row,
                                            const int32_t* lbt, int key_base, int ctx, int nblk,
                                            int kv_head, int hkv, int dr = D) {
    constexpr int CPR = PrefillShape<D>::kCPR;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int x = 0; x < PrefillShape<D>::kLoadsPerThread; ++x) {
        const int slot0 = (x * kWaves + wave) * 64;  // first 16-byte LDS slot of this load
        const int p = slot0 + lane;
        const int row = p / CPR;
        const int lchunk = (p % CPR) ^ (chunk_swizzle<D>(row) & (CPR - 1));
        const int key = key_base + row;
        const int lb = key >> 4;
        int pb = -1;
        if (key < ctx && lb < nblk) pb = lbt[lb];
        const __bf16* ks = zero_row;
        const __bf16* vs = zero_row;
        if (pb >= 0 && (!kPad || lchunk * 8 < dr)) {
            const int64_t base =
                ((static_cast<int64_t>(pb) * kBlock + (key & (kBlock - 1))) * hkv + kv_head) *
                (kPad ? dr : D);
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

// Any-layout staging (cache rows of any 2-byte alignment, blocks of any size `bs`, any
// head dim dr <= D): the same tile layout as stage_issue, built in two steps so the loads'
// latency overlaps the attention of the current tile -- stage_any_load reads each lane's
// 16-byte chunk element by element (elements past dr, rows past the context or in
// unmapped blocks read as zeros; one 16-byte load when `vec`: rows 16-byte aligned; two
// shifted 16-byte loads for other chunks that lie wholly inside their row; 2-byte elements
// for a row's last, partial chunk) and records the rows' validity; stage_any_write stores
// the chunks into the tile.
template <int D>
struct AnyStage {
    u32x4 k[PrefillShape<D>::kLoadsPerThread];
    u32x4 v[PrefillShape<D>::kLoadsPerThread];
};

template <int D>
__device__ __forceinline__ void stage_any_load(AnyStage<D>& r, uint8_t* lvalid,
                                               const __bf16* k_cache, const __bf16* v_cache,
                                               const int32_t* lbt, int key_base, int ctx,
                                               int nblk, int kv_head, int hkv, int dr, int bs,
                                               bool vec) {
    constexpr int CPR = PrefillShape<D>::kCPR;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int x = 0; x < PrefillShape<D>::kLoadsPerThread; ++x) {
        const int p = (x * kWaves + wave) * 64 + lane;
        const int row = p / CPR;
        const int lchunk = (p % CPR) ^ (chunk_swizzle<D>(row) & (CPR - 1));
        const int key = key_base + row;
        const int lb = key / bs;
        int pb = -1;
        if (key < ctx && lb < nblk) pb = lbt[lb];
        const int64_t base =
            ((static_cast<int64_t>(pb < 0 ? 0 : pb) * bs + key % bs) * hkv + kv_head) * dr;
        const uint16_t* ks = reinterpret_cast<const uint16_t*>(k_cache) + base;
        const uint16_t* vs = reinterpret_cast<const uint16_t*>(v_cache) + base;
        u32x4 kw{0u, 0u, 0u, 0u}, vw{0u, 0u, 0u, 0u};
        if (vec) {
            // 16-byte aligned rows of a multiple of 8 elements: one load per chunk
            if (pb >= 0 && lchunk * 8 < dr) {
                kw = *reinterpret_cast<const u32x4*>(ks + lchunk * 8);
                vw = *reinterpret_cast<const u32x4*>(vs + lchunk * 8);
            }
        } else if (pb >= 0 && lchunk * 8 + 8 <= dr) {
            // a chunk wholly inside its row: two aligned loads shifted into place
            kw = load_shifted<4, u32x4>(ks + lchunk * 8);
            vw = load_shifted<4, u32x4>(vs + lchunk * 8);
        } else if (pb >= 0) {
            // the row's last, partial chunk: element by element
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = lchunk * 8 + i;
                if (e < dr) {
                    kw[i >> 1] |= static_cast<uint32_t>(ks[e]) << (16 * (i & 1));
                    vw[i >> 1] |= static_cast<uint32_t>(vs[e]) << (16 * (i & 1));
                }
            }
        }
        r.k[x] = kw;
        r.v[x] = vw;
        if ((p % CPR) == 0) lvalid[row] = static_cast<uint8_t>(pb >= 0);
    }
}

template <int D>
__device__ __forceinline__ void stage_any_write(const AnyStage<D>& r, __bf16* lk, __bf16* lv) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int x = 0; x < PrefillShape<D>::kLoadsPerThread; ++x) {
        const int p = (x * kWaves + wave) * 64 + lane;
        *reinterpret_cast<u32x4*>(lk + p * 8) = r.k[x];
        *reinterpret_cast<u32x4*>(lv + p * 8) = r.v[x];
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
constexpr float kMaxInit = -1.0e30f;

// kPad: q / cache / output rows hold dr < D dims; the kernel runs at D with the missing dims
// zero. kAny: any layout -- rows of any head dim dr <= D and any 2-byte alignment, cache
// blocks of `block_size` tokens -- through element-wise staging (stage_any_*), Q loads and
// output stores.
template <int D, bool kPad = false, bool kAny = false>
__global__ __launch_bounds__(kThreads) void prefill_tile_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k_cache,
    const __bf16* __restrict__ v_cache, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ context_lens,
    __bf16* __restrict__ out, const int32_t* __restrict__ counts,
    const TileEntry* __restrict__ tiles, const __bf16* __restrict__ zero_row, int total_tokens,
    int mbpr, int hq, int hkv, int block_size, float scale_log2, int dr) {
    if constexpr (!kAny) block_size = kBlock;  // the fast path is specialised for 16-token blocks
    // kAny: rows 16-byte aligned (cache pointers aligned, dr a multiple of 8) load whole chunks
    [[maybe_unused]] const bool any_vec =
        kAny && dr % 8 == 0 &&
        ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15u) == 0;
    const int ds = (kPad || kAny) ? dr : D;  // row stride of q / cache / output (elements)
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
        const __bf16* qv = q + (static_cast<int64_t>(qb + (live ? tq : 0)) * hq + q_head) * ds;
#pragma unroll
        for (int kk = 0; kk < S; ++kk) {
            u32x4 w = u32x4{0, 0, 0, 0};
            if constexpr (kAny) {
                const uint16_t* qe = reinterpret_cast<const uint16_t*>(qv);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int e = (kk * 4 + g) * 8 + i;
                    if (e < dr) w[i >> 1] |= static_cast<uint32_t>(qe[e]) << (16 * (i & 1));
                }
            } else {
                const bool ok = !kPad || (kk * 4 + g) * 8 < dr;
                w = load16(qv + (ok ? (kk * 4 + g) * 8 : 0));
                if (!ok) w = u32x4{0, 0, 0, 0};
            }
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
    // the host sends the native tile kernel table rows of at most kMaxTableLds blocks.
    const int nblk_vis = (kv_end + block_size - 1) / block_size;
    const int nblk = min(nblk_vis, mbpr);
    // kAny with more visible blocks than the LDS table holds: the staging reads the ids
    // from the table row in global memory instead (cached; one read per staged chunk).
    const bool bt_global = kAny && nblk > kMaxTableLds;
    for (int lb = threadIdx.x; lb < nblk; lb += kThreads) {
        const int pb = req_blocks[lb];
        if (!bt_global) lds_bt[lb] = pb;
        if (pb < 0) s_holes = 1;
    }
    __syncthreads();
    const bool holes = s_holes != 0 || nblk_vis > mbpr;
    [[maybe_unused]] const int32_t* stage_bt = bt_global ? req_blocks : lds_bt;

    if constexpr (kAny) {
        AnyStage<D> r0;
        stage_any_load<D>(r0, lds_valid0, k_cache, v_cache, stage_bt, 0, ctx, nblk, kvh, hkv, dr,
                          block_size, any_vec);
        stage_any_write<D>(r0, lds_k0, lds_v0);
    } else {
        stage_issue<D, kPad>(lds_k0, lds_v0, lds_valid0, k_cache, v_cache, zero_row, lds_bt, 0,
                             ctx, nblk, kvh, hkv, dr);
        __builtin_amdgcn_s_waitcnt(0);  // this wavefront's direct-to-LDS loads have landed
    }
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
        [[maybe_unused]] AnyStage<D> rn;
        if (more) {
            if constexpr (kAny)
                stage_any_load<D>(rn, nvalid, k_cache, v_cache, stage_bt, (t + 1) * kKeysPerTile,
                                  ctx, nblk, kvh, hkv, dr, block_size, any_vec);
            else
                stage_issue<D, kPad>(nk, nv, nvalid, k_cache, v_cache, zero_row, lds_bt,
                                     (t + 1) * kKeysPerTile, ctx, nblk, kvh, hkv, dr);
        }
        const int key0 = t * kKeysPerTile;
        if (key0 <= wave_max_key) {
            const uint64_t vmask = decltype(mask_tag)::value
                                       ? __builtin_amdgcn_ballot_w64(cvalid[lane] != 0)
                                       : ~0ull;
            attend_tile(ck, cv, vmask, key0, mask_tag);
        }
        if constexpr (kAny) {
            if (more) stage_any_write<D>(rn, nk, nv);
        } else {
            if (more) __builtin_amdgcn_s_waitcnt(0);  // next tile resident before the barrier
        }
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
        __bf16* o = out + (static_cast<int64_t>(qb + tq) * hq + q_head) * ds;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            if constexpr (kAny) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (16 * n + 4 * g + r < dr)
                        reinterpret_cast<uint16_t*>(o)[16 * n + 4 * g + r] =
                            static_cast<uint16_t>(pack_bf16x2(acc[qt][n][r] * inv, 0.f));
                continue;
            }
            if (kPad && 16 * n + 4 * g >= dr) continue;  // padded dims
            u32x2 w;
            w[0] = pack_bf16x2(acc[qt][n][0] * inv, acc[qt][n][1] * inv);
            w[1] = pack_bf16x2(acc[qt][n][2] * inv, acc[qt][n][3] * inv);
            *reinterpret_cast<u32x2*>(o + 16 * n + 4 * g) = w;
        }
    }
}

// ---------------------------------------------------------------------------
// Pipelined tile kernel (head_dim 64 / 128).
//
// One workgroup = 8 wavefronts (two per SIMD, <= 256 VGPRs each); each wavefront owns 32
// query rows of one q-head and the workgroup covers the Hq/Hkv heads that share a KV head,
// so every K/V tile staged in LDS feeds all of them. The matrix work uses the 32x32x16 bf16
// MFMA: per 32-key half, S^T = K . Q^T is one 32x32 accumulator (keys x query rows) and
// O^T += V^T . P^T runs over D/32 dim tiles x 2 key steps. Per MFMA the 32x32x16 shape
// leaves twice the VALU issue room of the 16x16x32 one, which the softmax needs. Work
// advances in 32-key halves through a software pipeline so that each wavefront always has
// independent MFMA and VALU work:
//     X_i: P_i (first key step) = exp2(S_i * scale - m)  ||  S_{i+1} = K_{i+1} . Q^T
//     Y_i: O += V_i^T . P_i^T, with the second key step's exp beside the first PV MFMAs
//                                                         ||  row max of S_{i+1}
// with the instruction interleave pinned by sched_group_barrier. Masked halves seed the
// S accumulator with 0 / -inf instead of masking the scores afterwards. K/V tiles are
// triple-buffered in LDS: at the barrier in the middle of tile t every wavefront has
// finished tile t-1 and tile t+1 has landed, so tile t+2 streams into the freed buffer
// while tiles t and t+1 are read.
// ---------------------------------------------------------------------------
template <int D>
struct PipeShape {
    static constexpr int kRows = 32;                     // query rows per wavefront
    static constexpr int kWaves = 8;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kCPR = D / 8;                   // 16-byte chunks per K/V row
    static constexpr int kLoads = kKeysPerTile * kCPR / kThreads;  // per K or V
    static_assert(kKeysPerTile * kCPR % kThreads == 0, "staging must split evenly");
};

__host__ __device__ constexpr bool pipe_head_dim(int d) { return d == 64 || d == 128; }

// F8: the cache holds OCP E4M3 bytes with row scales (k_scale / v_scale). Tiles are then
// staged as bytes into a two-tile ring and dequantised (byte * row scale, rounded to bf16)
// into a two-tile ring of bf16 tiles in the same swizzled layout, so everything after the
// staging is the bf16 kernel.
// kPad (bf16 only): q / cache / output rows hold dr < D dims (a multiple of 8). Staging
// fetches chunk 0 of the row again in place of the missing chunks (finite values: the Q
// operand is zero in those dims, so they add exactly 0 to the scores), and the missing
// output dims are not stored.
template <int D, bool F8 = false, bool kPad = false>
__global__ __launch_bounds__((PipeShape<D>::kThreads))
void prefill_pipe_kernel(const __bf16* __restrict__ q, const void* __restrict__ k_cache_v,
                         const void* __restrict__ v_cache_v, const float* __restrict__ k_scale,
                         const float* __restrict__ v_scale,
                         const int32_t* __restrict__ block_table,
                         const int32_t* __restrict__ qsl,
                         const int32_t* __restrict__ context_lens, __bf16* __restrict__ out,
                         const int32_t* __restrict__ counts, const TileEntry* __restrict__ tiles,
                         int total_tokens, int mbpr, int hq, int hkv, float scale_log2,
                         int dr, dcore::ItemArgs dec_items, int dec_wgs, int dec_hkv,
                         int dec_rep) {
    static_assert(!(F8 && kPad), "fp8 runs the native head dims only");
    const int ds = kPad ? dr : D;  // row stride of q / cache / output (elements)
    using Sh = PipeShape<D>;
    constexpr int S2 = D / 16;   // QK k-steps (32x32x16 MFMA)
    constexpr int NT2 = D / 32;  // PV dim tiles
    constexpr int CPR = Sh::kCPR;
    constexpr int NL = Sh::kLoads;
    constexpr int kPipeWaves = Sh::kWaves;
    constexpr int kPipeThreads = Sh::kThreads;
    constexpr int kPipeRows = Sh::kRows;
    const __bf16* __restrict__ k_cache = static_cast<const __bf16*>(k_cache_v);
    const __bf16* __restrict__ v_cache = static_cast<const __bf16*>(v_cache_v);
    // Three K/V buffers as distinct arrays (see prefill_tile_kernel: the compiler then knows
    // the direct-to-LDS loads into one buffer never alias reads of another). fp8 uses two
    // bf16 buffers plus two byte-staging buffers.
    constexpr int kTileElems = kKeysPerTile * D;
    constexpr int kBuf2 = F8 ? 8 : kTileElems;
    constexpr int kF8Bytes = F8 ? kTileElems : 16;
    __shared__ __attribute__((aligned(16))) __bf16 lds_k0[kTileElems];
    __shared__ __attribute__((aligned(16))) __bf16 lds_k1[kTileElems];
    __shared__ __attribute__((aligned(16))) __bf16 lds_k2[kBuf2];
    __shared__ __attribute__((aligned(16))) __bf16 lds_v0[kTileElems];
    __shared__ __attribute__((aligned(16))) __bf16 lds_v1[kTileElems];
    __shared__ __attribute__((aligned(16))) __bf16 lds_v2[kBuf2];
    __shared__ __attribute__((aligned(16))) uint8_t lds_k8_0[kF8Bytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds_k8_1[kF8Bytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds_v8_0[kF8Bytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds_v8_1[kF8Bytes];
    __shared__ uint8_t lds_valid0[kKeysPerTile];
    __shared__ uint8_t lds_valid1[kKeysPerTile];
    __shared__ uint8_t lds_valid2[kKeysPerTile];
    // The block table in LDS (fp8 staging only; the bf16 staging reads its block ids from
    // global memory into a register window).
    __shared__ int32_t lds_bt[F8 ? kMaxTableLds : 1];
    __shared__ int s_holes[kPipeWaves];

    // The first dec_wgs workgroups run the batch's single-token requests instead: one per
    // (request, virtual kv head), the decode kernels' group body with prefill semantics,
    // its partial rows in four of the bf16 K/V buffers (two wavefronts' 16 x D floats per
    // buffer) and its (m, l) pairs in a fifth buffer.
    if (static_cast<int>(blockIdx.x) < dec_wgs) {
        static_assert(dcore::GroupShape<D>::kWaves == kPipeWaves &&
                          kTileElems * 2 >= 2 * dcore::GroupShape<D>::kMaxG * D * 4 &&
                          (F8 ? kF8Bytes : kTileElems * 2) >= 2 * kPipeWaves * 16 * 4,
                      "the group body's partial rows fit two per K/V buffer");
        auto part = [&](int w) {
            __bf16* b;
            if constexpr (F8)
                b = w < 2 ? lds_k0 : w < 4 ? lds_k1 : w < 6 ? lds_v0 : lds_v1;
            else
                b = w < 2 ? lds_k0 : w < 4 ? lds_k1 : w < 6 ? lds_k2 : lds_v0;
            return reinterpret_cast<float*>(b) + (w & 1) * dcore::GroupShape<D>::kMaxG * D;
        };
        float* lm = F8 ? reinterpret_cast<float*>(lds_k8_0) : reinterpret_cast<float*>(lds_v1);
        dcore::decode_group_body<D, F8, kPad, true, 0>(
            q, const_cast<void*>(k_cache_v), const_cast<void*>(v_cache_v), k_scale, v_scale,
            block_table, context_lens, out, dec_items, mbpr, hq, dec_hkv, scale_log2, dr,
            dec_rep, static_cast<int>(blockIdx.x), part, lm,
            lm + kPipeWaves * dcore::GroupShape<D>::kMaxG);
        return;
    }
    const int bid = static_cast<int>(blockIdx.x) - dec_wgs;
    const int G = hq / hkv;
    const int HPW = heads_per_wg(G);
    const int WPH = kPipeWaves / HPW;
    const int U = hkv * (G / HPW);
    const int tile_idx = bid / U;
    if (tile_idx >= counts[0]) return;
    const int u = bid % U;
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
    const int rows = qe - qb;
    const int TT = WPH * kPipeRows;
    const int kv_end = prefix + min(t0 + TT, rows);  // keys past it are masked for every row
    // Positions past the table row are invalid: no tile needs to reach them.
    const int kv_lim = min(kv_end, mbpr * kBlock);
    const int ntiles = (kv_lim + kKeysPerTile - 1) / kKeysPerTile;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int head_local = wave / WPH;
    const int tw = t0 + (wave % WPH) * kPipeRows;
    const int q_head = kvh * G + hg * HPW + head_local;
    const int32_t* req_blocks = block_table + static_cast<int64_t>(req) * mbpr;

    const int nblk_vis = (kv_end + kBlock - 1) / kBlock;
    const int nblk = min(nblk_vis, mbpr);
    // Block ids this wavefront stages, held in one register: lane i has the id of load
    // i % NL's cache block in tile kWin * bt_win + i / NL (-1 past the visible table). A
    // stage reads its ids with readlane; the window is reloaded from the table row every
    // kWin tiles, so the table length is not bounded by LDS.
    constexpr int kWin = 64 / NL;
    int btw;
    int bt_win = -1;
    auto bt_window = [&](int win) __attribute__((always_inline)) {
        const int x = lane % NL;
        const int blk = ((x * kPipeWaves + wave) * 64 / CPR) >> 4;
        const int lb = (win * kWin + lane / NL) * (kKeysPerTile / kBlock) + blk;
        btw = lb < nblk ? req_blocks[lb] : -1;
        bt_win = win;
    };
    // The first window's load goes out before the table scan below, so the two overlap.
    if constexpr (!F8) bt_window(0);

    // Block-table slice in LDS (fp8): entries for every block the tiles touch, -1 past the
    // visible range or the table row. Holes (negative ids inside the visible range, or a
    // visible range longer than the row) force the masked path on every tile; each
    // wavefront records whether its share of the scan found one.
    // Block ids whose byte offset does not fit the 32-bit buffer offset of the fast staging
    // path are treated like holes (the checked path addresses with 64 bits).
    const int max_fast_pb = static_cast<int>(
        min(static_cast<int64_t>(0x7fffffff),
            static_cast<int64_t>(0xffffffffll / (static_cast<int64_t>(kBlock) * hkv * ds * 2)) - 1));
    bool bad = false;
    for (int lb = threadIdx.x; lb < (F8 ? ntiles * (kKeysPerTile / kBlock) : nblk);
         lb += kPipeThreads) {
        const int pb = lb < nblk ? req_blocks[lb] : -1;
        if constexpr (F8) lds_bt[lb] = pb;
        bad = bad || (lb < nblk && (pb < 0 || pb > max_fast_pb));
    }
    {
        const bool any = __builtin_amdgcn_ballot_w64(bad) != 0;
        if (lane == 0) s_holes[wave] = any ? 1 : 0;
    }

    // Staging constants. Load x of a wavefront fills the 64 16-byte LDS slots starting at
    // slot0 = (x * waves + wave) * 64: rows slot0/CPR .. +64/CPR-1, which lie in one 16-row
    // cache block, so the block id is wave-uniform and each address is a scalar block base
    // plus this lane's 32-bit byte offset inside the block (row-in-block, kv head, chunk,
    // with the LDS chunk swizzle applied on the source side).
    int st_row[NL];
    uint32_t st_off[NL];
#pragma unroll
    for (int x = 0; x < NL; ++x) {
        const int p = (x * kPipeWaves + wave) * 64 + lane;
        const int row = p / CPR;
        const int lch = (p % CPR) ^ (chunk_swizzle<D>(row) & (CPR - 1));
        st_row[x] = row;
        const int src = kPad && lch * 8 >= dr ? 0 : lch * 8;
        st_off[x] = static_cast<uint32_t>((((row & (kBlock - 1)) * hkv + kvh) * ds + src) * 2);
    }
    const int64_t blk_bytes = static_cast<int64_t>(kBlock) * hkv * ds * 2;

    // Per-lane LDS read offsets (elements); lane l = 32 h + c (c = l % 32, h = l / 32).
    // K operand of k-step kk: key row c, logical chunk 2 kk + h. Rows 16 apart share a
    // swizzle, so one offset per k-step serves both 32-key halves and every buffer.
    // V^T operand of dim tile n, k-step s: two transposing reads, of key rows
    // 16 s + 4 h + (c%16)/4 and 8 rows further, dims 32 n + 16 (c/16) + 4 (c%4) .. +3 (the
    // 16-lane group's 4 x 16 block, transposed so lane c receives one dim for 4 keys).
    const int c32 = lane & 31;
    const int h32 = lane >> 5;
    int koff[S2];
#pragma unroll
    for (int kk = 0; kk < S2; ++kk) koff[kk] = lds_off<D>(c32, kk * 2 + h32);
    int voffa[NT2], voffb[NT2];
    {
        const int s16 = lane & 15;
        const int row0 = 4 * h32 + (s16 >> 2);
#pragma unroll
        for (int n = 0; n < NT2; ++n) {
            const int dim = 32 * n + 16 * ((lane >> 4) & 1) + 4 * (s16 & 3);
            voffa[n] = lds_off<D>(row0, dim >> 3) + (dim & 7);
            voffb[n] = lds_off<D>(row0 + 8, dim >> 3) + (dim & 7);
        }
    }

    // Rows past kv_end or in unmapped blocks are not loaded: their LDS slots are written with
    // zeros instead, and the mask gives them probability 0.
#if defined(__HIP_DEVICE_COMPILE__)
    // (device pass only: the host pass cannot type the buffer builtins, and a kernel
    // template that fails there loses its launch stub silently)
    const __amdgpu_buffer_rsrc_t k_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)k_cache, 0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t v_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)v_cache, 0, -1, 0x00020000);
#endif
    // kHoles: the table has holes in the visible range; then every tile goes through the
    // checked path, which also records per-row validity for the mask. Otherwise only a tile
    // that reaches past kv_end does (its rows past kv_end are zero-filled).
    auto stage = [&](int t, __bf16* lk, __bf16* lv, uint8_t* lvalid, auto holes_tag)
                     __attribute__((always_inline)) {
        constexpr bool kHoles = decltype(holes_tag)::value;
        const int key_base = t * kKeysPerTile;
        if (t / kWin != bt_win) bt_window(t / kWin);  // wave-uniform, once per kWin tiles
#if defined(__HIP_DEVICE_COMPILE__)
        if (!kHoles && key_base + kKeysPerTile <= kv_end) {
            // Buffer loads: the block's byte offset is the scalar offset, the lane's offset
            // inside the block the vector offset (every id here fits 32 bits, see above).
#pragma unroll
            for (int x = 0; x < NL; ++x) {
                const int slot0 = (x * kPipeWaves + wave) * 64;
                const int pb = __builtin_amdgcn_readlane(btw, (t % kWin) * NL + x);
                const int soff = pb * static_cast<int>(blk_bytes);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    k_rsrc, (__attribute__((address_space(3))) void*)(lk + slot0 * 8), 16,
                    st_off[x], soff, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    v_rsrc, (__attribute__((address_space(3))) void*)(lv + slot0 * 8), 16,
                    st_off[x], soff, 0, 0);
            }
            return;
        }
#endif
#pragma unroll
        for (int x = 0; x < NL; ++x) {
            const int slot0 = (x * kPipeWaves + wave) * 64;
            const int row = st_row[x];
            const int pb = __builtin_amdgcn_readlane(btw, (t % kWin) * NL + x);
            const bool in_range = key_base + row < kv_end;
            if (pb >= 0) {
                const int64_t boff = static_cast<int64_t>(pb) * blk_bytes;
                const char* kb = reinterpret_cast<const char*>(k_cache) + boff;
                const char* vb = reinterpret_cast<const char*>(v_cache) + boff;
                // Opaque scalar bases: keeps the address as SGPR base + 32-bit lane offset
                // (otherwise the compiler hoists 64-bit per-lane sums out of the loop).
                asm("" : "+s"(kb), "+s"(vb));
                if (in_range) {
                    __builtin_amdgcn_global_load_lds(
                        (void*)(kb + st_off[x]),  // a char* argument makes clang drop the
                                                  // kernel's host launch stub silently
                        (__attribute__((address_space(3))) void*)(lk + slot0 * 8), 16, 0, 0);
                    __builtin_amdgcn_global_load_lds(
                        (void*)(vb + st_off[x]),
                        (__attribute__((address_space(3))) void*)(lv + slot0 * 8), 16, 0, 0);
                }
            }
            // Slots not loaded get zeros (LDS holds undefined bits at workgroup start; the
            // mask gives these rows probability 0, and 0 * V must stay finite).
            if (!(pb >= 0 && in_range)) {
                *reinterpret_cast<u32x4*>(lk + (slot0 + lane) * 8) = u32x4{0, 0, 0, 0};
                *reinterpret_cast<u32x4*>(lv + (slot0 + lane) * 8) = u32x4{0, 0, 0, 0};
            }
            if (kHoles && ((slot0 + lane) % CPR) == 0)
                lvalid[row] = static_cast<uint8_t>(pb >= 0 && in_range);
        }
    };

    // ---- fp8 staging: tile t's bytes (16 per lane, linear in LDS) and its row scales ----
    // Thread p (< kCh8) later converts 16-byte chunk p of the tile: row p / CPR8, dims
    // 16 (p % CPR8) .. +16; it also fetches that row's two scales when the tile is staged.
    constexpr int CPR8 = D / 16;
    constexpr int kCh8 = kKeysPerTile * CPR8;
    constexpr int NL8 = (kCh8 + kPipeThreads - 1) / kPipeThreads;
    const uint8_t* __restrict__ k_cache8 = static_cast<const uint8_t*>(k_cache_v);
    const uint8_t* __restrict__ v_cache8 = static_cast<const uint8_t*>(v_cache_v);
    const int64_t blk_bytes8 = static_cast<int64_t>(kBlock) * hkv * D;
    auto stage8 = [&](int t, uint8_t* lk8, uint8_t* lv8, uint8_t* lvalid, float& sk, float& sv)
                      __attribute__((always_inline)) {
        const int key_base = t * kKeysPerTile;
#pragma unroll
        for (int x = 0; x < NL8; ++x) {
            const int slot0 = (x * kPipeWaves + wave) * 64;
            if (slot0 >= kCh8) break;  // wave-uniform
            const int p = slot0 + lane;
            const int row = p / CPR8;
            const int pb = __builtin_amdgcn_readfirstlane(
                lds_bt[t * (kKeysPerTile / kBlock) + ((slot0 / CPR8) >> 4)]);
            const bool in_range = key_base + row < kv_end;
            if (pb >= 0 && in_range) {
                const int64_t off = static_cast<int64_t>(pb) * blk_bytes8 +
                                    ((row & (kBlock - 1)) * hkv + kvh) * D + (p % CPR8) * 16;
                __builtin_amdgcn_global_load_lds(
                    (void*)(k_cache8 + off),
                    (__attribute__((address_space(3))) void*)(lk8 + slot0 * 16), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(
                    (void*)(v_cache8 + off),
                    (__attribute__((address_space(3))) void*)(lv8 + slot0 * 16), 16, 0, 0);
            }
            if (!(pb >= 0 && in_range)) {  // zero bytes: row scale 0 must give 0, not NaN
                *reinterpret_cast<u32x4*>(lk8 + (slot0 + lane) * 16) = u32x4{0, 0, 0, 0};
                *reinterpret_cast<u32x4*>(lv8 + (slot0 + lane) * 16) = u32x4{0, 0, 0, 0};
            }
            if ((p % CPR8) == 0) lvalid[row] = static_cast<uint8_t>(pb >= 0 && in_range);
        }
        sk = 0.f;
        sv = 0.f;
        if (static_cast<int>(threadIdx.x) < kCh8) {
            const int row = threadIdx.x / CPR8;
            const int pb = lds_bt[t * (kKeysPerTile / kBlock) + (row >> 4)];
            if (pb >= 0 && key_base + row < kv_end) {
                const int64_t si = (static_cast<int64_t>(pb) * hkv + kvh) * kBlock + (row & 15);
                sk = k_scale[si];
                sv = v_scale[si];
            }
        }
    };
    // Bytes of one staged tile -> bf16 tile (byte * row scale, rounded to bf16), written in
    // the swizzled layout the operand reads expect. A row whose scale is a normal power of
    // two (what the fp8 write stores) converts in one instruction per byte pair: the
    // hardware's scaled conversion applies exactly the exponent of its scale operand, and
    // byte * 2^e is exact in bf16. Any other scale takes the general path.
    auto convert8 = [&](const uint8_t* lk8, const uint8_t* lv8, __bf16* lk, __bf16* lv,
                        float sk, float sv) __attribute__((always_inline)) {
        const int p = threadIdx.x;
        if (p >= kCh8) return;
        const int row = p / CPR8;
        const int c = p % CPR8;
        auto deq = [&](const uint8_t* src, __bf16* dst, float sc) __attribute__((always_inline)) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(src + p * 16);
            u32x4 o[2];
            const uint32_t sb = __float_as_uint(sc);
            if ((sb & 0x007fffffu) == 0u && (sb & 0x7f800000u) != 0u) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    o[i >> 1][(i & 1) * 2] = e4m3x2_to_bf16x2<false>(w[i], sc);
                    o[i >> 1][(i & 1) * 2 + 1] = e4m3x2_to_bf16x2<true>(w[i], sc);
                }
                *reinterpret_cast<u32x4*>(dst + lds_off<D>(row, 2 * c)) = o[0];
                *reinterpret_cast<u32x4*>(dst + lds_off<D>(row, 2 * c + 1)) = o[1];
                return;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = e4m3x2_to_bf16x2<false>(w[i]);
                const uint32_t hi = e4m3x2_to_bf16x2<true>(w[i]);
                o[i >> 1][(i & 1) * 2] =
                    pack_bf16x2(__uint_as_float(lo << 16) * sc, __uint_as_float(lo & 0xffff0000u) * sc);
                o[i >> 1][(i & 1) * 2 + 1] =
                    pack_bf16x2(__uint_as_float(hi << 16) * sc, __uint_as_float(hi & 0xffff0000u) * sc);
            }
            *reinterpret_cast<u32x4*>(dst + lds_off<D>(row, 2 * c)) = o[0];
            *reinterpret_cast<u32x4*>(dst + lds_off<D>(row, 2 * c + 1)) = o[1];
        };
        deq(lk8, lk, sk);
        deq(lv8, lv, sv);
    };
    float sk8[2] = {0.f, 0.f}, sv8[2] = {0.f, 0.f};  // scales of the tiles staged in ring slot

    // Q^T operands: lane (c, h) holds dims 16 kk + 8 h .. +8 of query row tw + c.
    bf16x8 qop[S2];
    {
        const int tq = tw + c32;
        const bool live = tq < rows;
        const __bf16* qv = q + (static_cast<int64_t>(qb + (live ? tq : 0)) * hq + q_head) * ds;
#pragma unroll
        for (int kk = 0; kk < S2; ++kk) {
            // rows past the tile's end read row 0 (finite) and are never stored
            const bool ok = !kPad || kk * 16 + h32 * 8 < dr;
            u32x4 w = load16(qv + (ok ? kk * 16 + h32 * 8 : 0));
            if (!ok) w = u32x4{0, 0, 0, 0};
            qop[kk] = __builtin_bit_cast(bf16x8, w);
        }
    }
    __syncthreads();  // block table scanned (and, for fp8, staged)
    bool any_hole = false;
#pragma unroll
    for (int w = 0; w < kPipeWaves; ++w) any_hole = any_hole || s_holes[w] != 0;
    const bool holes = any_hole || nblk_vis > mbpr;

    // O^T: lane (c, h), element v of dim tile n holds dim 32 n + 8 (v/4) + 4 h + v%4 of
    // query row tw + c. lsum: this lane's share of the row sum of query row tw + c (the
    // bf16 probabilities it holds); lanes c and c + 32 together hold the whole sum.
    f32x16 acc[NT2];
    float lsum = 0.f;
    // A finite "no key yet" reference: exp2(s - m) needs no -inf guard, the first half with
    // a visible key always outgrows it (rescale with alpha = 0), and fully masked scores
    // (-inf) still give probability 0.
    float m = kMaxInit;
    const int limit = prefix + tw + c32;  // last key visible to query row tw + c
#pragma unroll
    for (int n = 0; n < NT2; ++n)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[n][v] = 0.f;

    // ---- pipeline pieces (hh = 32-key half of a 64-key tile) ----
    // S^T of one half: lane (c, h), element v holds key 8 (v/4) + 4 h + v%4 of the half.
    // The accumulator starts at 0, or, for a masked half, at the seed mask_seed wrote
    // (0 where visible, -inf where masked: -inf + finite products stays -inf).
    auto qk_half = [&](const __bf16* lk, int hh, f32x16& st, auto seeded_tag)
                       __attribute__((always_inline)) {
        if constexpr (!decltype(seeded_tag)::value) {
#pragma unroll
            for (int v = 0; v < 16; ++v) st[v] = 0.f;
        }
#pragma unroll
        for (int kk = 0; kk < S2; ++kk) {
            const bf16x8 kop = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(lk + hh * 32 * D + koff[kk]));
            st = mfma32x32x16(kop, qop[kk], st);
        }
    };
    // Mask seed of one half (key0 = its first key): 0 for visible keys, -inf for keys past
    // the row's causal limit and, with kBits, for keys whose validity bit is clear (only
    // needed when the table has holes: otherwise every key past kv_end is past every row's
    // limit too).
    auto vbits_of = [&](const uint8_t* lvalid, int hh) __attribute__((always_inline)) {
        const uint64_t v = __builtin_amdgcn_ballot_w64(lvalid[lane] != 0);
        return static_cast<uint32_t>(v >> (32 * hh));
    };
    auto mask_seed = [&](f32x16& st, int key0, const uint8_t* lvalid, int hh, auto bits_tag)
                         __attribute__((always_inline)) {
        constexpr bool kBits = decltype(bits_tag)::value;
        if (!kBits && key0 + 31 <= prefix + tw) {  // wave-uniform: every key visible
#pragma unroll
            for (int v = 0; v < 16; ++v)
                st[v] = 0.f;
            return;
        }
        const int thr = limit - key0 - 4 * h32;
        uint32_t vb = 0u;
        if constexpr (kBits) vb = vbits_of(lvalid, hh) >> (4 * h32);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int kt = 8 * (v >> 2) + (v & 3);
            bool ok = kt <= thr;
            if constexpr (kBits) ok = ok && ((vb >> kt) & 1u);
            st[v] = ok ? 0.f : kNegInf;
        }
    };
    // Row max of one half (scaled, log2 units); returns whether the row outgrew the slack.
    auto max_half = [&](const f32x16& st, float& mt) __attribute__((always_inline)) {
        float x0 = fmaxf(fmaxf(st[0], st[1]), st[2]);
        float x1 = fmaxf(fmaxf(st[3], st[4]), st[5]);
        float x2 = fmaxf(fmaxf(st[6], st[7]), st[8]);
        float x3 = fmaxf(fmaxf(st[9], st[10]), st[11]);
        float x4 = fmaxf(fmaxf(st[12], st[13]), st[14]);
        float x = fmaxf(fmaxf(x0, x1), fmaxf(fmaxf(x2, x3), fmaxf(x4, st[15])));
        x = wave_max_swap32(x) * scale_log2;
        mt = x;
        return x > m + kRescaleSlack;
    };
    auto rescale = [&](bool grow, const float& mt) __attribute__((always_inline)) {
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float m_new = fmaxf(m, mt);
            const float alpha = __builtin_amdgcn_exp2f(m - m_new);
            lsum = lsum * alpha;
#pragma unroll
            for (int n = 0; n < NT2; ++n) acc[n] = acc[n] * alpha;
            m = m_new;
        }
    };
    // P^T operands of one half: pop[s] holds elements 8 s .. 8 s + 7 (keys 16 s + 8 (e/4) +
    // 4 h + e%4, e = 0..7), the B operand of PV k-step s. The lane's share of the row sum
    // adds the same bf16 probabilities (v_dot2 with ones on each packed pair).
    auto exp_part = [&](const f32x16& st, int s, bf16x8& pops) __attribute__((always_inline)) {
        using bf16x2 = __bf16 __attribute__((ext_vector_type(2)));
        const bf16x2 one2 = __builtin_bit_cast(bf16x2, 0x3f803f80u);
        const float mneg = -m;
        u32x4 pw;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            const float p0 =
                __builtin_amdgcn_exp2f(__builtin_fmaf(st[8 * s + 2 * x], scale_log2, mneg));
            const float p1 =
                __builtin_amdgcn_exp2f(__builtin_fmaf(st[8 * s + 2 * x + 1], scale_log2, mneg));
            const uint32_t pk = pack_bf16x2(p0, p1);
            lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk), one2, lsum,
                                                   false);
            pw[x] = pk;
        }
        pops = __builtin_bit_cast(bf16x8, pw);
    };
    // V^T operand (A, 32 dims x 16 keys): lane (c, h) holds dim c of the tile for keys
    // 16 s + 4 h + r (r < 4) and 16 s + 8 + 4 h + r, matching pop[s]'s key order.
    auto pv_part = [&](const __bf16* lv, int hh, int s, const bf16x8& pops)
                       __attribute__((always_inline)) {
        using v4s = short __attribute__((ext_vector_type(4)));
        using v8s = short __attribute__((ext_vector_type(8)));
#pragma unroll
        for (int n = 0; n < NT2; ++n) {
            const __bf16* base = lv + (hh * 32 + 16 * s) * D;
            const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4s*)(base + voffa[n]));
            const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4s*)(base + voffb[n]));
            const v8s ab = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
            acc[n] = mfma32x32x16(__builtin_bit_cast(bf16x8, ab), pops, acc[n]);
        }
    };

    // Interleave patterns for the two pipeline phases (igrouplp masks: 0x8 MFMA, 0x100 DS
    // read, 0x402 VALU incl. transcendental). X: one QK MFMA per K read, with the exp work
    // of the current half spread between them. Y: one PV MFMA per V^T operand (two
    // transposing reads), with the next half's mask / max work in between.
    constexpr int kXGroups = S2;
    constexpr int kXValu = 3;
    constexpr int kYValuA = 6;  // exp of the second P operand beside PV k-step 0
    constexpr int kYValuB = 3;  // next half's row max beside PV k-step 1
    constexpr int kXPre = 2;  // K operand reads issued ahead of the MFMAs using them
    constexpr int kYPre = 2;  // V^T operands read ahead
    auto interleave_x = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_sched_group_barrier(0x100, kXPre, 0);
#pragma unroll
        for (int i = 0; i < kXGroups; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x402, kXValu, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i + kXPre < kXGroups) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    };
    auto interleave_y = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * kYPre, 0);
#pragma unroll
        for (int i = 0; i < 2 * NT2; ++i) {
            if (i < NT2)
                __builtin_amdgcn_sched_group_barrier(0x402, kYValuA, 0);
            else
                __builtin_amdgcn_sched_group_barrier(0x402, kYValuB, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i + kYPre < 2 * NT2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
    };

    f32x16 sc;  // S of the half being exponentiated
    f32x16 sn;  // S of the next half
    bf16x8 pop[2];
    float mt;
    // The tile loop, compiled twice: with the per-key validity bits (tables with holes) and
    // without; each workgroup runs one of them.
    // Whether stage(t) issues exactly 2 NL loads per wavefront (the unchecked path), so a
    // vmcnt bound can wait for older tiles only.
    auto full_stage = [&](int t) __attribute__((always_inline)) {
        return !holes && t < ntiles && (t + 1) * kKeysPerTile <= kv_end;
    };
    auto run = [&](auto holes_tag) __attribute__((always_inline)) {
        // Prologue: tiles 0 and 1 in flight, S of tile 0 / half 0 formed, masked and maxed.
        if constexpr (F8) {
            stage8(0, lds_k8_0, lds_v8_0, lds_valid0, sk8[0], sv8[0]);
            if (ntiles > 1) stage8(1, lds_k8_1, lds_v8_1, lds_valid1, sk8[1], sv8[1]);
            __builtin_amdgcn_s_waitcnt(0x0F70);
            __syncthreads();
            convert8(lds_k8_0, lds_v8_0, lds_k0, lds_v0, sk8[0], sv8[0]);
        } else {
            stage(0, lds_k0, lds_v0, lds_valid0, holes_tag);
            if (ntiles > 1) stage(1, lds_k1, lds_v1, lds_valid1, holes_tag);
            // Tile 0 landed: vmcnt bounded by tile 1's loads when their count is exact (the
            // checked path may issue fewer), else everything.
            if (full_stage(1))
                __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * NL));
            else
                __builtin_amdgcn_s_waitcnt(0x0F70);
        }
        __syncthreads();
        mask_seed(sc, 0, lds_valid0, 0, holes_tag);
        qk_half(lds_k0, 0, sc, std::true_type{});
        const bool grow_first = max_half(sc, mt);
        rescale(grow_first, mt);

        // One tile step. Entering: sc = S of (tile t, half 0), already masked and rescaled for.
        // kLast: tile t is the last one (no next tile to start).
        auto step = [&](int t, auto cur, auto nxt, auto ld, auto mask_tag, auto last_tag)
                        __attribute__((always_inline)) {
            constexpr int BC = decltype(cur)::value;
            constexpr int BN = decltype(nxt)::value;
            constexpr int BL = decltype(ld)::value;
            constexpr bool kMask = decltype(mask_tag)::value;
            constexpr bool kLast = decltype(last_tag)::value;
            static_assert(!F8 || (BC < 2 && BN < 2 && BL < 2), "fp8 runs a two-tile ring");
            const __bf16* kc = BC == 0 ? lds_k0 : (BC == 1 ? lds_k1 : lds_k2);
            const __bf16* vc = BC == 0 ? lds_v0 : (BC == 1 ? lds_v1 : lds_v2);
            const uint8_t* valc = BC == 0 ? lds_valid0 : (BC == 1 ? lds_valid1 : lds_valid2);
            const __bf16* kn = BN == 0 ? lds_k0 : (BN == 1 ? lds_k1 : lds_k2);
            const uint8_t* valn = BN == 0 ? lds_valid0 : (BN == 1 ? lds_valid1 : lds_valid2);
            __bf16* kl = BL == 0 ? lds_k0 : (BL == 1 ? lds_k1 : lds_k2);
            __bf16* vl = BL == 0 ? lds_v0 : (BL == 1 ? lds_v1 : lds_v2);
            uint8_t* vall = BL == 0 ? lds_valid0 : (BL == 1 ? lds_valid1 : lds_valid2);
            const int key0 = t * kKeysPerTile;

            // Halves wholly above this wavefront's last row contribute nothing: in masked
            // steps their MFMAs and exps are skipped (wave-uniform; skip0 -> skip1 -> skipn0).
            const int wave_lim = prefix + tw + kPipeRows - 1;
            const bool skip0 = kMask && key0 > wave_lim;
            const bool skip1 = kMask && key0 + 32 > wave_lim;
            const bool skipn0 = kMask && key0 + kKeysPerTile > wave_lim;
            auto fill_neg_inf = [](f32x16& st) __attribute__((always_inline)) {
#pragma unroll
                for (int v = 0; v < 16; ++v) st[v] = kNegInf;
            };
            // X: exp of (t, 0) || QK of (t, 1)
            __builtin_amdgcn_sched_barrier(0);
            if (!skip1) {
                exp_part(sc, 0, pop[0]);
                if constexpr (kMask) mask_seed(sn, key0 + 32, valc, 1, holes_tag);
                qk_half(kc, 1, sn, mask_tag);
                interleave_x();
            } else {
                if (!skip0) exp_part(sc, 0, pop[0]);
                fill_neg_inf(sn);
            }
            // Y: PV of (t, 0), exp of its second P operand || max of (t, 1)
            __builtin_amdgcn_sched_barrier(0);
            bool grow1 = false;  // skip0: S of (t, 1) is -inf, its max cannot grow
            if (!skip0) {
                pv_part(vc, 0, 0, pop[0]);
                exp_part(sc, 1, pop[1]);
                pv_part(vc, 0, 1, pop[1]);
                grow1 = max_half(sn, mt);
                interleave_y();
            }
            __builtin_amdgcn_sched_barrier(0);
            rescale(grow1, mt);
            if constexpr (!kLast) {
                __builtin_amdgcn_s_waitcnt(0x0F70);  // this wavefront's loads of tile t+1 landed
                __syncthreads();                     // ... and everyone's; tile t-1 is free
                if constexpr (F8) {
                    // tile t+1: bytes (ring slot BN) -> bf16 (slot BN, which held tile t-1);
                    // then tile t+2's bytes go to slot BL (= BC, converted one step ago)
                    convert8(BN == 0 ? lds_k8_0 : lds_k8_1, BN == 0 ? lds_v8_0 : lds_v8_1,
                             BN == 0 ? lds_k0 : lds_k1, BN == 0 ? lds_v0 : lds_v1, sk8[BN], sv8[BN]);
                    __syncthreads();
                    if (t + 2 < ntiles)
                        stage8(t + 2, BL == 0 ? lds_k8_0 : lds_k8_1, BL == 0 ? lds_v8_0 : lds_v8_1,
                               vall, sk8[BL], sv8[BL]);
                } else {
                    if (t + 2 < ntiles) stage(t + 2, kl, vl, vall, holes_tag);
                }
            }
            // X: exp of (t, 1) || QK of (t+1, 0)
            __builtin_amdgcn_sched_barrier(0);
            if (!skipn0) {
                exp_part(sn, 0, pop[0]);
                if constexpr (!kLast) {
                    if constexpr (kMask)
                        mask_seed(sc, key0 + kKeysPerTile, valn, 0, holes_tag);
                    qk_half(kn, 0, sc, mask_tag);
                }
                if constexpr (!kLast) interleave_x();
            } else {
                if (!skip1) exp_part(sn, 0, pop[0]);
                if constexpr (!kLast) fill_neg_inf(sc);
            }
            // Y: PV of (t, 1), exp of its second P operand || max of (t+1, 0)
            __builtin_amdgcn_sched_barrier(0);
            bool grow0 = false;  // skip1 -> skipn0: S of (t+1, 0) is -inf
            if (!skip1) {
                pv_part(vc, 1, 0, pop[0]);
                exp_part(sn, 1, pop[1]);
                pv_part(vc, 1, 1, pop[1]);
                if constexpr (!kLast) {
                    grow0 = max_half(sc, mt);
                    interleave_y();
                }
            }
            if constexpr (!kLast) {
                __builtin_amdgcn_sched_barrier(0);
                rescale(grow0, mt);
            }
        };
        using B0 = std::integral_constant<int, 0>;
        using B1 = std::integral_constant<int, 1>;
        using B2 = std::integral_constant<int, 2>;
        using F = std::false_type;
        using T = std::true_type;

        // Steps whose tiles t and t+1 lie wholly below the workgroup's first query row need no
        // mask (unless the table has holes); they run in triples so buffer roles stay static.
        const int mask_free_tiles = holes ? 0 : (prefix + t0 + 1) / kKeysPerTile;
        const int mf_steps = max(0, min(ntiles - 1, mask_free_tiles - 1));
        int t = 0;
        if constexpr (F8) {
            // two-tile ring: tile t in slot t % 2; the stage target of step t is slot t % 2 too
            for (; t + 2 <= mf_steps; t += 2) {
                step(t, B0{}, B1{}, B0{}, F{}, F{});
                step(t + 1, B1{}, B0{}, B1{}, F{}, F{});
            }
            for (;;) {
                if (t >= ntiles - 1) break;
                step(t, B0{}, B1{}, B0{}, T{}, F{});
                ++t;
                if (t >= ntiles - 1) break;
                step(t, B1{}, B0{}, B1{}, T{}, F{});
                ++t;
            }
            if (t % 2 == 0)
                step(t, B0{}, B1{}, B0{}, T{}, T{});
            else
                step(t, B1{}, B0{}, B1{}, T{}, T{});
        } else {
        for (; t + 3 <= mf_steps; t += 3) {
            step(t, B0{}, B1{}, B2{}, F{}, F{});
            step(t + 1, B1{}, B2{}, B0{}, F{}, F{});
            step(t + 2, B2{}, B0{}, B1{}, F{}, F{});
        }
        for (;;) {
            if (t >= ntiles - 1) break;
            step(t, B0{}, B1{}, B2{}, T{}, F{});
            ++t;
            if (t >= ntiles - 1) break;
            step(t, B1{}, B2{}, B0{}, T{}, F{});
            ++t;
            if (t >= ntiles - 1) break;
            step(t, B2{}, B0{}, B1{}, T{}, F{});
            ++t;
        }
        switch (t % 3) {
            case 0: step(t, B0{}, B1{}, B2{}, T{}, T{}); break;
            case 1: step(t, B1{}, B2{}, B0{}, T{}, T{}); break;
            default: step(t, B2{}, B0{}, B1{}, T{}, T{}); break;
        }
        }
    };
    if (holes)
        run(std::true_type{});
    else
        run(std::false_type{});

    // Epilogue: lane (c, h) holds O[tw + c][32 n + 8 i + 4 h + r] = acc[n][4 i + r].
    {
        const float l_tot = lsum + __uint_as_float(__builtin_amdgcn_permlane32_swap(
                                           __float_as_uint(lsum), __float_as_uint(lsum),
                                           false, false)[h32 ? 0 : 1]);
        const int tq = tw + c32;
        if (tq < rows) {
            const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
            __bf16* o = out + (static_cast<int64_t>(qb + tq) * hq + q_head) * ds;
#pragma unroll
            for (int n = 0; n < NT2; ++n) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (kPad && 32 * n + 8 * i + 4 * h32 >= dr) continue;  // padded dims
                    u32x2 w;
                    w[0] = pack_bf16x2(acc[n][4 * i] * inv, acc[n][4 * i + 1] * inv);
                    w[1] = pack_bf16x2(acc[n][4 * i + 2] * inv, acc[n][4 * i + 3] * inv);
                    *reinterpret_cast<u32x2*>(o + 32 * n + 8 * i + 4 * h32) = w;
                }
            }
        }
    }
}

struct PrefillLayout {
    size_t counts_off, zero_off, tiles_off, dec_off, big_off, decode_ws_off, total;
    int max_tiles;
    int tile_tokens;
    DecodePlan plan;
};

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int tile_tokens_for(int head_dim, int G) {
    if (pipe_head_dim(head_dim))
        return (PipeShape<64>::kWaves / heads_per_wg(G)) * PipeShape<64>::kRows;
    return (kWaves / heads_per_wg(G)) * PrefillShape<256>::kQW;
}

PrefillLayout prefill_layout(int batch_size, int total_query_tokens, int max_blocks_per_req,
                             int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                             bool fp8) {
    PrefillLayout L{};
    const int G = num_q_heads / num_kv_heads;
    const int D = decode_mfma_dim(head_dim);  // the kernels' (padded) head dim
    L.tile_tokens = tile_tokens_for(D, G);
    L.max_tiles = total_query_tokens / L.tile_tokens + batch_size;
    L.plan = plan_decode_items(batch_size, num_q_heads, num_kv_heads, head_dim,
                               max_blocks_per_req * block_size, fp8);
    size_t off = 0;
    L.counts_off = off;
    off = align256(off + 2 * sizeof(int32_t));
    L.zero_off = off;  // one all-zero K/V row (D bf16), rewritten by the planner
    off = align256(off + static_cast<size_t>(D) * 2);
    L.tiles_off = off;
    off = align256(off + static_cast<size_t>(L.max_tiles) * sizeof(TileEntry));
    L.dec_off = off;
    off = align256(off + static_cast<size_t>(batch_size) * sizeof(int32_t));
    L.big_off = off;  // the planner's per-request arrays for batches it cannot keep in LDS
    if (batch_size > kMaxPlanRequests)
        off = align256(off + 2 * static_cast<size_t>(batch_size) * sizeof(int32_t));
    L.decode_ws_off = off;
    off = align256(off + decode_workspace_bytes(batch_size, num_q_heads, head_dim, L.plan));
    L.total = off;
    return L;
}

// dr: the head dim of q / cache / output rows (dr == D unless kPad).
template <int D, bool F8, bool kPad>
hipError_t launch_tiles(const void* q, const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale,
                        const int32_t* block_table, const int32_t* qsl,
                        const int32_t* context_lens, void* output, int total_query_tokens,
                        int mbpr, int hq, int hkv, int block_size, const int32_t* counts,
                        const TileEntry* tiles, const void* zero_row, int max_tiles,
                        hipStream_t stream, int dr, int batch_size, bool fused_dec) {
    const int G = hq / hkv;
    const int U = hkv * (G / heads_per_wg(G));
    const float scale_log2 = kLog2e / sqrtf(static_cast<float>(dr));
    if constexpr (pipe_head_dim(D)) {
        // fused_dec: the single-token requests run in the first workgroups of this launch,
        // one per (request, virtual kv head), with prefill semantics (no 1e-6 in the
        // denominator, malformed rows untouched).
        const int rep = dcore::decode_head_rep(G);
        dcore::ItemArgs it{};
        int dec_wgs = 0;
        if (fused_dec) {
            it.num_items = batch_size;
            it.qsl = qsl;
            it.singles_total = total_query_tokens;
            dec_wgs = batch_size * hkv * rep;
        }
        const int64_t grid = static_cast<int64_t>(max_tiles) * U + dec_wgs;
        prefill_pipe_kernel<D, F8, kPad>
            <<<static_cast<unsigned>(grid), PipeShape<D>::kThreads, 0, stream>>>(
            static_cast<const __bf16*>(q), k_cache, v_cache, k_scale, v_scale, block_table, qsl,
            context_lens,
            static_cast<__bf16*>(output), counts, tiles, total_query_tokens, mbpr, hq, hkv,
            scale_log2, dr, it, dec_wgs, hkv * rep, rep);
        return hipGetLastError();
    } else if constexpr (F8) {
        return hipErrorInvalidValue;  // fp8 has the pipelined path only
    } else {
        const int64_t grid = static_cast<int64_t>(max_tiles) * U;
        prefill_tile_kernel<D, kPad><<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(
            static_cast<const __bf16*>(q), static_cast<const __bf16*>(k_cache),
            static_cast<const __bf16*>(v_cache), block_table, qsl, context_lens,
            static_cast<__bf16*>(output), counts, tiles, static_cast<const __bf16*>(zero_row),
            total_query_tokens, mbpr, hq, hkv, block_size, scale_log2, dr);
        return hipGetLastError();
    }
}

}  // namespace

bool prefill_fast_supported(int num_q_heads, int num_kv_heads, int head_dim,
                            int max_blocks_per_req) {
    if (num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0) return false;
    // Head dims run at the MFMA size 64 / 128 / 256 (smaller ones padded with zeros). The
    // 64 / 128 kernels (bf16) stage any table length; the 256 kernel keeps the table row in
    // LDS.
    const int D = decode_mfma_dim(head_dim);
    if (D == 64 || D == 128) return true;
    return D == 256 && max_blocks_per_req <= kMaxTableLds;
}

bool prefill_fp8_supported(int head_dim, int max_blocks_per_req) {
    return pipe_head_dim(head_dim) && max_blocks_per_req <= kMaxTableLds;
}

size_t prefill_workspace_bytes(int batch_size, int total_query_tokens, int max_blocks_per_req,
                               int num_q_heads, int num_kv_heads, int head_dim,
                               int block_size) {
    // One size serves the bf16 and the fp8 prefill, whose decode-item plans differ.
    return std::max(prefill_layout(batch_size, total_query_tokens, max_blocks_per_req,
                                   num_q_heads, num_kv_heads, head_dim, block_size, false)
                        .total,
                    prefill_layout(batch_size, total_query_tokens, max_blocks_per_req,
                                   num_q_heads, num_kv_heads, head_dim, block_size, true)
                        .total);
}

namespace {

// Mixed batches of at least this many requests run their decode items on the caller's side
// stream (when one is given) beside the tile kernel; smaller batches -- typically pure
// prompt batches with no decode items -- run them on the caller's stream before the tiles,
// where their near-empty launches take no CUs from the tiles (and, ahead of the tile
// kernel rather than behind it, cost ~0.7 us less per step).
constexpr int kOverlapMinRequests = 32;
// The fused route's limits: at most this many (request, virtual kv head) workgroups ahead of
// the tiles (each of a pure prompt batch's requests costs one that only reads its query
// length), and table rows of at most this many positions (one workgroup streams a whole
// row through one CU: ~34 us at 2048 positions, ~65 us at 4096). Measured on one box
// against the decode launches (serial, split plan): configs[2] 149.1 -> 143.7 us, 16 x 512
// prompts 45.5 -> 43.1, 64 x 128 prompts 61.4 -> 42.3; mixed batches of 128-1024 prompt
// tokens with 4-60 single-token requests of 200-2000 positions 31.5 / 57.7 / 91.5 -> 27.5 /
// 34.2 / 62.0 us. With rows of up to 4000 positions a batch of one 16-token prompt and 4
// long single-token requests ran 35.6 -> 46.5 us, hence the 2048 bound. Group counts (same
// box, bound 512 -> 1024 / 2048): 128 x 128 prompts 79.5 -> 74.4 us, 2 prompts + 126
// single-token requests of 1500-2000 positions 253.5 -> 192.3 us; at ~2000 groups 4 prompts
// + 250 requests of 200-2000 positions ran 181.3 -> 194.8 us (beyond ~1000 single-token
// requests per launch the split plan streams them faster), hence 1024.
constexpr int64_t kFusedDecodeGroups = 1024;
constexpr int64_t kFusedDecodeMaxCtx = 2048;

}  // namespace

namespace {

template <bool F8>
hipError_t prefill_impl(const void* q, const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale, const int32_t* block_table,
                        const int32_t* query_start_loc, const int32_t* context_lens,
                        void* output, int batch_size, int total_query_tokens,
                        int max_blocks_per_req, int num_q_heads, int num_kv_heads, int head_dim,
                        int block_size, void* workspace, hipStream_t stream,
                        const PrefillOverlap* overlap) {
    const PrefillLayout L = prefill_layout(batch_size, total_query_tokens, max_blocks_per_req,
                                           num_q_heads, num_kv_heads, head_dim, block_size, F8);
    char* ws = static_cast<char*>(workspace);
    int32_t* counts = reinterpret_cast<int32_t*>(ws + L.counts_off);
    TileEntry* tiles = reinterpret_cast<TileEntry*>(ws + L.tiles_off);
    int32_t* dec = reinterpret_cast<int32_t*>(ws + L.dec_off);
    uint32_t* zero_row = reinterpret_cast<uint32_t*>(ws + L.zero_off);
    if (batch_size > kMaxPlanRequests) {
        int* big = reinterpret_cast<int*>(ws + L.big_off);
        prefill_plan_kernel<true><<<1, 1024, 0, stream>>>(
            query_start_loc, context_lens, batch_size, total_query_tokens, L.tile_tokens, counts,
            tiles, dec, zero_row, decode_mfma_dim(head_dim) / 2, big, big + batch_size, 1);
    } else {
        prefill_plan_kernel<false><<<1, 1024, 0, stream>>>(
            query_start_loc, context_lens, batch_size, total_query_tokens, L.tile_tokens, counts,
            tiles, dec, zero_row, decode_mfma_dim(head_dim) / 2, nullptr, nullptr, 1);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    // Single-token requests of a mixed batch go through the split-KV decode (prefill
    // semantics). Given the caller's side stream and events, batches of kOverlapMinRequests
    // or more run them there, concurrently with the tile kernel: they write other output rows
    // and other workspace, and the memory-bound decode work fills CUs the MFMA-bound tiles
    // leave idle. The fork and join are event records and waits only (no host sync), which
    // is also legal under stream capture. Otherwise they run on the caller's stream between
    // the planner and the tile kernel.
    DecodeItems items;
    items.num_items = batch_size;
    items.item_count = counts + 1;
    items.item_req = dec;
    items.query_start_loc = query_start_loc;
    items.denom_eps = 0.0f;
    items.zero_invalid = false;
    auto launch_decode_items = [&](hipStream_t s) {
        if constexpr (F8)
            return decode_attention_fp8(q, k_cache, v_cache, k_scale, v_scale, block_table,
                                        context_lens, output, items, max_blocks_per_req,
                                        num_q_heads, num_kv_heads, head_dim, L.plan,
                                        ws + L.decode_ws_off, s);
        else
            return decode_attention(q, k_cache, v_cache, block_table, context_lens, output,
                                    items, max_blocks_per_req, num_q_heads, num_kv_heads,
                                    head_dim, block_size, L.plan, ws + L.decode_ws_off, s);
    };
    // Small batches whose table rows are short enough run their single-token requests
    // inside the tile launch (fused_dec): no decode launches at all, which a pure prompt
    // batch -- most prefill steps -- would otherwise pay for work known on the device only.
    const int Dk = decode_mfma_dim(head_dim);
    const int64_t dec_groups = static_cast<int64_t>(batch_size) * num_kv_heads *
                               dcore::decode_head_rep(num_q_heads / num_kv_heads);
    const bool fused_dec = pipe_head_dim(Dk) && dec_groups <= kFusedDecodeGroups &&
                           static_cast<int64_t>(max_blocks_per_req) * block_size <=
                               kFusedDecodeMaxCtx;
    const bool fork = !fused_dec && overlap != nullptr && overlap->side != nullptr &&
                      batch_size >= kOverlapMinRequests;
    // Once the side stream has waited on the fork event it is joined back on every path,
    // errors included (an unjoined fork would invalidate a capture of the caller's stream).
    auto join = [&](hipError_t first) {
        const hipError_t je = hipEventRecord(overlap->join, overlap->side);
        const hipError_t jw = je == hipSuccess ? hipStreamWaitEvent(stream, overlap->join, 0) : je;
        return first != hipSuccess ? first : jw;
    };
    if (fork) {
        err = hipEventRecord(overlap->fork, stream);
        if (err != hipSuccess) return err;
        err = hipStreamWaitEvent(overlap->side, overlap->fork, 0);
        if (err != hipSuccess) return err;
        err = launch_decode_items(overlap->side);
        if (err != hipSuccess) return join(err);
    } else if (!fused_dec) {
        err = launch_decode_items(stream);
        if (err != hipSuccess) return err;
    }
    const int D = decode_mfma_dim(head_dim);
    const bool pad = D != head_dim;
#define CCI_TILES(DD, PP)                                                                    \
    launch_tiles<DD, F8, PP>(q, k_cache, v_cache, k_scale, v_scale, block_table,             \
                             query_start_loc, context_lens, output, total_query_tokens,      \
                             max_blocks_per_req, num_q_heads, num_kv_heads, block_size,      \
                             counts, tiles, zero_row, L.max_tiles, stream, head_dim,         \
                             batch_size, fused_dec)
    if (F8 && pad) {
        err = hipErrorInvalidValue;  // fp8 runs the native head dims only
    } else {
        switch (D) {
            case 64:
                err = pad ? CCI_TILES(64, !F8) : CCI_TILES(64, false);
                break;
            case 128:
                err = pad ? CCI_TILES(128, !F8) : CCI_TILES(128, false);
                break;
            case 256:
                err = pad ? CCI_TILES(256, !F8) : CCI_TILES(256, false);
                break;
            default:
                err = hipErrorInvalidValue;
        }
    }
#undef CCI_TILES
    return fork ? join(err) : err;
}

}  // namespace

hipError_t prefill_attention(const void* q, const void* k_cache, const void* v_cache,
                             const int32_t* block_table, const int32_t* query_start_loc,
                             const int32_t* context_lens, void* output, int batch_size,
                             int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                             int num_kv_heads, int head_dim, int block_size, void* workspace,
                             hipStream_t stream, const PrefillOverlap* overlap) {
    return prefill_impl<false>(q, k_cache, v_cache, nullptr, nullptr, block_table,
                               query_start_loc, context_lens, output, batch_size,
                               total_query_tokens, max_blocks_per_req, num_q_heads, num_kv_heads,
                               head_dim, block_size, workspace, stream, overlap);
}

// ---- any-layout prefill (the tile kernel with kAny) ----
namespace {

int any_dim(int dr) { return dr <= 64 ? 64 : dr <= 128 ? 128 : 256; }

struct AnyLayout {
    size_t counts_off, tiles_off, dec_off, big_off, total;
    int max_tiles, tile_tokens;
};

AnyLayout any_layout(int batch_size, int total_query_tokens, int num_q_heads, int num_kv_heads,
                     int head_dim) {
    AnyLayout L{};
    const int G = num_q_heads / num_kv_heads;
    L.tile_tokens = (kWaves / heads_per_wg(G)) *
                    (any_dim(head_dim) <= 128 ? PrefillShape<128>::kQW : PrefillShape<256>::kQW);
    // every request may be a one-row tile here (single-token requests are tiles too)
    L.max_tiles = total_query_tokens / L.tile_tokens + batch_size;
    size_t off = 0;
    L.counts_off = off;
    off = align256(off + 2 * sizeof(int32_t));
    L.tiles_off = off;
    off = align256(off + static_cast<size_t>(L.max_tiles) * sizeof(TileEntry));
    L.dec_off = off;
    off = align256(off + static_cast<size_t>(batch_size) * sizeof(int32_t));
    L.big_off = off;
    if (batch_size > kMaxPlanRequests)
        off = align256(off + 2 * static_cast<size_t>(batch_size) * sizeof(int32_t));
    L.total = off;
    return L;
}

}  // namespace

bool prefill_any_supported(int num_q_heads, int num_kv_heads, int head_dim,
                           int max_blocks_per_req) {
    (void)max_blocks_per_req;  // longer table rows are read from global memory
    return num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && head_dim > 0 &&
           head_dim <= 256;
}

size_t prefill_any_workspace_bytes(int batch_size, int total_query_tokens, int num_q_heads,
                                   int num_kv_heads, int head_dim) {
    return any_layout(batch_size, total_query_tokens, num_q_heads, num_kv_heads, head_dim).total;
}

hipError_t prefill_attention_any(const void* q, const void* k_cache, const void* v_cache,
                                 const int32_t* block_table, const int32_t* query_start_loc,
                                 const int32_t* context_lens, void* output, int batch_size,
                                 int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                                 int num_kv_heads, int head_dim, int block_size,
                                 void* workspace, hipStream_t stream) {
    const AnyLayout L =
        any_layout(batch_size, total_query_tokens, num_q_heads, num_kv_heads, head_dim);
    char* ws = static_cast<char*>(workspace);
    int32_t* counts = reinterpret_cast<int32_t*>(ws + L.counts_off);
    TileEntry* tiles = reinterpret_cast<TileEntry*>(ws + L.tiles_off);
    int32_t* dec = reinterpret_cast<int32_t*>(ws + L.dec_off);
    // single-token requests run as one-row tiles (the decode kernels take 16-token blocks)
    if (batch_size > kMaxPlanRequests) {
        int* big = reinterpret_cast<int*>(ws + L.big_off);
        prefill_plan_kernel<true><<<1, 1024, 0, stream>>>(
            query_start_loc, context_lens, batch_size, total_query_tokens, L.tile_tokens, counts,
            tiles, dec, nullptr, 0, big, big + batch_size, 0);
    } else {
        prefill_plan_kernel<false><<<1, 1024, 0, stream>>>(
            query_start_loc, context_lens, batch_size, total_query_tokens, L.tile_tokens, counts,
            tiles, dec, nullptr, 0, nullptr, nullptr, 0);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int G = num_q_heads / num_kv_heads;
    const int U = num_kv_heads * (G / heads_per_wg(G));
    const int64_t grid = static_cast<int64_t>(L.max_tiles) * U;
    const float scale_log2 = kLog2e / sqrtf(static_cast<float>(head_dim));
    auto go = [&](auto kernel) {
        kernel<<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(
            static_cast<const __bf16*>(q), static_cast<const __bf16*>(k_cache),
            static_cast<const __bf16*>(v_cache), block_table, query_start_loc, context_lens,
            static_cast<__bf16*>(output), counts, tiles, nullptr, total_query_tokens,
            max_blocks_per_req, num_q_heads, num_kv_heads, block_size, scale_log2, head_dim);
        return hipGetLastError();
    };
    switch (any_dim(head_dim)) {
        case 64: return go(prefill_tile_kernel<64, false, true>);
        case 128: return go(prefill_tile_kernel<128, false, true>);
        default: return go(prefill_tile_kernel<256, false, true>);
    }
}

hipError_t prefill_attention_fp8(const void* q, const void* k_cache, const void* v_cache,
                                 const float* k_scale, const float* v_scale,
                                 const int32_t* block_table, const int32_t* query_start_loc,
                                 const int32_t* context_lens, void* output, int batch_size,
                                 int total_query_tokens, int max_blocks_per_req,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 void* workspace, hipStream_t stream,
                                 const PrefillOverlap* overlap) {
    if (!pipe_head_dim(head_dim)) return hipErrorInvalidValue;
    return prefill_impl<true>(q, k_cache, v_cache, k_scale, v_scale, block_table,
                              query_start_loc, context_lens, output, batch_size,
                              total_query_tokens, max_blocks_per_req, num_q_heads, num_kv_heads,
                              head_dim, kBlock, workspace, stream, overlap);
}

}  // namespace ccinfer::hipk
