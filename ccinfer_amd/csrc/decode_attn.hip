// Paged decode attention for gfx950: split-KV (flash-decoding) on bf16 MFMA tiles. The
// device building blocks (chunk loads, online softmax, the split loop, the group body) live
// in decode_core.hpp, which the prefill launch includes too.
//
// Semantics follow the reference decode (src/kernel/attention/decode_attn.cu:364-473):
//   out[b, hq, :] = softmax(q . K_ctx^T / sqrt(D)) . V_ctx  with kv_head = hq / (Hq/Hkv),
//   positions addressed through block_table (16-token blocks), negative block ids skipped,
//   ctx <= 0 or ceil(ctx/16) > max_blocks_per_req -> zeros, denominator sum + 1e-6.
//
// Work decomposition: a split is a run of consecutive 32-token chunks of one (query row,
//   kv_head) (at most 2048 positions). All Hq/Hkv query heads of the GQA group are handled
//   by the same wavefront, so every K/V byte of a (request, kv_head) is read from HBM
//   exactly once.
//   Batches of 4..256 items use the flat plan -- every wavefront reads the items' context
//   lengths, lays their chunks end to end and takes one of W equal ranges of them, across
//   item boundaries (a range that crosses one is processed as one split per item), so a
//   ragged batch is evenly loaded in one round of one workgroup per CU; wave-wide prefix
//   scans find the range's splits and number each item's partial rows. Split 0 of every
//   row writes a merge descriptor (first partial slot, split count) that the merge kernel
//   reads, so the merge does not repeat the scan. This also covers the decode items of a
//   mixed prefill batch, whose list and count the prefill planner writes on the device.
//   Other batches use a fixed split length chosen on the host from the longest possible
//   context (one wavefront per (item, kv_head, split)).
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
// Memory pipeline: chunks are double-buffered in registers with a branch-free prefetch (the
// chunk index is clamped instead of skipping the load) so the compiler's wait counts only
// ever wait for the chunk being consumed. The split's block-table entries are loaded once
// into lanes and broadcast with readlane, so no scalar load sits between two chunks.
//
// Split merge: each split writes (unnormalised O, running max m, sum l) to the workspace and
// a second kernel merges the splits of every row with a log-sum-exp weighting (the kernel
// boundary orders the partial writes before the merge reads; an in-kernel last-arrival merge
// would need agent-scope release/acquire fences, which on gfx950 write back and invalidate
// the whole L2 and cost far more than the extra launch). A row whose context fits one split
// is written directly by the first kernel and skipped by the merge.
#include <algorithm>
#include <type_traits>

#include "attn_common.hpp"
#include "decode_core.hpp"
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

using namespace dcore;

// Wavefronts the fixed split plan aims for on batches of 4+ requests: two resident per SIMD
// on 1024 SIMDs, two rounds (splits are sized for the longest possible row, so their work
// varies). Plans whose splits carry equal work -- the on-device flat plan, and the fixed plan
// of 1-3 requests -- run fastest with kEvenWaves, one 4-wavefront workgroup per CU.
constexpr int64_t kTargetWaves = 4096;
constexpr int64_t kEvenWaves = 1024;
// The fp8 cache's flat plan: twice the wavefronts (half the bytes per chunk, the same
// conversion and MFMA work): configs[1]'s batch 61.2 -> 56.0 us against kEvenWaves, while
// bf16 runs 96.3 us at kEvenWaves and 98.3 at twice that.
constexpr int64_t kEvenWavesFp8 = 2048;
// bf16 rows of up to 80 dims (160 bytes): the shorter chunks leave the one wavefront per SIMD
// waiting on its chunk loop, and a second one helps. 64 x 4096 positions, 1024 -> 2048:
// d=32 68.2 -> 58.0 us, d=80 137.3 -> 132.9 (16 x 4096: 37.1 -> 33.9), d=64 93.6 -> 92.4;
// slower at d=96 (146.6 -> 147.5), 112, 120, 128 and 192.
constexpr int kShortRowDims = 80;
constexpr int64_t flat_waves(bool fp8, int head_dim) {
    return fp8 || head_dim <= kShortRowDims ? kEvenWavesFp8 : kEvenWaves;
}
constexpr int kFlatMinItems = 4;
// Flat launches of at least this many wavefronts (two rounds at the split kernel's two waves
// per SIMD) snap their ranges to request boundaries (decode_flat_index_kernel).
constexpr int kSnapWaves = 4096;
// The group plan (one workgroup per (request, kv_head), parts merged in LDS) streams a row
// from one CU, which reads ~30 GB/s; it pays off only where the row is short enough that
// one launch beats the split plan's two. Measured (one MI355X, 16q/8kv or 32q/8kv, d=128):
// batch 1, 512 positions, 16 q-heads: 8.1 us vs 8.6 (split + merge); batch 1 with 32
// q-heads, batch 2 or 3, or 1,024+ positions: slower (10.1-67 us vs 8.9-26).
constexpr int kGroupMaxCtx = 512;
constexpr int kGroupMaxRows = 16;  // (request, q-head) rows of a plain decode batch


__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_up(v, off);
        if (lane >= off) v += u;
    }
    return v;
}

__device__ __forceinline__ int wave_max_int(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// ---- flat split plan (evaluated identically by every wavefront) ----
// The rows' 32-token chunks laid end to end (C in total, per kv head) are cut into ranges of
// T = clamp(ceil(C / W), 1, kMaxSplitTokens / kChunk) chunks, one per wavefront, whatever
// the row boundaries: every wavefront streams the same number of chunks (the last one
// fewer), so W wavefronts -- one 4-wavefront workgroup per CU -- stay evenly loaded on
// ragged batches. A range that crosses a row boundary is processed as one segment per row.
// Row r (chunk offset P_r, c_r chunks) gets one split per range it meets, numbered from
// the range that holds its first chunk, with its partial rows at S_r, the exclusive sum of
// the split counts before it.
struct FlatSegment {
    int req;         // request (item) of the segment
    int split;       // split index within the request
    int nsplit;      // splits of the request
    int first_slot;  // partial slot of the request's first split (S_r)
    int begin, end;  // positions of the segment
    int ctx;         // effective context of the request
    bool more;       // the range continues into a later request
};

// The k-th segment of wavefront w's range. Returns false past the last one. *invalid_w:
// whether request w's context is invalid (then no range holds a chunk of it).
__device__ __forceinline__ bool flat_segment(const int32_t* __restrict__ context_lens, const ItemArgs& items,
                             int mbpr, int W, int w, int k, int lane, FlatSegment* out,
                             bool* invalid_w) {
    int B = items.num_items;
    if (items.item_count != nullptr) B = min(B, *items.item_count);
    const int rounds = (B + 63) / 64;  // B <= kFlatMaxItems
    int cr[kFlatMaxItems / 64];
    int ectx[kFlatMaxItems / 64];
    int bx[kFlatMaxItems / 64];
    int total = 0;
#pragma unroll
    for (int x = 0; x < kFlatMaxItems / 64; ++x) {
        cr[x] = 0;
        ectx[x] = -1;
        bx[x] = 0;
        if (x < rounds) {
            const int r = x * 64 + lane;
            if (r < B) {
                const int req = items.item_req != nullptr ? items.item_req[r] : r;
                const int ctx = effective_ctx(context_lens[req], mbpr, items.zero_invalid);
                ectx[x] = ctx;
                bx[x] = item_first(items, r);
                cr[x] = ctx > 0 ? (ctx - bx[x] + kChunk - 1) / kChunk : 0;
            }
            total += cr[x];
        }
    }
    const int C = wave_sum_i32(total);
    *invalid_w = false;
#pragma unroll
    for (int x = 0; x < kFlatMaxItems / 64; ++x)
        if (w < B && (w >> 6) == x) *invalid_w = __builtin_amdgcn_readlane(ectx[x], w & 63) < 0;
    int T = (C + W - 1) / W;
    T = T < 1 ? 1 : (T > kMaxSplitTokens / kChunk ? kMaxSplitTokens / kChunk : T);
    const int lo = w * T;
    if (lo >= C) return false;
    const int hi = min(lo + T, C);
    int carry_p = 0, carry_s = 0, found = 0;
#pragma unroll
    for (int x = 0; x < kFlatMaxItems / 64; ++x) {
        if (x >= rounds) break;
        const int r = x * 64 + lane;
        const int c = cr[x];
        const int p = wave_inclusive_scan(c, lane) - c + carry_p;
        const int nsr = c > 0 ? (p + c - 1) / T - p / T + 1 : 0;
        const int sr = wave_inclusive_scan(nsr, lane) - nsr + carry_s;
        const bool hit = r < B && c > 0 && p < hi && p + c > lo;
        const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
        const int n = __builtin_popcountll(static_cast<long long>(m));
        if (k < found + n) {
            uint64_t mm = m;
            for (int i = 0; i < k - found; ++i) mm &= mm - 1;  // drop the lower segments
            const int src = __builtin_ffsll(static_cast<long long>(mm)) - 1;
            const int ps = __builtin_amdgcn_readlane(p, src);
            const int cs = __builtin_amdgcn_readlane(c, src);
            out->req = x * 64 + src;
            out->ctx = __builtin_amdgcn_readlane(ectx[x], src);
            out->nsplit = __builtin_amdgcn_readlane(nsr, src);
            out->first_slot = __builtin_amdgcn_readlane(sr, src);
            const int b0 = __builtin_amdgcn_readlane(bx[x], src);
            out->split = w - ps / T;
            out->begin = b0 + (max(lo, ps) - ps) * kChunk;
            out->end = min(out->ctx, b0 + (min(hi, ps + cs) - ps) * kChunk);
            out->more = ps + cs < hi;
            return true;
        }
        found += n;
        carry_p = __builtin_amdgcn_readlane(p + c, 63);
        carry_s = __builtin_amdgcn_readlane(sr + nsr, 63);
    }
    return false;
}

// ---- the flat plan's index: batches past kFlatMaxItems requests, and reshaped ranges ----
// Scanning every request in every wavefront gets costly for large batches, so one
// 1024-thread workgroup (decode_flat_index_kernel, launched just before the split kernel)
// writes the plan once:
//   idx[0] = T, idx[1] = C,
//   P[0..B]       chunk offset of each request (P[B] = C),
//   S[0..B]       first partial slot of each request (S[B] = total splits),
//   V[0..B)       the first range that holds a chunk of the request,
//   L[0..slots]   the first chunk of each range (L[slots] = C),
//   F[0..slots)   the request holding chunk L[w],
//   O             1 when the plan needed more than `slots` ranges or partial slots (the host
//                 bound in plan_decode rules that out; should it ever be under-computed, the
//                 merge kernel writes NaN to every output row instead of merging partials
//                 that were never written).
// Range w is the chunks [L[w], L[w+1]). Equal ranges: L[w] = min(w * T, C), as in
// flat_segment. Launches of many rounds of wavefronts (snap) reshape them, since the
// dispatcher evens out unequal ranges there and a request cut in two costs a second
// segment (a pipeline start, a partial write and a merge):
// - whole requests: when the longest request is short next to one resident wavefront's
//   share, each request gets its own ranges (pieces of at most kMaxSplitTokens tokens);
// - snapped ranges otherwise: a range start within min(T / 2, (kMaxSplitTokens / kChunk -
//   T) / 2) chunks of a request boundary moves to the nearer boundary, so a request of
//   about T chunks runs whole in one wavefront and no range outgrows a split.
__device__ __forceinline__ int items_live(const ItemArgs& items) {
    int B = items.num_items;
    if (items.item_count != nullptr) B = min(B, *items.item_count);
    return B;
}

__device__ __forceinline__ int item_chunks(const int32_t* __restrict__ context_lens,
                                           const ItemArgs& items, int mbpr, int r, int* ectx) {
    const int req = items.item_req != nullptr ? items.item_req[r] : r;
    const int ctx = effective_ctx(context_lens[req], mbpr, items.zero_invalid);
    *ectx = ctx;
    return ctx > 0 ? (ctx - item_first(items, r) + kChunk - 1) / kChunk : 0;
}

// Exclusive prefix sum of v over the 1024 threads of the block (s_part: 16 ints of LDS);
// *total receives the sum of all. Every thread must call it.
__device__ int block_exclusive_scan_1024(int v, int* s_part, int* total) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int incl = wave_inclusive_scan(v, lane);
    if (lane == 63) s_part[wave] = incl;
    __syncthreads();
    int base = 0, all = 0;
#pragma unroll
    for (int x = 0; x < 16; ++x) {
        const int t = s_part[x];
        base += x < wave ? t : 0;
        all += t;
    }
    __syncthreads();
    *total = all;
    return base + incl - v;
}

struct FlatIndex {
    int32_t *P, *S, *V, *L, *F, *O;
};

__device__ __forceinline__ FlatIndex flat_index_arrays(int32_t* idx, int num_items, int slots) {
    FlatIndex x;
    x.P = idx + 2;
    x.S = x.P + num_items + 1;
    x.V = x.S + num_items + 1;
    x.L = x.V + num_items;
    x.F = x.L + slots + 1;
    x.O = x.F + slots;
    return x;
}

// The last range starting at or before chunk c (c < C). L[w] lies within T / 2 of w * T, so
// the search starts just above c / T and steps down at most a few ranges.
__device__ __forceinline__ int range_of(const int32_t* L, int c, int T, int slots) {
    int w = min(slots, (c + T) / T);
    while (L[w] > c) --w;
    return w;
}

__global__ __launch_bounds__(1024) void decode_flat_index_kernel(
    const int32_t* __restrict__ context_lens, ItemArgs items, int mbpr, int W, int slots,
    int snap, int resident, int32_t* __restrict__ idx) {
    __shared__ int s_part[16];
    __shared__ int s_max[16];
    constexpr int kMaxT = kMaxSplitTokens / kChunk;
    const int B = items_live(items);
    const FlatIndex x = flat_index_arrays(idx, items.num_items, slots);
    const int per = (B + 1023) / 1024;
    const int lo = static_cast<int>(threadIdx.x) * per;
    const int hi = min(B, lo + per);
    int e;
    int sum = 0, cmax = 0;
    for (int r = lo; r < hi; ++r) {
        const int c = item_chunks(context_lens, items, mbpr, r, &e);
        sum += c;
        cmax = max(cmax, c);
    }
    cmax = wave_max_int(cmax);
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = cmax;
    int C;
    int run = block_exclusive_scan_1024(sum, s_part, &C);  // its barriers publish s_max
#pragma unroll
    for (int v = 0; v < 16; ++v) cmax = max(cmax, s_max[v]);
    int T = (C + W - 1) / W;
    T = T < 1 ? 1 : (T > kMaxT ? kMaxT : T);
    // Whole rows: the longest request holds at most half of one resident wavefront's share of
    // the launch, so one range per request (pieces of at most kMaxT chunks) leaves no tail
    // worth balancing, and no request is cut into two segments.
    const bool rows = snap && 2 * static_cast<int64_t>(cmax) * resident <= C;
    if (rows) {
        int npieces = 0;
        for (int r = lo; r < hi; ++r) {
            const int c = item_chunks(context_lens, items, mbpr, r, &e);
            npieces += (c + kMaxT - 1) / kMaxT;
        }
        int NS;
        int srun = block_exclusive_scan_1024(npieces, s_part, &NS);
        for (int r = lo; r < hi; ++r) {
            const int c = item_chunks(context_lens, items, mbpr, r, &e);
            const int ns = (c + kMaxT - 1) / kMaxT;
            const int len = ns > 0 ? (c + ns - 1) / ns : 0;
            x.P[r] = run;
            x.S[r] = srun;
            x.V[r] = srun;
            for (int k = 0; k < ns && srun + k < slots; ++k) {
                x.L[srun + k] = run + k * len;
                x.F[srun + k] = r;
            }
            run += c;
            srun += ns;
        }
        for (int w = NS + static_cast<int>(threadIdx.x); w <= slots; w += 1024) x.L[w] = C;
        if (threadIdx.x == 0) {
            idx[0] = T;
            idx[1] = C;
            x.P[B] = C;
            x.S[B] = NS;
            *x.O = NS > slots ? 1 : 0;
        }
        return;
    }
    // Range starts: every grid point w * T < C lies in exactly one non-empty request. A start
    // moves by at most `slack` chunks, so a range holds at most T + 2 * slack chunks, within
    // the split kernel's table load.
    const int slack = snap ? min(T / 2, (kMaxT - T) / 2) : -1;
    for (int r = lo; r < hi; ++r) {
        const int c = item_chunks(context_lens, items, mbpr, r, &e);
        x.P[r] = run;
        for (int w = (run + T - 1) / T; w * T < run + c && w < slots; ++w) {
            const int dl = w * T - run, dr = run + c - w * T;
            int start = w * T, req = r;
            if (dl <= slack && dl <= dr) {
                start = run;
            } else if (dr <= slack) {
                start = run + c;
                req = r + 1;
            }
            x.L[w] = start;
            x.F[w] = req;
        }
        run += c;
    }
    for (int w = (C + T - 1) / T + static_cast<int>(threadIdx.x); w <= slots; w += 1024)
        x.L[w] = C;
    if (threadIdx.x == 0) x.P[B] = C;
    __syncthreads();  // L is complete (workgroup-scope visibility of the global writes)
    // Splits of each request: the ranges from the one holding its first chunk to the one
    // holding its last (a snapped range that starts and ends on one boundary is empty and
    // never the last range at or before a chunk).
    int nsum = 0;
    for (int r = lo; r < hi; ++r) {
        const int p = x.P[r], q = x.P[r + 1];
        if (q > p) {
            const int v = range_of(x.L, p, T, slots);
            x.V[r] = v;
            nsum += range_of(x.L, q - 1, T, slots) - v + 1;
        }
    }
    int NS;
    int srun = block_exclusive_scan_1024(nsum, s_part, &NS);
    for (int r = lo; r < hi; ++r) {
        const int p = x.P[r], q = x.P[r + 1];
        x.S[r] = srun;
        if (q > p) srun += range_of(x.L, q - 1, T, slots) - x.V[r] + 1;
    }
    if (threadIdx.x == 0) {
        idx[0] = T;
        idx[1] = C;
        x.S[B] = NS;
        *x.O = (NS > slots || (C + T - 1) / T > slots) ? 1 : 0;
    }
}

// flat_segment from the index: the k-th request with chunks in range w.
__device__ __forceinline__ bool flat_segment_indexed(const int32_t* __restrict__ idx,
                                                     const int32_t* __restrict__ context_lens,
                                                     const ItemArgs& items, int mbpr,
                                                     int slots, int w, int k, FlatSegment* out,
                                                     bool* invalid_w) {
    const int B = __builtin_amdgcn_readfirstlane(items_live(items));
    const FlatIndex x = flat_index_arrays(const_cast<int32_t*>(idx), items.num_items, slots);
    *invalid_w = false;
    if (w < B) {
        int e;
        item_chunks(context_lens, items, mbpr, w, &e);
        *invalid_w = __builtin_amdgcn_readfirstlane(e) < 0;
    }
    const int lo = __builtin_amdgcn_readfirstlane(x.L[w]);
    const int hi = __builtin_amdgcn_readfirstlane(x.L[w + 1]);
    if (lo >= hi) return false;
    int found = 0;
    for (int r = __builtin_amdgcn_readfirstlane(x.F[w]); r < B; ++r) {
        const int p = __builtin_amdgcn_readfirstlane(x.P[r]);
        if (p >= hi) break;
        const int c = __builtin_amdgcn_readfirstlane(x.P[r + 1]) - p;
        if (c == 0) continue;
        if (found++ < k) continue;
        int e;
        item_chunks(context_lens, items, mbpr, r, &e);
        const int s0 = __builtin_amdgcn_readfirstlane(x.S[r]);
        out->req = r;
        out->ctx = __builtin_amdgcn_readfirstlane(e);
        out->nsplit = __builtin_amdgcn_readfirstlane(x.S[r + 1]) - s0;
        out->first_slot = s0;
        const int b0 = __builtin_amdgcn_readfirstlane(item_first(items, r));
        out->split = w - __builtin_amdgcn_readfirstlane(x.V[r]);
        out->begin = b0 + (max(lo, p) - p) * kChunk;
        out->end = min(out->ctx, b0 + (min(hi, p + c) - p) * kChunk);
        out->more = p + c < hi;
        return true;
    }
    return false;
}

// Log-sum-exp merge of the ns splits of one (item, head) row by one wavefront; writes bf16.
// Split weights are computed one split per lane and broadcast with readlane; every lane then
// accumulates its D/64 dims over the splits, 8 splits' partial rows loaded before any is
// used so a row costs a couple of memory latencies, not one per split.

template <int D>
__device__ void merge_row(const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
                          int64_t base, int ns, float eps, __bf16* __restrict__ o, int lane,
                          int dr = D) {
    constexpr int kPer = MergeCols<D>::kPer;
    constexpr int kBatch = 8;
    // The first batch of partial rows is loaded together with the (m, l) pairs, before the
    // row max is known (two memory round trips per row instead of three).
    float v_first[kBatch][kPer];
    {
        const float* po = ws_o + base * D;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int t = min(u, ns - 1);
#pragma unroll
            for (int x = 0; x < kPer; ++x) v_first[u][x] = po[t * D + MergeCols<D>::col(lane, x)];
        }
    }
    float mmax = kNegInf;
    for (int s = lane; s < ns; s += 64) mmax = fmaxf(mmax, ws_ml[(base + s) * 2]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, off));
    float acc[kPer];
#pragma unroll
    for (int x = 0; x < kPer; ++x) acc[x] = 0.f;
    float lsum = 0.f;
    if (mmax != kNegInf) {
        for (int sb = 0; sb < ns; sb += 64) {
            const int s = sb + lane;
            float w = 0.f;
            if (s < ns) {
                w = __builtin_amdgcn_exp2f(ws_ml[(base + s) * 2] - mmax);
                lsum += ws_ml[(base + s) * 2 + 1] * w;
            }
            const int nt = min(64, ns - sb);
            const float* po = ws_o + (base + sb) * D;
            for (int t0 = 0; t0 < nt; t0 += kBatch) {
                float v[kBatch][kPer];
                if (sb == 0 && t0 == 0) {
#pragma unroll
                    for (int u = 0; u < kBatch; ++u)
#pragma unroll
                        for (int x = 0; x < kPer; ++x) v[u][x] = v_first[u][x];
                } else {
#pragma unroll
                    for (int u = 0; u < kBatch; ++u) {
                        const int t = min(t0 + u, nt - 1);  // clamped: a repeat's weight is 0
#pragma unroll
                        for (int x = 0; x < kPer; ++x)
                            v[u][x] = po[t * D + MergeCols<D>::col(lane, x)];
                    }
                }
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const int t = t0 + u;
                    const float wt = t < nt ? __int_as_float(__builtin_amdgcn_readlane(
                                                  __float_as_int(w), t & 63))
                                            : 0.f;
#pragma unroll
                    for (int x = 0; x < kPer; ++x) acc[x] += v[u][x] * wt;
                }
            }
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) lsum += __shfl_xor(lsum, off);
    const float inv = lsum > 0.f ? 1.f / (lsum + eps) : 0.f;
#pragma unroll
    for (int x = 0; x < kPer; ++x)
        if (lane * kPer + x < dr) o[lane * kPer + x] = static_cast<__bf16>(acc[x] * inv);
}

// Log-sum-exp merge of a row whose partials sit in two lists: ns split partials at `base`
// of the workspace and sn shared-prefix partials at `sbase` of the shared area (the rows of
// decode_attention_shared). A plain loop: these rows are few per launch.
template <int D>
__device__ void merge_row_two(const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
                              int64_t base, int ns, const float* __restrict__ sh_o,
                              const float* __restrict__ sh_ml, int64_t sbase, int sn,
                              float eps, __bf16* __restrict__ o, int lane, int dr) {
    constexpr int kPer = MergeCols<D>::kPer;
    constexpr int kBatch = 8;
    const int n = ns + sn;
    auto row = [&](int t) {
        return t < ns ? ws_o + (base + t) * D : sh_o + (sbase + t - ns) * D;
    };
    auto ml = [&](int t, int w) {
        return t < ns ? ws_ml[(base + t) * 2 + w] : sh_ml[(sbase + t - ns) * 2 + w];
    };
    float mmax = kNegInf;
    for (int t = lane; t < n; t += 64) mmax = fmaxf(mmax, ml(t, 0));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, off));
    float acc[kPer];
#pragma unroll
    for (int x = 0; x < kPer; ++x) acc[x] = 0.f;
    float lsum = 0.f;
    if (mmax != kNegInf) {
        for (int tb = 0; tb < n; tb += 64) {
            // lane t: the weight of partial tb + t
            const int t = tb + lane;
            float w = 0.f;
            if (t < n) {
                w = __builtin_amdgcn_exp2f(ml(t, 0) - mmax);
                lsum += ml(t, 1) * w;
            }
            const int nt = min(64, n - tb);
            for (int t0 = 0; t0 < nt; t0 += kBatch) {
                float v[kBatch][kPer];
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {  // clamped: a repeat's weight is 0
                    const float* po = row(tb + min(t0 + u, nt - 1));
#pragma unroll
                    for (int x = 0; x < kPer; ++x) v[u][x] = po[MergeCols<D>::col(lane, x)];
                }
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const float wt = t0 + u < nt ? __int_as_float(__builtin_amdgcn_readlane(
                                                       __float_as_int(w), t0 + u))
                                                 : 0.f;
#pragma unroll
                    for (int x = 0; x < kPer; ++x) acc[x] += v[u][x] * wt;
                }
            }
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) lsum += __shfl_xor(lsum, off);
    const float inv = lsum > 0.f ? 1.f / (lsum + eps) : 0.f;
#pragma unroll
    for (int x = 0; x < kPer; ++x)
        if (lane * kPer + x < dr) o[lane * kPer + x] = static_cast<__bf16>(acc[x] * inv);
}

// ---- shared-prefix decode (decode_attention_shared) ----
// Requests whose block-table rows start with the same block ids hold one cached prompt
// prefix in common (the reference counts such prefix-cache hits in BlockTable::shared_count,
// src/cache/block.h:85-97, when KVCacheManager::lookup_prefix_cache reuses the blocks,
// src/cache/kv_cache_manager.cpp:93-173). A planner groups them on the device by their first
// block id; a group's common prefix -- the leading block ids all members share, cut to whole
// 32-token chunks and to before every member's last position -- is attended once per
// subgroup of up to 16 / G members, whose G query heads each fill the 16 columns of the
// decode MFMA tile together (one request alone uses G of them), so each K/V byte of the
// prefix is read once per subgroup instead of once per request. Each member's positions from
// the end of the prefix on run through the ordinary split plan (items start there), and the
// merge adds the prefix partials to the row. Requests in no group run as in plain decode.
constexpr int kSharedSplitTokens = 128;   // prefix positions per shared-kernel wavefront
constexpr int kSharedMinTokens = 64;      // shorter common prefixes are not worth a subgroup
constexpr int kSharedMaxItems = 2048;     // the planner's hash table holds 2x this many keys
constexpr int kSharedHash = 4096;
constexpr int kSharedCols = 16;           // columns of the 16x16x32 MFMA tile
constexpr int kSharedSlotsPerHead = 128;  // shared-kernel wavefronts per kv head

struct SharedPlan {
    int32_t* nsub;      // [1] subgroups
    int32_t* sub_len;   // [B] prefix positions of subgroup s
    int32_t* sub_n;     // [B] members of subgroup s
    int32_t* sub_mem;   // [B][16] its members (items)
    int32_t* begin;     // [B] first position item r attends in the split plan
    int32_t* sh_splits; // [B] prefix partials of item r's rows
};

__global__ __launch_bounds__(1024) void decode_shared_plan_kernel(
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ context_lens, int B,
    int mbpr, int M, SharedPlan sp) {
    __shared__ int h_key[kSharedHash];
    __shared__ int h_lead[kSharedHash];
    __shared__ int h_count[kSharedHash];
    __shared__ int h_minctx[kSharedHash];
    __shared__ int h_common[kSharedHash];
    __shared__ int h_base[kSharedHash];
    __shared__ int h_slot[kSharedMaxItems];  // each request's hash slot (-1: not grouped)
    __shared__ int s_nsub;
    constexpr int kPer = kSharedMaxItems / 1024;
    const int tid = threadIdx.x;
    for (int i = tid; i < kSharedHash; i += 1024) {
        h_key[i] = -1;
        h_lead[i] = 0x7fffffff;
        h_count[i] = 0;
        h_minctx[i] = 0x7fffffff;
        h_common[i] = 0x7fffffff;
        h_base[i] = 0;  // the fill counter until the subgroups are numbered
    }
    if (tid == 0) s_nsub = 0;
    __syncthreads();
    // 1. hash every eligible request on its first block id (decode semantics: a row whose
    //    context is invalid writes zeros and is never grouped)
    int slot[kPer];
#pragma unroll
    for (int x = 0; x < kPer; ++x) {
        slot[x] = -1;
        const int r = tid + 1024 * x;
        if (r >= B) continue;
        sp.begin[r] = 0;
        sp.sh_splits[r] = 0;
        const int ctx = context_lens[r];
        const int key = ctx > kSharedMinTokens && (ctx + kBlock - 1) / kBlock <= mbpr
                            ? block_table[static_cast<int64_t>(r) * mbpr]
                            : -1;
        if (key < 0) continue;
        int h = static_cast<int>((static_cast<uint32_t>(key) * 2654435761u) >> 20) &
                (kSharedHash - 1);
        for (;;) {
            const int prev = atomicCAS(&h_key[h], -1, key);
            if (prev == -1 || prev == key) break;
            h = (h + 1) & (kSharedHash - 1);
        }
        atomicMin(&h_lead[h], r);
        atomicAdd(&h_count[h], 1);
        atomicMin(&h_minctx[h], ctx);
        slot[x] = h;
    }
    __syncthreads();
    // 2. each member's run of block ids equal to the group leader's, within the blocks that
    //    lie wholly before the shortest member's last position: one wavefront per request,
    //    64 ids per step, the first mismatch found by a ballot
#pragma unroll
    for (int x = 0; x < kPer; ++x) h_slot[tid + 1024 * x] = slot[x];
    __syncthreads();
    {
        // four requests per wavefront at a time, so their loads are in flight together
        constexpr int U = 4;
        const int lane = tid & 63;
        for (int r0 = (tid >> 6) * U; r0 < B; r0 += 16 * U) {
            int h[U], nb[U], cb[U], lead[U];
            int nbmax = 0;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = r0 + u;
                h[u] = r < B ? h_slot[r] : -1;
                const bool grouped = h[u] >= 0 && h_count[h[u]] >= 2;
                nb[u] = grouped ? (h_minctx[h[u]] - 1) / kBlock : 0;
                lead[u] = grouped ? h_lead[h[u]] : 0;
                cb[u] = nb[u];
                nbmax = max(nbmax, nb[u]);
            }
            // 128 ids per step (two per lane), all loads of a step in flight together
            for (int j0 = 0; j0 < nbmax; j0 += 128) {
                bool diff[U][2];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int32_t* a = block_table + static_cast<int64_t>(r0 + u) * mbpr;
                    const int32_t* b = block_table + static_cast<int64_t>(lead[u]) * mbpr;
#pragma unroll
                    for (int hx = 0; hx < 2; ++hx) {
                        const int j = j0 + 64 * hx + lane;
                        const bool in = j < cb[u];
                        diff[u][hx] = in && a[in ? j : 0] != b[in ? j : 0];
                    }
                }
                bool more = false;
#pragma unroll
                for (int u = 0; u < U; ++u) {
#pragma unroll
                    for (int hx = 1; hx >= 0; --hx) {  // the lower half's mismatch wins
                        const uint64_t d = __builtin_amdgcn_ballot_w64(diff[u][hx]);
                        if (d != 0)
                            cb[u] = min(cb[u], j0 + 64 * hx +
                                                   __builtin_ffsll(static_cast<long long>(d)) - 1);
                    }
                    more = more || cb[u] > j0 + 128;
                }
                if (!more) break;  // wave-uniform
            }
            if (lane == 0) {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (nb[u] > 0) atomicMin(&h_common[h[u]], cb[u]);
            }
        }
    }
    __syncthreads();
    // 3. groups with a long enough common prefix get ceil(count / M) subgroups
    for (int i = tid; i < kSharedHash; i += 1024) {
        if (h_key[i] < 0 || h_count[i] < 2) continue;
        const int len = min(h_common[i] * kBlock, h_minctx[i] - 1) / kChunk * kChunk;
        if (len < kSharedMinTokens) {
            h_count[i] = 0;
            continue;
        }
        h_common[i] = len;
        h_lead[i] = atomicAdd(&s_nsub, (h_count[i] + M - 1) / M);  // first subgroup
    }
    __syncthreads();
    // 4. members into subgroups (in arrival order: a member's result does not depend on its
    //    column or on the other members of its subgroup)
#pragma unroll
    for (int x = 0; x < kPer; ++x) {
        const int r = tid + 1024 * x;
        const int h = slot[x];
        if (h < 0 || h_count[h] < 2) continue;
        const int i = atomicAdd(&h_base[h], 1);
        const int sub = h_lead[h] + i / M;
        const int len = h_common[h];
        sp.sub_mem[sub * kSharedCols + i % M] = r;
        sp.begin[r] = len;
        sp.sh_splits[r] = (len + kSharedSplitTokens - 1) / kSharedSplitTokens;
        if (i % M == 0) {
            sp.sub_len[sub] = len;
            sp.sub_n[sub] = min(M, h_count[h] - (i / M) * M);
        }
    }
    if (tid == 0) *sp.nsub = s_nsub;
}

// Prefix attention of the subgroups: each wavefront takes work items (128-position piece,
// kv head h, subgroup) in turn. Lane column j holds
// member j / G's query head h G + j % G; the partial (O, m, l) of each member row goes to
// the shared area at ((member * Hq + head) * k + piece).
// Runs in the split kernel's extra workgroups (wg of nwg), beside the split work, which
// needs the same inputs and nothing from it.
template <int D, bool kPad>
__device__ __forceinline__ void shared_prefix_work(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k_cache,
    const __bf16* __restrict__ v_cache, const int32_t* __restrict__ block_table,
    const SharedPlan& sp, float* __restrict__ sh_o, float* __restrict__ sh_ml, int mbpr, int hq,
    int hkv, int sh_k, float scale_log2, int dr, int wg_raw, int nwg) {
    constexpr int S = DecodeShape<D>::kSteps;
    constexpr int NV = DecodeShape<D>::kNV;
    const int ds = kPad ? dr : D;
    const int lane = threadIdx.x & 63;
    // Work item (piece, kv head, subgroup), subgroup fastest: the wavefronts of a workgroup
    // read the same K/V rows (they hit in the CU's cache), and workgroups are renumbered so
    // that consecutive ones run on one XCD (workgroups are dealt to the 8 XCDs in turn),
    // keeping the subgroups of a piece in one L2.
    // nwg: a multiple of 8; the split workgroups before these are a multiple of 8 too
    const int wg = (wg_raw % 8) * (nwg / 8) + wg_raw / 8;
    const int wi = wg * kWavesPerGroup + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = hq / hkv;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int nsub = *sp.nsub;
    const int nwork = nsub * hkv * sh_k;
    for (int w = wi; w < nwork; w += nwg * kWavesPerGroup) {
        const int sub = w % nsub;
        const int h = (w / nsub) % hkv;
        const int piece = w / (nsub * hkv);
        const int len = sp.sub_len[sub];
        const int begin = piece * kSharedSplitTokens;
        if (begin >= len) continue;  // wave-uniform
        const int end = min(len, begin + kSharedSplitTokens);
        const int nmem = sp.sub_n[sub];
        const int32_t* mem = sp.sub_mem + sub * kSharedCols;
        const int m = j / G;
        const bool live = m < nmem;
        const int r = mem[live ? m : 0];
        const int head = h * G + j % G;
        SplitInputs<D> in;
        // block ids: any member's row (the prefix's ids are the same in all of them)
        const int32_t* rb = block_table + static_cast<int64_t>(mem[0]) * mbpr;
        const int lb0 = begin / kBlock;
        const int nblk = (end - begin + kBlock - 1) / kBlock;
        in.bt_lo = lane < nblk ? rb[lb0 + lane] : -1;
        in.bt_hi = lane + 64 < nblk ? rb[lb0 + lane + 64] : -1;
        const __bf16* qv = q + (static_cast<int64_t>(r) * hq + head) * ds;
#pragma unroll
        for (int kk = 0; kk < S; ++kk) {
            const int dim0 = (kk * 4 + g) * 8;
            const bool ok = !kPad || dim0 < dr;
            u32x4 v = load16(qv + (ok ? dim0 : 0));
            if (!live || !ok) v = u32x4{0, 0, 0, 0};
            in.qop[kk] = __builtin_bit_cast(bf16x8, v);
        }
        SoftmaxState<D> st;
        // cached loads (kTL): every subgroup of the group reads these blocks
        run_split<D, false, kPad, true>(k_cache, v_cache, nullptr, nullptr, in, hkv, h, begin,
                                        end, scale_log2, lane, st, dr);
        const float l_tot = wave_sum_xor16_32(st.l);
        if (live) {
            const int64_t slot = (static_cast<int64_t>(r) * hq + head) * sh_k + piece;
            float* po = sh_o + slot * D;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                for (int n = 0; n < NV; ++n) po[NV * (4 * g + rr) + n] = st.acc[n][rr];
            if (g == 0) {
                sh_ml[slot * 2 + 0] = st.m;
                sh_ml[slot * 2 + 1] = l_tot;
            }
        }
    }
}

// F8: the cache holds E4M3 bytes with row scales (k_scale / v_scale); else bf16.
// kPad: head_dim dr < D (see load_chunk); q and output rows hold dr elements.
// kTL: the K/V loads stay in L2 (see kv_load).
// kShared: workgroups from split_wgs on run shared_prefix_work (decode_attention_shared).
// Wavefronts per SIMD: one at D = 192 / 256, three at D = 96 (168 VGPRs, no spills), else
// two.
template <int D, bool F8, bool kPad, bool kTL, bool kShared = false,
          int KS = DecodeShape<D>::kSteps, int NBUF = 2, int kU = 0>
__global__ __launch_bounds__(256, D >= 192 ? 1 : D == 96 ? 3 : 2) void decode_split_kernel(
    const __bf16* __restrict__ q, void* k_cache_v, void* v_cache_v,
    const float* __restrict__ k_scale,
    const float* __restrict__ v_scale, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ context_lens, __bf16* __restrict__ out, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, MergeDesc* __restrict__ desc, ItemArgs items, int mbpr, int hq,
    int hkv, int splits, int split_tokens, int flat_w, int slots, float scale_log2, int dr,
    int rep, const int32_t* __restrict__ flat_idx, SharedPlan sp, float* __restrict__ sh_o,
    float* __restrict__ sh_ml, int sh_k, int split_wgs) {
    if constexpr (kShared && !F8) {
        if (static_cast<int>(blockIdx.x) >= split_wgs) {
            shared_prefix_work<D, kPad>(q, static_cast<const __bf16*>(k_cache_v),
                                        static_cast<const __bf16*>(v_cache_v), block_table, sp,
                                        sh_o, sh_ml, mbpr, hq, hkv, sh_k, scale_log2, dr,
                                        static_cast<int>(blockIdx.x) - split_wgs,
                                        static_cast<int>(gridDim.x) - split_wgs);
            return;
        }
    }
    const int ds = kPad ? dr : D;  // q / output row stride
    constexpr int NV = DecodeShape<D>::kNV;
    using Cache = std::conditional_t<F8, uint8_t, __bf16>;
    // Neither const nor restrict: the fused new-token write (write_new_token) stores
    // through these pointers before the split's loads read the same rows.
    Cache* k_cache = static_cast<Cache*>(k_cache_v);
    Cache* v_cache = static_cast<Cache*>(v_cache_v);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wi = blockIdx.x * kWavesPerGroup + wave;
    // kv_head fastest: the Hkv wavefronts of one (item, split) run side by side and read
    // interleaved 256-byte pieces of the same cache blocks (the layout puts the heads of a
    // slot next to each other), which measured 10-20% faster than split-fastest ordering.
    const int h = wi % hkv;
    const int rest = wi / hkv;
    // flat_w > 0: the on-device flat plan with W = flat_w wavefronts per kv head,
    // partial slots numbered per q-head from 0 to slots; 0: the fixed plan.
    const bool slotted = flat_w != 0;
    const int G = hq / hkv;

    // One split (the item's s-th of ns, over positions [begin, end)). The lane index comes
    // in as an argument: at head dim 96 and the padded head dims up to 128 the flat plan
    // passes it through an empty asm on every segment, so the compiler recomputes the
    // lane-derived addressing per segment instead of holding it across the segment loop
    // (padded: 70 spilled VGPRs without, 17 with, outside the chunk loop; head dim 96 at
    // three wavefronts per SIMD: 27 without, none with); elsewhere that recomputation
    // measured slower.
    auto process = [&](int lane, int item, int s, int ns, int first_slot, int ctx, int begin,
                       int end) __attribute__((always_inline)) {
    const int j = lane & 15;
    const int g = lane >> 4;
    int req, qrow;
    if (!resolve_item(items, item, &req, &qrow)) return;
    if (desc != nullptr && s == 0 && lane < G) {
        const int head = h * G + lane;
        desc[static_cast<int64_t>(item) * hq + head] = MergeDesc{
            slotted ? static_cast<int64_t>(head) * slots + first_slot
                    : (static_cast<int64_t>(item) * hq + head) * splits,
            ctx > 0 ? ns : 0};
    }

    if (ctx < 0) {
        // Decode semantics: invalid context -> zeros (written once, by split 0).
        if (items.zero_invalid && s == 0) {
            for (int x = lane; x < G * ds; x += 64) {
                out[(static_cast<int64_t>(qrow) * hq + h * G) * ds + x] = static_cast<__bf16>(0.0f);
            }
        }
        return;
    }
    if (begin >= end) return;
    if constexpr (!F8) {
        if (items.new_k != nullptr && end == ctx)
            write_new_token<kPad>(k_cache, v_cache, items, block_table + static_cast<int64_t>(req) * mbpr,
                                  req, ctx, hkv / rep, h / rep, ds, lane);
    }
    SplitInputs<D> in;
    load_split_inputs<D, F8, kPad>(q, block_table + static_cast<int64_t>(req) * mbpr, mbpr, qrow,
                                   hq, h, G, begin, end, lane, in, dr);
    SoftmaxState<D> st;
    run_split<D, F8, kPad, kTL, KS, NBUF, kU>(k_cache, v_cache, k_scale, v_scale, in,
                                              hkv / rep, h / rep, begin, end, scale_log2, lane,
                                              st, dr);
    const float l_tot = wave_sum_xor16_32(st.l);
    const bool live = j < G;
    const int head = h * G + j;
    if (ns == 1 && item_shared(items, item) == 0) {
        if (!live) return;
        const float inv = l_tot > 0.f ? 1.f / (l_tot + items.eps) : 0.f;
        __bf16* o = out + (static_cast<int64_t>(qrow) * hq + head) * ds;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint32_t w[NV / 2];
#pragma unroll
            for (int x = 0; x < NV / 2; ++x)
                w[x] = pack_bf16x2(st.acc[2 * x][r] * inv, st.acc[2 * x + 1][r] * inv);
            if (kPad && NV * (4 * g + r) >= dr) continue;  // padded dims
            uint32_t* dst = reinterpret_cast<uint32_t*>(o + NV * (4 * g + r));
#pragma unroll
            for (int x = 0; x < NV / 2; ++x) dst[x] = w[x];
        }
        return;
    }

    // Partial of this split; decode_merge_kernel combines the splits.
    if (!live) return;
    // Partials of one row are contiguous over its splits.
    const int64_t slot = slotted ? static_cast<int64_t>(head) * slots + first_slot + s
                                 : (static_cast<int64_t>(item) * hq + head) * splits + s;
    float* po = ws_o + slot * D;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        if constexpr (NV == 4) {
            *reinterpret_cast<f32x4*>(po + NV * (4 * g + r)) =
                f32x4{st.acc[0][r], st.acc[1][r], st.acc[2][r], st.acc[3][r]};
        } else if constexpr (NV == 8) {
            *reinterpret_cast<f32x4*>(po + NV * (4 * g + r)) =
                f32x4{st.acc[0][r], st.acc[1][r], st.acc[2][r], st.acc[3][r]};
            *reinterpret_cast<f32x4*>(po + NV * (4 * g + r) + 4) =
                f32x4{st.acc[4][r], st.acc[5][r], st.acc[6][r], st.acc[7][r]};
        } else if constexpr (NV == 6) {
#pragma unroll
            for (int x = 0; x < 3; ++x)
                *reinterpret_cast<f32x2*>(po + NV * (4 * g + r) + 2 * x) =
                    f32x2{st.acc[2 * x][r], st.acc[2 * x + 1][r]};
        } else if constexpr (NV == 2) {
            *reinterpret_cast<f32x2*>(po + NV * (4 * g + r)) = f32x2{st.acc[0][r], st.acc[1][r]};
        } else if constexpr (NV == 12) {
#pragma unroll
            for (int x = 0; x < 3; ++x)
                *reinterpret_cast<f32x4*>(po + NV * (4 * g + r) + 4 * x) =
                    f32x4{st.acc[4 * x][r], st.acc[4 * x + 1][r], st.acc[4 * x + 2][r],
                          st.acc[4 * x + 3][r]};
        } else {
#pragma unroll
            for (int n = 0; n < NV; ++n) po[NV * (4 * g + r) + n] = st.acc[n][r];
        }
    }
    if (g == 0) {
        ws_ml[slot * 2 + 0] = st.m;
        ws_ml[slot * 2 + 1] = l_tot;
    }
    };

    if (flat_w > 0) {
        // Flat plan: wavefront `rest` walks the segments of its chunk range; it also owns
        // the zero output and empty merge descriptor of request `rest` when that request's
        // context is invalid (no range holds a chunk of it).
        if (rest >= slots) return;
        const int W = flat_w;
        FlatSegment fs;
        bool invalid_w = false;
        auto segment = [&](int k) __attribute__((always_inline)) {
            return flat_idx != nullptr
                       ? flat_segment_indexed(flat_idx, context_lens, items, mbpr, slots, rest, k,
                                              &fs, &invalid_w)
                       : flat_segment(context_lens, items, mbpr, W, rest, k, lane, &fs,
                                      &invalid_w);
        };
        bool ok = segment(0);
        if (invalid_w) process(lane, rest, 0, 0, 0, -1, 0, 0);
        for (int k = 1; ok; ++k) {
            int lane_k = lane;
            if constexpr ((kPad && D == 128) || D == 96) asm volatile("" : "+v"(lane_k));
            process(lane_k, fs.req, fs.split, fs.nsplit, fs.first_slot, fs.ctx, fs.begin,
                    fs.end);
            if (!fs.more) break;
            ok = segment(k);
        }
        return;
    }
    const int s = rest % splits;
    const int item = rest / splits;
    int req, qrow;
    if (!resolve_item(items, item, &req, &qrow)) return;
    const int ctx = effective_ctx(context_lens[req], mbpr, items.zero_invalid);
    const int b0 = item_first(items, item);
    const int ns = ctx > 0 ? (ctx - b0 + split_tokens - 1) / split_tokens : 0;
    const int begin = b0 + s * split_tokens;
    process(lane, item, s, ns, 0, ctx, begin, ctx > 0 ? min(ctx, begin + split_tokens) : 0);
}

// One workgroup per (item, kv_head) group: decode_group_body.
template <int D, bool F8, bool kPad, bool kTL, int kU = 0>
__global__ __launch_bounds__(64 * GroupShape<D>::kWaves) void decode_group_kernel(
    const __bf16* __restrict__ q, void* k_cache_v, void* v_cache_v,
    const float* __restrict__ k_scale,
    const float* __restrict__ v_scale, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ context_lens, __bf16* __restrict__ out, ItemArgs items,
    int mbpr, int hq, int hkv, float scale_log2, int dr, int rep) {
    constexpr int W = GroupShape<D>::kWaves;
    constexpr int kMaxG = GroupShape<D>::kMaxG;
    __shared__ float lds_o[W * kMaxG * D];
    __shared__ float lds_m[W * kMaxG];
    __shared__ float lds_l[W * kMaxG];
    decode_group_body<D, F8, kPad, kTL, kU>(
        q, k_cache_v, v_cache_v, k_scale, v_scale, block_table, context_lens, out, items, mbpr,
        hq, hkv, scale_log2, dr, rep, static_cast<int>(blockIdx.x),
        [&](int w) { return lds_o + w * kMaxG * D; }, lds_m, lds_l);
}

// One wavefront per (item, q_head) row with more than one split: log-sum-exp merge.
template <int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(
    __bf16* __restrict__ out, const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    const MergeDesc* __restrict__ desc, ItemArgs items, int hq, int dr,
    const int32_t* __restrict__ flat_idx, int slots, const float* __restrict__ sh_o,
    const float* __restrict__ sh_ml, int sh_k) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wi = blockIdx.x * kWavesPerGroup + wave;
    const int head = wi % hq;
    const int item = wi / hq;
    if (item >= items.num_items) return;
    const MergeDesc d = desc[static_cast<int64_t>(item) * hq + head];
    int req, qrow;
    if (!resolve_item(items, item, &req, &qrow)) return;
    if (flat_idx != nullptr && *flat_index_arrays(const_cast<int32_t*>(flat_idx),
                                                  items.num_items, slots).O != 0) {
        // bf16 quiet-NaN bits (the build's -fno-honor-nans makes NaN arithmetic undefined)
        uint16_t* o = reinterpret_cast<uint16_t*>(out + (static_cast<int64_t>(qrow) * hq + head) * dr);
        for (int x = lane; x < dr; x += 64) o[x] = 0x7fc0u;
        return;
    }
    const int sn = item_shared(items, item);
    if (sn > 0) {
        merge_row_two<D>(ws_o, ws_ml, d.base, static_cast<int>(d.ns), sh_o, sh_ml,
                         (static_cast<int64_t>(req) * hq + head) * sh_k, sn, items.eps,
                         out + (static_cast<int64_t>(qrow) * hq + head) * dr, lane, dr);
        return;
    }
    if (d.ns <= 1) return;  // invalid row, or written directly by the split kernel
    merge_row<D>(ws_o, ws_ml, d.base, static_cast<int>(d.ns), items.eps,
                 out + (static_cast<int64_t>(qrow) * hq + head) * dr, lane, dr);
}

struct DecodeWs {
    float* o;
    float* ml;
    MergeDesc* desc;
    int32_t* index;  // the flat plan's index (when plan.flat_index)
};

// Partial rows of the plan: (item, q_head, split) in fixed mode, (q_head, slot) flat.
size_t partial_rows(int num_items, int hq, const DecodePlan& plan) {
    return plan.flat ? static_cast<size_t>(hq) * plan.slots
                         : static_cast<size_t>(num_items) * hq * plan.splits;
}

// Partials (O rows, then (m, l) pairs), then one MergeDesc per (item, q_head) row.
size_t desc_offset(size_t rows, int d) {
    return (rows * (d + 2) * sizeof(float) + 15) & ~static_cast<size_t>(15);
}

// The flat plan's index follows the merge descriptors: T, C, P[B + 1], S[B + 1], F[slots].
size_t index_offset(size_t rows, int d, int num_items, int hq) {
    return (desc_offset(rows, d) + static_cast<size_t>(num_items) * hq * sizeof(MergeDesc) +
            15) & ~static_cast<size_t>(15);
}

size_t index_bytes(int num_items, int slots) {
    // T, C, P[B + 1], S[B + 1], V[B], L[slots + 1], F[slots], O
    return (2 + 3 * static_cast<size_t>(num_items) + 2 + 2 * static_cast<size_t>(slots) + 2) *
           sizeof(int32_t);
}

DecodeWs carve(void* workspace, size_t rows, int d, int num_items, int hq) {
    DecodeWs w{};
    char* p = static_cast<char*>(workspace);
    w.o = reinterpret_cast<float*>(p);
    w.ml = reinterpret_cast<float*>(p + rows * d * sizeof(float));
    w.desc = reinterpret_cast<MergeDesc*>(p + desc_offset(rows, d));
    w.index = reinterpret_cast<int32_t*>(p + index_offset(rows, d, num_items, hq));
    return w;
}

// dr: the head dim of q / cache / output rows (dr == D unless kPad).
// Split-kernel wavefronts resident on the chip at once: 256 CUs x 4 SIMDs x the waves per
// SIMD its registers allow (about 156 / 217 / 430 VGPRs at head dims 64 / 128 / 256).
template <int D>
constexpr int resident_waves() {
    return 1024 * (D <= 64 || D == 96 ? 3 : D <= 128 ? 2 : 1);
}

// The shared-prefix partials the merge adds to the rows of decode_attention_shared.
struct SharedParts {
    float* o = nullptr;   // [B][Hq][k][D]
    float* ml = nullptr;  // [B][Hq][k][2]
    int k = 0;            // partial slots per row
    SharedPlan sp{};      // the planner's output
    int nwg = 0;          // workgroups of the prefix work (a multiple of 8)
};

template <int D, bool F8, bool kPad, int kU = 0>
hipError_t launch_decode(const void* q, const void* k_cache, const void* v_cache,
                         const float* k_scale, const float* v_scale,
                         const int32_t* block_table, const int32_t* context_lens, void* output,
                         const ItemArgs& it, int mbpr, int hq, int hkv, const DecodePlan& plan,
                         void* workspace, hipStream_t stream, int dr,
                         const SharedParts& shared = SharedParts{}) {
    const float scale_log2 = kLog2e / sqrtf(static_cast<float>(dr));
    // Query groups larger than one MFMA N-tile run as `rep` virtual kv heads of hq / hkv /
    // rep query heads each; virtual head v reads cache head v / rep.
    const int rep = decode_head_rep(hq / hkv);
    hkv *= rep;
    // Padded rows, virtual heads, 2-byte pieces and rows that are not whole 128-byte lines
    // (head dim 96: neighbouring kv heads' rows share lines) read lines more than once:
    // those loads stay in L2.
    const bool tl = kPad || rep > 1 || kU != 0 || D % 64 != 0;
    if (plan.group) {
        const int64_t groups = static_cast<int64_t>(it.num_items) * hkv;
        auto go = [&](auto tl_tag) {
            decode_group_kernel<D, F8, kPad, decltype(tl_tag)::value, kU>
                <<<static_cast<unsigned>(groups), 64 * GroupShape<D>::kWaves, 0, stream>>>(
                    static_cast<const __bf16*>(q), const_cast<void*>(k_cache),
                    const_cast<void*>(v_cache), k_scale, v_scale, block_table, context_lens,
                    static_cast<__bf16*>(output), it, mbpr, hq, hkv, scale_log2, dr, rep);
        };
        if (kPad || tl)
            go(std::true_type{});
        else if constexpr (!kPad && D % 64 == 0)
            go(std::false_type{});
        return hipGetLastError();
    }
    const int64_t waves = plan.flat
                              ? static_cast<int64_t>(plan.slots) * hkv
                              : static_cast<int64_t>(it.num_items) * hkv * plan.splits;
    const int grid = static_cast<int>((waves + kWavesPerGroup - 1) / kWavesPerGroup);
    const bool merge = plan.flat || plan.splits > 1 || shared.o != nullptr;
    DecodeWs w{};
    if (merge) w = carve(workspace, partial_rows(it.num_items, hq, plan), D, it.num_items, hq);
    if (plan.flat_index) {
        decode_flat_index_kernel<<<1, 1024, 0, stream>>>(context_lens, it, mbpr, plan.wave_target,
                                                         plan.slots, plan.flat_snap ? 1 : 0,
                                                         resident_waves<D>() / hkv, w.index);
        const hipError_t ie = hipGetLastError();
        if (ie != hipSuccess) return ie;
    }
    const int bw = plan.flat ? plan.wave_target : 0;
    // Shared-prefix decode: the prefix work runs in extra workgroups of the same launch (the
    // split part padded to a multiple of 8 workgroups so the prefix part starts on XCD 0).
    const bool shr = shared.o != nullptr;
    const int split_wgs = shr ? (grid + 7) / 8 * 8 : grid;
    const int total_wgs = split_wgs + (shr ? shared.nwg : 0);
    auto go = [&](auto tl_tag, auto sh_tag) {
        constexpr bool kTLv = decltype(tl_tag)::value;
        constexpr bool kShv = decltype(sh_tag)::value;
        // Padded rows that leave whole K steps empty (head dims 80 / 96 at D = 128, 192 at
        // D = 256): those steps are compiled out -- no loads, no MFMAs, 5-16 fewer VGPRs
        // (the D = 128 kernel's spills go away). Bit-identical; 64 x 4096 positions: d=80
        // 139.4 -> 137.6 us, d=96 154.8 -> 152.3, d=192 195.0 -> 175.8.
        constexpr int KSp = D == 128 ? 3 : D == 256 ? 6 : DecodeShape<D>::kSteps;
        auto kernel = decode_split_kernel<D, F8, kPad, kTLv, kShv>;
        if constexpr (kU != 0) {
            kernel = decode_split_kernel<D, F8, kPad, kTLv, kShv, DecodeShape<D>::kSteps, 2,
                                         kU>;
        } else if constexpr (!F8 && kPad && !kShv && KSp < DecodeShape<D>::kSteps) {
            if (dr <= KSp * 32) kernel = decode_split_kernel<D, F8, kPad, kTLv, kShv, KSp, 2>;
        }
        kernel<<<total_wgs, 256, 0, stream>>>(
            static_cast<const __bf16*>(q), const_cast<void*>(k_cache), const_cast<void*>(v_cache),
            k_scale, v_scale, block_table, context_lens, static_cast<__bf16*>(output), w.o, w.ml,
            w.desc, it, mbpr, hq, hkv,
            plan.splits, plan.split_tokens, bw, plan.slots, scale_log2, dr, rep,
            plan.flat_index ? w.index : nullptr, shared.sp, shared.o, shared.ml, shared.k,
            split_wgs);
    };
    if (shr) {
        if constexpr (!F8 && kU == 0) {
            if (tl)
                go(std::true_type{}, std::true_type{});
            else if constexpr (!kPad && D % 64 == 0)
                go(std::false_type{}, std::true_type{});
        }
    } else if (tl) {
        go(std::true_type{}, std::false_type{});
    } else if constexpr (!kPad && D % 64 == 0) {
        go(std::false_type{}, std::false_type{});
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !merge) return err;
    const int64_t rows = static_cast<int64_t>(it.num_items) * hq;
    const int mgrid = static_cast<int>((rows + kWavesPerGroup - 1) / kWavesPerGroup);
    decode_merge_kernel<D><<<mgrid, 256, 0, stream>>>(static_cast<__bf16*>(output), w.o, w.ml,
                                                      w.desc, it, hq, dr,
                                                      plan.flat_index ? w.index : nullptr,
                                                      plan.slots, shared.o, shared.ml,
                                                      shared.k);
    return hipGetLastError();
}

}  // namespace

DecodePlan plan_decode(int num_items, int num_q_heads, int num_kv_heads, int head_dim,
                       int max_ctx, bool allow_flat, bool fp8, bool allow_group) {
    // Query groups above one MFMA N-tile run as several virtual kv heads (launch_decode).
    num_kv_heads *= decode_head_rep(num_q_heads / num_kv_heads);
    DecodePlan p;
    // Tiny batches: one workgroup per (request, kv_head) merges its parts in LDS (a single
    // launch; these batches are latency-bound).
    if (allow_group && static_cast<int64_t>(num_items) * num_q_heads <= kGroupMaxRows &&
        max_ctx <= kGroupMaxCtx) {
        p.group = true;
        return p;
    }
    const int chunks = max_ctx > 0 ? (max_ctx + kChunk - 1) / kChunk : 1;
    constexpr int kMaxChunksPerSplit = kMaxSplitTokens / kChunk;
    // Small batches keep the fixed plan: their splits are already even and the on-device
    // plan would only add its lookup to a latency-bound launch.
    if (allow_flat && num_items >= kFlatMinItems && chunks > 1) {
        p.flat = true;
        // One workgroup per CU, and at least one range per request and kv head (many short
        // rows would otherwise crowd several segments into each range).
        p.wave_target = static_cast<int>(std::max<int64_t>(
            std::max<int64_t>(1, flat_waves(fp8, head_dim) / num_kv_heads),
            num_items));
        p.flat_snap = static_cast<int64_t>(p.wave_target) * num_kv_heads >= kSnapWaves;
        p.flat_index = num_items > kFlatMaxItems || p.flat_snap;
        // Splits per kv_head: one per range plus one per row boundary inside a range, so at
        // most C/T + B with T >= C/W (or, with T at its cap, B * chunks / cap + B), and
        // never more than one per chunk.
        const int64_t capped =
            static_cast<int64_t>(num_items) * ((chunks + kMaxChunksPerSplit - 1) / kMaxChunksPerSplit);
        const int64_t bound = std::max<int64_t>(p.wave_target, capped) + num_items;
        p.slots = static_cast<int>(std::min<int64_t>(bound, static_cast<int64_t>(num_items) * chunks));
        p.splits = 0;
        p.split_tokens = 0;
        return p;
    }
    // Splits sized for the longest possible row. Batches of 1-3 requests: at most kEvenWaves
    // wavefronts after rounding (one workgroup per CU: a few workgroups more than CUs would
    // leave those CUs running two in a row); measured against the kTargetWaves sizing, one
    // request of 8K / 16K / 32K positions 26.7 / 50.4 / 61.6 -> 18.0 / 23.2 / 32.6 us. Larger
    // batches on this plan (past the flat plan's request limit, or without it) keep
    // kTargetWaves: 300 requests of 100-3000 positions ran 456 -> 497 us with kEvenWaves.
    const int64_t groups = static_cast<int64_t>(num_items) * num_kv_heads;
    const int64_t target = num_items < kFlatMinItems ? kEvenWaves : kTargetWaves;
    int64_t cpw = (groups * chunks + target - 1) / target;
    if (cpw < 1) cpw = 1;
    while (num_items < kFlatMinItems && cpw < chunks &&
           groups * ((chunks + cpw - 1) / cpw) > kEvenWaves)
        ++cpw;
    if (cpw > kMaxChunksPerSplit) cpw = kMaxChunksPerSplit;
    if (cpw > chunks) cpw = chunks;
    p.split_tokens = static_cast<int>(cpw) * kChunk;
    p.splits = (chunks + static_cast<int>(cpw) - 1) / static_cast<int>(cpw);
    return p;
}

int decode_mfma_dim(int head_dim) {
    // The MFMA tile's head dim for a cache of head_dim: native at 64 / 128 / 256; smaller
    // dims run padded with zeros when every per-lane piece (8 dims of K, D/16 of V) is
    // either wholly valid or wholly padding.
    if (head_dim <= 0 || head_dim % 8 != 0) return 0;
    if (head_dim <= 64) return 64;
    if (head_dim <= 128) return 128;
    return head_dim <= 256 && head_dim % 16 == 0 ? 256 : 0;
}

// The decode kernels' head dim: the MFMA size above, except head dims 32, 96 and 192,
// which have tiles of their own (1 / 3 / 6 K steps, 2 / 6 / 12 V dims per lane): in the
// padded tile a quarter or half of every V load's lanes would sit idle. 64 x 4096
// positions: d=32 58.1 -> 47.9 us, d=96 152 -> 146 us, d=192 175.5 -> 150.6 us.
int decode_tile_dim(int head_dim) {
    return head_dim == 32 || head_dim == 96 || head_dim == 192 ? head_dim
                                                               : decode_mfma_dim(head_dim);
}

DecodePlan plan_decode_items(int num_items, int num_q_heads, int num_kv_heads, int head_dim,
                             int max_ctx, bool fp8) {
    // The decode items of a prefill batch: their count is known on the device only, and is
    // often zero (a pure prompt batch). One launch of one workgroup per possible (item,
    // kv_head) costs far less than the split plan's two launches, each of which dispatches a
    // grid sized for the batch's longest context.
    constexpr int64_t kMaxGroups = 2048;
    const int64_t groups = static_cast<int64_t>(num_items) * num_kv_heads *
                           decode_head_rep(num_q_heads / num_kv_heads);
    if (max_ctx <= kGroupMaxCtx && groups <= kMaxGroups) {
        DecodePlan p;
        p.group = true;
        return p;
    }
    return plan_decode(num_items, num_q_heads, num_kv_heads, head_dim, max_ctx, true, fp8);
}

size_t decode_workspace_bytes(int num_items, int num_q_heads, int head_dim,
                              const DecodePlan& plan) {
    if (plan.group || (!plan.flat && plan.splits <= 1)) return 0;
    // partial O (rows of the kernels' head dim) + (m, l) per partial row, then the merge
    // descriptors
    const int d = decode_tile_dim(head_dim);
    const size_t rows = partial_rows(num_items, num_q_heads, plan);
    if (plan.flat_index)
        return index_offset(rows, d, num_items, num_q_heads) +
               index_bytes(num_items, plan.slots);
    return desc_offset(rows, d) +
           static_cast<size_t>(num_items) * num_q_heads * sizeof(MergeDesc);
}

bool decode_fast_supported(int num_q_heads, int num_kv_heads, int head_dim, int block_size) {
    if (block_size != kBlock || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0)
        return false;
    const int G = num_q_heads / num_kv_heads;
    return G >= 1 && decode_mfma_dim(head_dim) != 0;
}

bool decode_fp8_supported(int num_q_heads, int num_kv_heads, int head_dim, int block_size) {
    return decode_fast_supported(num_q_heads, num_kv_heads, head_dim, block_size) &&
           decode_mfma_dim(head_dim) == head_dim;
}

hipError_t decode_attention(const void* q, const void* k_cache, const void* v_cache,
                            const int32_t* block_table, const int32_t* context_lens, void* output,
                            const DecodeItems& items, int max_blocks_per_req, int num_q_heads,
                            int num_kv_heads, int head_dim, int block_size,
                            const DecodePlan& plan, void* workspace, hipStream_t stream) {
    (void)block_size;
    ItemArgs it{items.num_items, items.item_count, items.item_req, items.query_start_loc,
                items.denom_eps, items.zero_invalid ? 1 : 0,
                static_cast<const __bf16*>(items.new_k), static_cast<const __bf16*>(items.new_v),
                items.max_slots};
    const int D = decode_tile_dim(head_dim);
    const bool pad = D != head_dim;
    // Caches whose rows are not 16-byte aligned run the kernels with 4-byte or 2-byte piece
    // loads.
    const uintptr_t cache_bits =
        reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache);
    const int unaligned = (cache_bits & 15u) == 0 ? 0 : (cache_bits & 3u) == 0 ? 4 : 2;
#define CCI_DECODE_U(DD, PP, UU)                                                              \
    launch_decode<DD, false, PP, UU>(q, k_cache, v_cache, nullptr, nullptr, block_table,      \
                                     context_lens, output, it, max_blocks_per_req,            \
                                     num_q_heads, num_kv_heads, plan, workspace, stream,      \
                                     head_dim)
#define CCI_DECODE(DD, PP)                                                                   \
    return unaligned == 0 ? CCI_DECODE_U(DD, PP, 0)                                           \
                          : unaligned == 4 ? CCI_DECODE_U(DD, PP, 4) : CCI_DECODE_U(DD, PP, 2)
    switch (D) {
        case 64:
            if (pad) CCI_DECODE(64, true);
            CCI_DECODE(64, false);
        case 32:
            CCI_DECODE(32, false);
        case 96:
            CCI_DECODE(96, false);
        case 192:
            CCI_DECODE(192, false);
        case 128:
            if (pad) CCI_DECODE(128, true);
            CCI_DECODE(128, false);
        case 256:
            if (pad) CCI_DECODE(256, true);
            CCI_DECODE(256, false);
        default:
            return hipErrorInvalidValue;
    }
#undef CCI_DECODE
#undef CCI_DECODE_U
}

hipError_t decode_attention_fp8(const void* q, const void* k_cache, const void* v_cache,
                                const float* k_scale, const float* v_scale,
                                const int32_t* block_table, const int32_t* context_lens,
                                void* output, const DecodeItems& items, int max_blocks_per_req,
                                int num_q_heads, int num_kv_heads, int head_dim,
                                const DecodePlan& plan, void* workspace, hipStream_t stream) {
    ItemArgs it{items.num_items, items.item_count, items.item_req, items.query_start_loc,
                items.denom_eps, items.zero_invalid ? 1 : 0,
                static_cast<const __bf16*>(items.new_k), static_cast<const __bf16*>(items.new_v),
                items.max_slots};
    switch (head_dim) {
        case 64:
            return launch_decode<64, true, false>(q, k_cache, v_cache, k_scale, v_scale, block_table,
                                           context_lens, output, it, max_blocks_per_req,
                                           num_q_heads, num_kv_heads, plan, workspace, stream, 64);
        case 128:
            return launch_decode<128, true, false>(q, k_cache, v_cache, k_scale, v_scale, block_table,
                                            context_lens, output, it, max_blocks_per_req,
                                            num_q_heads, num_kv_heads, plan, workspace, stream, 128);
        case 256:
            return launch_decode<256, true, false>(q, k_cache, v_cache, k_scale, v_scale, block_table,
                                            context_lens, output, it, max_blocks_per_req,
                                            num_q_heads, num_kv_heads, plan, workspace, stream, 256);
        default:
            return hipErrorInvalidValue;
    }
}

// ---- shared-prefix decode ----
namespace {

struct SharedLayout {
    DecodePlan plan;
    size_t regular, plan_off, o_off, ml_off, total;
    int k;
};

SharedLayout shared_layout(int B, int mbpr, int hq, int hkv, int head_dim) {
    SharedLayout L{};
    // the suffixes: plain decode's split plan (never the group plan, whose rows do not go
    // through the merge), with the merge always on
    L.plan = plan_decode(B, hq, hkv, head_dim, mbpr * kBlock, true, false, false);
    const int d = decode_tile_dim(head_dim);
    const size_t rows = partial_rows(B, hq, L.plan);
    L.regular = L.plan.flat_index ? index_offset(rows, d, B, hq) + index_bytes(B, L.plan.slots)
                                  : desc_offset(rows, d) +
                                        static_cast<size_t>(B) * hq * sizeof(MergeDesc);
    L.regular = (L.regular + 255) & ~static_cast<size_t>(255);
    L.k = (mbpr * kBlock + kSharedSplitTokens - 1) / kSharedSplitTokens;
    L.plan_off = L.regular;
    const size_t plan_ints = 1 + static_cast<size_t>(B) * (3 + kSharedCols + 2);
    L.o_off = (L.plan_off + plan_ints * sizeof(int32_t) + 255) & ~static_cast<size_t>(255);
    const size_t parts = static_cast<size_t>(B) * hq * L.k;
    L.ml_off = L.o_off + parts * d * sizeof(float);
    L.total = L.ml_off + parts * 2 * sizeof(float);
    return L;
}

template <int D, bool kPad>
hipError_t launch_decode_shared(const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* block_table, const int32_t* context_lens,
                                void* output, int B, int mbpr, int hq, int hkv, int dr,
                                const SharedLayout& L, char* ws, hipStream_t stream) {
    int32_t* pi = reinterpret_cast<int32_t*>(ws + L.plan_off);
    SharedPlan sp;
    sp.nsub = pi;
    sp.sub_len = pi + 1;
    sp.sub_n = sp.sub_len + B;
    sp.begin = sp.sub_n + B;
    sp.sh_splits = sp.begin + B;
    sp.sub_mem = sp.sh_splits + B;
    float* sh_o = reinterpret_cast<float*>(ws + L.o_off);
    float* sh_ml = reinterpret_cast<float*>(ws + L.ml_off);
    const int G = hq / hkv;
    decode_shared_plan_kernel<<<1, 1024, 0, stream>>>(block_table, context_lens, B, mbpr,
                                                      kSharedCols / G, sp);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int waves = kSharedSlotsPerHead * hkv;
    const int nwg = ((waves + kWavesPerGroup - 1) / kWavesPerGroup + 7) / 8 * 8;
    ItemArgs it{};
    it.num_items = B;
    it.eps = 1e-6f;
    it.zero_invalid = 1;
    it.begin = sp.begin;
    it.sh_splits = sp.sh_splits;
    SharedParts parts;
    parts.o = sh_o;
    parts.ml = sh_ml;
    parts.k = L.k;
    parts.sp = sp;
    parts.nwg = nwg;
    return launch_decode<D, false, kPad>(q, k_cache, v_cache, nullptr, nullptr, block_table,
                                         context_lens, output, it, mbpr, hq, hkv, L.plan, ws,
                                         stream, dr, parts);
}

}  // namespace

bool decode_shared_supported(int batch_size, int num_q_heads, int num_kv_heads, int head_dim,
                             int block_size) {
    if (!decode_fast_supported(num_q_heads, num_kv_heads, head_dim, block_size)) return false;
    const int G = num_q_heads / num_kv_heads;
    return batch_size >= 1 && batch_size <= kSharedMaxItems && G <= kSharedCols / 2;
}

size_t decode_shared_workspace_bytes(int batch_size, int max_blocks_per_req, int num_q_heads,
                                     int num_kv_heads, int head_dim) {
    return shared_layout(batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim)
        .total;
}

hipError_t decode_attention_shared(const void* q, const void* k_cache, const void* v_cache,
                                   const int32_t* block_table, const int32_t* context_lens,
                                   void* output, int batch_size, int max_blocks_per_req,
                                   int num_q_heads, int num_kv_heads, int head_dim,
                                   void* workspace, hipStream_t stream) {
    const SharedLayout L = shared_layout(batch_size, max_blocks_per_req, num_q_heads,
                                         num_kv_heads, head_dim);
    char* ws = static_cast<char*>(workspace);
    const int D = decode_tile_dim(head_dim);
    const bool pad = D != head_dim;
#define CCI_SHARED(DD, PP)                                                                  \
    return launch_decode_shared<DD, PP>(q, k_cache, v_cache, block_table, context_lens,    \
                                        output, batch_size, max_blocks_per_req, num_q_heads, \
                                        num_kv_heads, head_dim, L, ws, stream)
    switch (D) {
        case 64:
            if (pad) CCI_SHARED(64, true);
            CCI_SHARED(64, false);
        case 32:
            CCI_SHARED(32, false);
        case 96:
            CCI_SHARED(96, false);
        case 192:
            CCI_SHARED(192, false);
        case 128:
            if (pad) CCI_SHARED(128, true);
            CCI_SHARED(128, false);
        case 256:
            if (pad) CCI_SHARED(256, true);
            CCI_SHARED(256, false);
        default:
            return hipErrorInvalidValue;
    }
#undef CCI_SHARED
}

}  // namespace ccinfer::hipk
