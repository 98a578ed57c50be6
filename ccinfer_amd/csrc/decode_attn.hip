// Paged decode attention for gfx950: split-KV (flash-decoding) on bf16 MFMA tiles.
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
#include "kernels.hpp"

namespace ccinfer::hipk {
namespace {

constexpr int kBlock = 16;        // tokens per KV block (the reference's kKVBlockSize)
constexpr int kChunk = 32;        // tokens per PV MFMA
constexpr int kWavesPerGroup = 4;
constexpr int kMaxSplitTokens = 2048;  // 128 blocks: two table entries per lane
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
// registers per piece in flight: 48-1198 spilled VGPRs here, 7.6x instead of 1.7x.)
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

// Log-sum-exp merge of the ns splits of one (item, head) row by one wavefront; writes bf16.
// Split weights are computed one split per lane and broadcast with readlane; every lane then
// accumulates its D/64 dims over the splits, 8 splits' partial rows loaded before any is
// used so a row costs a couple of memory latencies, not one per split.
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
// Wavefronts per SIMD: one at D = 256, three at D = 96 (168 VGPRs, no spills), else two.
template <int D, bool F8, bool kPad, bool kTL, bool kShared = false,
          int KS = DecodeShape<D>::kSteps, int NBUF = 2, int kU = 0>
__global__ __launch_bounds__(256, D == 256 ? 1 : D == 96 ? 3 : 2) void decode_split_kernel(
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

// Single-launch decode for batches with few (item, kv_head) groups: one workgroup of W
// wavefronts per group, wavefront w attending over the w-th of W equal parts of the
// context; the parts are merged through LDS with the same log-sum-exp weighting as
// merge_row, so no second kernel and no workspace. (For many groups the flat split plan
// spreads ragged contexts better.)
template <int D>
struct GroupShape {
    static constexpr int kWaves = D <= 128 ? 8 : 4;  // two wavefronts per SIMD at <= 256 VGPRs
    static constexpr int kMaxG = 16;                 // LDS: kWaves * 16 * D floats = 64 KiB
};

template <int D, bool F8, bool kPad, bool kTL, int kU = 0>
__global__ __launch_bounds__(64 * GroupShape<D>::kWaves) void decode_group_kernel(
    const __bf16* __restrict__ q, void* k_cache_v, void* v_cache_v,
    const float* __restrict__ k_scale,
    const float* __restrict__ v_scale, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ context_lens, __bf16* __restrict__ out, ItemArgs items,
    int mbpr, int hq, int hkv, float scale_log2, int dr, int rep) {
    const int ds = kPad ? dr : D;  // q / output row stride
    constexpr int W = GroupShape<D>::kWaves;
    constexpr int NV = DecodeShape<D>::kNV;
    constexpr int kMaxG = GroupShape<D>::kMaxG;
    using Cache = std::conditional_t<F8, uint8_t, __bf16>;
    __shared__ float lds_o[W * kMaxG * D];
    __shared__ float lds_m[W * kMaxG];
    __shared__ float lds_l[W * kMaxG];
    // Neither const nor restrict: the fused new-token write (write_new_token) stores
    // through these pointers before the split's loads read the same rows.
    Cache* k_cache = static_cast<Cache*>(k_cache_v);
    Cache* v_cache = static_cast<Cache*>(v_cache_v);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = blockIdx.x % hkv;
    const int item = blockIdx.x / hkv;
    int req, qrow;
    if (!resolve_item(items, item, &req, &qrow)) return;  // workgroup-uniform
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
        float* po = lds_o + (wave * kMaxG + j) * D;
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
#pragma unroll
                for (int x = 0; x < kPer; ++x)
                    acc[x] += lds_o[(w * kMaxG + jj) * D + MergeCols<D>::col(lane, x)] * wt;
            }
        }
        const float inv = lsum > 0.f ? 1.f / (lsum + items.eps) : 0.f;
        __bf16* o = out + (static_cast<int64_t>(qrow) * hq + h * G + jj) * ds;
#pragma unroll
        for (int x = 0; x < kPer; ++x)
            if (lane * kPer + x < dr) o[lane * kPer + x] = static_cast<__bf16>(acc[x] * inv);
    }
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

// Smallest r with G % r == 0 and G / r <= 16 (one MFMA N-tile of query heads).
int decode_head_rep(int G) {
    int r = (G + 15) / 16;
    while (G % r != 0) ++r;
    return r;
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

// The decode kernels' head dim: the MFMA size above, except head dim 96, which has a tile
// of its own (3 K steps, 6 V dims per lane): in the 128 tile a quarter of every V load's
// lanes sit idle and the same registers hold 12 KB of K/V per chunk instead of 16, and the
// loads in flight are what bounds this kernel.
int decode_tile_dim(int head_dim) {
    return head_dim == 96 ? 96 : decode_mfma_dim(head_dim);
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
        case 96:
            CCI_DECODE(96, false);
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
        case 96:
            CCI_SHARED(96, false);
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
