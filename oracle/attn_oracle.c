/*
 * CPU oracle for the paged-attention hot path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker;
 * the shipped library never links it. Function-by-function citations of the
 * reference (7QiC/ccInfer) are in attn_oracle.h and on each function below.
 *
 * Accumulation is fp32 in the same order as the reference's scalar CPU code
 * (sequential over head_dim, then over context positions).
 */
#include "attn_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* bf16 <-> fp32, round to nearest even on the 16 dropped mantissa bits.       */
/* ------------------------------------------------------------------------- */
uint16_t orc_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0) {
        return (uint16_t)((u >> 16) | 0x0040u); /* NaN stays NaN (quiet) */
    }
    const uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_f32_to_bf16_array(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_bf16(src[i]);
}

/* src/kernel/attention/attn_common.cuh:7-27 */
int orc_kv_base_offset(int ctx_pos, int kv_head, int head_dim, int num_kv_heads,
                       int cache_block_size, int max_blocks_per_req, const int32_t* req_blocks,
                       int64_t* out) {
    const int logical_block = ctx_pos / cache_block_size;
    const int offset_in_block = ctx_pos - logical_block * cache_block_size;
    if (logical_block < 0 || logical_block >= max_blocks_per_req) return 0;
    const int physical_block = req_blocks[logical_block];
    if (physical_block < 0) return 0;
    const int64_t slot = (int64_t)physical_block * cache_block_size + offset_in_block;
    *out = (slot * num_kv_heads + kv_head) * (int64_t)head_dim;
    return 1;
}

/* src/kernel/attention/write_kv_cache.cu:12-34 */
void orc_write_kv_cache(const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_cache,
                        uint16_t* v_cache, const int32_t* slot_mapping, int total_tokens,
                        int n_kv_heads, int head_dim, int max_slots) {
    const int64_t row = (int64_t)n_kv_heads * head_dim;
    for (int t = 0; t < total_tokens; ++t) {
        const int slot = slot_mapping[t];
        if (slot < 0 || slot >= max_slots) continue;
        memcpy(k_cache + (int64_t)slot * row, k_new + (int64_t)t * row, (size_t)row * 2);
        memcpy(v_cache + (int64_t)slot * row, v_new + (int64_t)t * row, (size_t)row * 2);
    }
}

/* ------------------------------------------------------------------------- */
/* One (query vector, kv_head) attention over positions [0, visible) of one    */
/* request's block-table row. Invalid positions (logical block out of range or  */
/* block id < 0) are skipped. `eps` is added to the softmax denominator:        */
/* decode uses 1e-6 (decode_attn.cu:455), prefill uses 0 (prefill_attn.cu:238). */
/* Writes zeros when no position is valid (both kernels end with 0 there).      */
/* ------------------------------------------------------------------------- */
static void attend_one(const uint16_t* qv, const uint16_t* k_cache, const uint16_t* v_cache,
                       const int32_t* req_blocks, int visible, int kv_head, int head_dim,
                       int num_kv_heads, int block_size, int mbpr, float scale, float eps,
                       float* scores, int64_t* bases, float* out) {
    float max_score = -INFINITY;
    int any = 0;
    for (int pos = 0; pos < visible; ++pos) {
        int64_t base;
        if (!orc_kv_base_offset(pos, kv_head, head_dim, num_kv_heads, block_size, mbpr,
                                req_blocks, &base)) {
            bases[pos] = -1;
            continue;
        }
        bases[pos] = base;
        float s = 0.0f;
        for (int d = 0; d < head_dim; ++d) {
            s += orc_bf16_to_f32(qv[d]) * orc_bf16_to_f32(k_cache[base + d]);
        }
        s *= scale;
        scores[pos] = s;
        if (s > max_score) max_score = s;
        any = 1;
    }
    for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
    if (!any) return;
    float denom = 0.0f;
    for (int pos = 0; pos < visible; ++pos) {
        if (bases[pos] < 0) continue;
        scores[pos] = expf(scores[pos] - max_score);
        denom += scores[pos];
    }
    const float inv = 1.0f / (denom + eps);
    for (int d = 0; d < head_dim; ++d) {
        float acc = 0.0f;
        for (int pos = 0; pos < visible; ++pos) {
            if (bases[pos] < 0) continue;
            acc += (scores[pos] * inv) * orc_bf16_to_f32(v_cache[bases[pos] + d]);
        }
        out[d] = acc;
    }
}

/* ------------------------------------------------------------------------- */
/* Thread pool helper: run fn(i, ctx) for i in [0, n) over nthreads workers.   */
/* ------------------------------------------------------------------------- */
typedef void (*work_fn)(int64_t i, void* ctx, float* scores, int64_t* bases);

typedef struct {
    work_fn fn;
    void* ctx;
    int64_t n;
    int64_t begin, end;
    int max_ctx;
} worker_arg;

static void* worker_main(void* p) {
    worker_arg* a = (worker_arg*)p;
    float* scores = (float*)malloc(sizeof(float) * (size_t)(a->max_ctx > 0 ? a->max_ctx : 1));
    int64_t* bases = (int64_t*)malloc(sizeof(int64_t) * (size_t)(a->max_ctx > 0 ? a->max_ctx : 1));
    for (int64_t i = a->begin; i < a->end; ++i) a->fn(i, a->ctx, scores, bases);
    free(scores);
    free(bases);
    return NULL;
}

static void run_parallel(work_fn fn, void* ctx, int64_t n, int nthreads, int max_ctx) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > n) nthreads = (int)(n > 0 ? n : 1);
    worker_arg* args = (worker_arg*)calloc((size_t)nthreads, sizeof(worker_arg));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    for (int t = 0; t < nthreads; ++t) {
        args[t].fn = fn;
        args[t].ctx = ctx;
        args[t].n = n;
        args[t].begin = n * t / nthreads;
        args[t].end = n * (t + 1) / nthreads;
        args[t].max_ctx = max_ctx;
    }
    if (nthreads == 1) {
        worker_main(&args[0]);
    } else {
        for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, worker_main, &args[t]);
        for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    }
    free(args);
    free(th);
}

/* ------------------------------------------------------------------------- */
/* Paged decode. Math: tests/kernel/test_decode_attn.cu:24-86. Edge cases of    */
/* the live kernel, src/kernel/attention/decode_attn.cu:384-473:                */
/*   ctx <= 0 -> zeros (:399-404); ceil(ctx/16) > MBPR -> zeros (:406-412);     */
/*   invalid block id -> position skipped (:423-440); denominator + 1e-6 (:455).*/
/* ------------------------------------------------------------------------- */
typedef struct {
    const uint16_t *q, *k, *v;
    const int32_t *bt, *ctx;
    float* out;
    int B, mbpr, hq, hkv, d, bs;
    const int32_t* pairs;
} decode_ctx;

static void decode_one(int64_t i, void* p, float* scores, int64_t* bases) {
    const decode_ctx* c = (const decode_ctx*)p;
    int req, qh;
    if (c->pairs) {
        req = c->pairs[2 * i];
        qh = c->pairs[2 * i + 1];
    } else {
        req = (int)(i / c->hq);
        qh = (int)(i % c->hq);
    }
    float* o = c->out + ((int64_t)req * c->hq + qh) * c->d;
    const int context_len = c->ctx[req];
    const int num_blocks = context_len > 0 ? (context_len + c->bs - 1) / c->bs : 0;
    if (context_len <= 0 || num_blocks > c->mbpr) {
        for (int d = 0; d < c->d; ++d) o[d] = 0.0f;
        return;
    }
    const int gqa = c->hq / c->hkv;
    const int kvh = qh / gqa;
    const float scale = 1.0f / sqrtf((float)c->d);
    attend_one(c->q + ((int64_t)req * c->hq + qh) * c->d, c->k, c->v,
               c->bt + (int64_t)req * c->mbpr, context_len, kvh, c->d, c->hkv, c->bs, c->mbpr,
               scale, 1e-6f, scores, bases, o);
}

static int max_ctx_of(const int32_t* ctx, int B) {
    int m = 1;
    for (int b = 0; b < B; ++b)
        if (ctx[b] > m) m = ctx[b];
    return m;
}

void orc_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                          const int32_t* block_table, const int32_t* context_lens, float* out,
                          int batch_size, int max_blocks_per_req, int num_q_heads,
                          int num_kv_heads, int head_dim, int cache_block_size, int nthreads) {
    decode_ctx c = {q, k_cache, v_cache, block_table, context_lens, out, batch_size,
                    max_blocks_per_req, num_q_heads, num_kv_heads, head_dim, cache_block_size,
                    NULL};
    run_parallel(decode_one, &c, (int64_t)batch_size * num_q_heads, nthreads,
                 max_ctx_of(context_lens, batch_size));
}

void orc_decode_attention_pairs(const uint16_t* q, const uint16_t* k_cache,
                                const uint16_t* v_cache, const int32_t* block_table,
                                const int32_t* context_lens, float* out, int batch_size,
                                int max_blocks_per_req, int num_q_heads, int num_kv_heads,
                                int head_dim, int cache_block_size, const int32_t* pairs,
                                int num_pairs, int nthreads) {
    decode_ctx c = {q, k_cache, v_cache, block_table, context_lens, out, batch_size,
                    max_blocks_per_req, num_q_heads, num_kv_heads, head_dim, cache_block_size,
                    pairs};
    run_parallel(decode_one, &c, num_pairs, nthreads, max_ctx_of(context_lens, batch_size));
}

/* ------------------------------------------------------------------------- */
/* Paged causal prefill: src/kernel/attention/prefill_attn.cu:80-241.           */
/*   request = last r with query_start_loc[r] <= token (linear scan, :83-86);  */
/*   prefix = ctx - qlen; rows with prefix < 0 or an inconsistent range are     */
/*   left unwritten (:92-113); query i sees positions [0, prefix + i] (:112);   */
/*   invalid positions skipped; no valid position -> 0 (:238).                  */
/* ------------------------------------------------------------------------- */
typedef struct {
    const uint16_t *q, *k, *v;
    const int32_t *bt, *qsl, *ctx;
    float* out;
    int B, T, mbpr, hq, hkv, d, bs;
    const int32_t* pairs;
} prefill_ctx;

static void prefill_one(int64_t i, void* p, float* scores, int64_t* bases) {
    const prefill_ctx* c = (const prefill_ctx*)p;
    int g, qh;
    if (c->pairs) {
        g = c->pairs[2 * i];
        qh = c->pairs[2 * i + 1];
    } else {
        g = (int)(i / c->hq);
        qh = (int)(i % c->hq);
    }
    int req = 0;
    while (req + 1 < c->B && c->qsl[req + 1] <= g) ++req;
    const int qbeg = c->qsl[req];
    const int qlen = c->qsl[req + 1] - qbeg;
    const int local = g - qbeg;
    if (qlen <= 0 || local < 0 || local >= qlen) return;
    const int context_len = c->ctx[req];
    const int prefix = context_len - qlen;
    if (prefix < 0) return;
    const int visible = prefix + local + 1;
    if (visible <= 0 || visible > context_len) return;
    const int gqa = c->hq / c->hkv;
    const int kvh = qh / gqa;
    const float scale = 1.0f / sqrtf((float)c->d);
    attend_one(c->q + ((int64_t)g * c->hq + qh) * c->d, c->k, c->v,
               c->bt + (int64_t)req * c->mbpr, visible, kvh, c->d, c->hkv, c->bs, c->mbpr, scale,
               0.0f, scores, bases, c->out + ((int64_t)g * c->hq + qh) * c->d);
}

void orc_prefill_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           const int32_t* block_table, const int32_t* query_start_loc,
                           const int32_t* context_lens, float* out, int batch_size,
                           int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                           int num_kv_heads, int head_dim, int cache_block_size, int nthreads) {
    prefill_ctx c = {q, k_cache, v_cache, block_table, query_start_loc, context_lens, out,
                     batch_size, total_query_tokens, max_blocks_per_req, num_q_heads,
                     num_kv_heads, head_dim, cache_block_size, NULL};
    run_parallel(prefill_one, &c, (int64_t)total_query_tokens * num_q_heads, nthreads,
                 max_ctx_of(context_lens, batch_size));
}

void orc_prefill_attention_pairs(const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, const int32_t* block_table,
                                 const int32_t* query_start_loc, const int32_t* context_lens,
                                 float* out, int batch_size, int total_query_tokens,
                                 int max_blocks_per_req, int num_q_heads, int num_kv_heads,
                                 int head_dim, int cache_block_size, const int32_t* pairs,
                                 int num_pairs, int nthreads) {
    prefill_ctx c = {q, k_cache, v_cache, block_table, query_start_loc, context_lens, out,
                     batch_size, total_query_tokens, max_blocks_per_req, num_q_heads,
                     num_kv_heads, head_dim, cache_block_size, pairs};
    run_parallel(prefill_one, &c, num_pairs, nthreads, max_ctx_of(context_lens, batch_size));
}

/* tests/kernel/test_naive_attn.cu:16-65: dense causal attention, row i sees keys
 * 0..i, normalised by the plain sum. */
void orc_naive_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, float* out,
                         int num_tokens, int n_q_heads, int n_kv_heads, int head_dim) {
    const int gqa = n_q_heads / n_kv_heads;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const int qs = n_q_heads * head_dim, ks = n_kv_heads * head_dim;
    float* sc = (float*)malloc(sizeof(float) * (size_t)(num_tokens > 0 ? num_tokens : 1));
    for (int hq = 0; hq < n_q_heads; ++hq) {
        const int hk = hq / gqa;
        for (int i = 0; i < num_tokens; ++i) {
            float mx = -1e30f;
            for (int j = 0; j <= i; ++j) {
                float s = 0.0f;
                for (int d = 0; d < head_dim; ++d)
                    s += orc_bf16_to_f32(q[i * qs + hq * head_dim + d]) *
                         orc_bf16_to_f32(k[j * ks + hk * head_dim + d]);
                sc[j] = s * scale;
                mx = fmaxf(mx, sc[j]);
            }
            float sum = 0.0f;
            for (int j = 0; j <= i; ++j) {
                sc[j] = expf(sc[j] - mx);
                sum += sc[j];
            }
            for (int j = 0; j <= i; ++j) sc[j] /= sum;
            for (int d = 0; d < head_dim; ++d) {
                float acc = 0.0f;
                for (int j = 0; j <= i; ++j) acc += sc[j] * orc_bf16_to_f32(v[j * ks + hk * head_dim + d]);
                out[i * qs + hq * head_dim + d] = acc;
            }
        }
    }
    free(sc);
}

/* tests/kernel/test_naive_attn.cu:67-74 */
void orc_lcg_fill(uint16_t* data, int n, unsigned int seed) {
    unsigned int s = seed;
    for (int i = 0; i < n; ++i) {
        s = s * 1103515245u + 12345u;
        const float v = (float)((s >> 16) & 0x7FFF) / 32768.0f - 1.0f;
        data[i] = orc_f32_to_bf16(v * 0.5f);
    }
}

/* ---------------------------------------------------------------------------------------
 * Decode-side prologue of one attention layer (the sequence of qwen3_model.cpp:174-244):
 * split the fused QKV projection, RMS-normalise q and k per head, apply split-half RoPE,
 * write the new K/V into the cache.
 * ------------------------------------------------------------------------------------- */

/* src/kernel/elementwise/elementwise.cu:34-64: qkv[t] = [q heads | k heads | v heads]. */
void orc_split_qkv(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T, int nq,
                   int nkv, int hd) {
    const int64_t qd = (int64_t)nq * hd, kd = (int64_t)nkv * hd, row = qd + 2 * kd;
    for (int64_t t = 0; t < T; ++t) {
        memcpy(q + t * qd, qkv + t * row, (size_t)qd * 2);
        memcpy(k + t * kd, qkv + t * row + qd, (size_t)kd * 2);
        memcpy(v + t * kd, qkv + t * row + qd + kd, (size_t)kd * 2);
    }
}

static float orc_bf16_round(float x) { return orc_bf16_to_f32(orc_f32_to_bf16(x)); }

/* Warp sum of cuda_common.cuh:14-20 over 32 lanes: shfl_down by 16, 8, 4, 2, 1; lanes past
 * the top read their own value back (shfl_down keeps it), so only lane 0's result is
 * meaningful and it sums pairs in that tree order. */
static float orc_warp_tree_sum(float v[32]) {
    for (int off = 16; off > 0; off >>= 1) {
        for (int l = 0; l + off < 32; ++l) v[l] = v[l] + v[l + off];
    }
    return v[0];
}

/* src/kernel/norm/rms_norm.cu:22-58 (dim even, the bf16x2 path) and :60-88 (dim odd, the
 * scalar path), with kBlockSize = 256 (:93) and block_reduce_sum of cuda_common.cuh:30-62:
 * per-thread partial sums of squares rounded to bf16 after every addition, a 32-lane tree
 * per warp, the 8 warp sums reduced by warp 0 with the same tree, the total rounded to bf16,
 * inv_rms = 1 / sqrt(total / dim + eps), out = bf16(x * inv_rms * w). In place is allowed. */
void orc_rms_norm(const uint16_t* input, const uint16_t* weight, uint16_t* output, int rows,
                  int dim, float eps) {
    enum { kBlock = 256, kWarp = 32 };
    float part[kBlock];
    for (int r = 0; r < rows; ++r) {
        const uint16_t* x = input + (int64_t)r * dim;
        uint16_t* o = output + (int64_t)r * dim;
        const int even = (dim % 2) == 0;
        for (int tid = 0; tid < kBlock; ++tid) {
            float s = 0.0f;
            if (even) {
                for (int i = tid; i < dim / 2; i += kBlock) {
                    const float a = orc_bf16_to_f32(x[2 * i]), b = orc_bf16_to_f32(x[2 * i + 1]);
                    const float term = a * a + b * b;
                    s = orc_bf16_round(s + term);
                }
            } else {
                for (int i = tid; i < dim; i += kBlock) {
                    const float a = orc_bf16_to_f32(x[i]);
                    s = orc_bf16_round(s + a * a);
                }
            }
            part[tid] = s;
        }
        float warp_sums[kWarp];
        for (int w = 0; w < kWarp; ++w) warp_sums[w] = 0.0f;
        for (int w = 0; w < kBlock / kWarp; ++w) warp_sums[w] = orc_warp_tree_sum(part + w * kWarp);
        const float total = orc_bf16_round(orc_warp_tree_sum(warp_sums));
        const float inv_rms = 1.0f / sqrtf(total / (float)dim + eps);
        /* read all of x before writing (the kernel's first loop completes before the second) */
        for (int i = 0; i < dim; ++i) {
            const float a = orc_bf16_to_f32(x[i]);
            const float w = orc_bf16_to_f32(weight[i]);
            o[i] = orc_f32_to_bf16(a * inv_rms * w);
        }
    }
}

/* src/kernel/pos/rope.cu:14-43 (split-half pairs (i, i + rotary_dim/2); the bf16x2 path at
 * :46-88 computes the same per-element formula): rows of q [T][nq][hd] and k [T][nkv][hd] in
 * place, rope_cache [max_pos][rotary_dim/2] of (cos, sin); tokens with pos < 0 or
 * pos >= rope_cache_max_position are left unchanged. */
void orc_rope(uint16_t* q, uint16_t* k, const int32_t* positions, const float* rope_cache,
              int T, int nq, int nkv, int hd, int rotary_dim, int rope_cache_max_position) {
    const int half = rotary_dim / 2;
    for (int t = 0; t < T; ++t) {
        const int pos = positions[t];
        if (pos < 0 || pos >= rope_cache_max_position) continue;
        for (int lh = 0; lh < nq + nkv; ++lh) {
            const int is_q = lh < nq;
            uint16_t* x = is_q ? q + ((int64_t)t * nq + lh) * hd
                               : k + ((int64_t)t * nkv + (lh - nq)) * hd;
            for (int p = 0; p < half; ++p) {
                const float c = rope_cache[((int64_t)pos * half + p) * 2];
                const float s = rope_cache[((int64_t)pos * half + p) * 2 + 1];
                const float x0 = orc_bf16_to_f32(x[p]), x1 = orc_bf16_to_f32(x[p + half]);
                x[p] = orc_f32_to_bf16(x0 * c - x1 * s);
                x[p + half] = orc_f32_to_bf16(x1 * c + x0 * s);
            }
        }
    }
}

/* The whole prologue: split, q/k RMSNorm (skipped when the weight is NULL), RoPE over the
 * full head_dim, KV-cache write. q_out [T][nq][hd]; k_tmp, v_tmp [T][nkv][hd] receive the
 * K/V rows that are written. */
void orc_qkv_prologue(const uint16_t* qkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                      const int32_t* positions, const float* rope_cache,
                      const int32_t* slot_mapping, uint16_t* q_out, uint16_t* k_tmp,
                      uint16_t* v_tmp, uint16_t* k_cache, uint16_t* v_cache, int T, int nq,
                      int nkv, int hd, int rope_cache_max_position, int max_slots, float eps) {
    orc_split_qkv(qkv, q_out, k_tmp, v_tmp, T, nq, nkv, hd);
    if (q_norm_w) orc_rms_norm(q_out, q_norm_w, q_out, T * nq, hd, eps);
    if (k_norm_w) orc_rms_norm(k_tmp, k_norm_w, k_tmp, T * nkv, hd, eps);
    orc_rope(q_out, k_tmp, positions, rope_cache, T, nq, nkv, hd, hd, rope_cache_max_position);
    orc_write_kv_cache(k_tmp, v_tmp, k_cache, v_cache, slot_mapping, T, nkv, hd, max_slots);
}

/* ------------------------------------------------------------------------- */
/* Batch metadata: the host loops of src/worker/batch_translator.cpp:213-302    */
/* (slot = table[pos / bs] * bs + pos % bs; positions kv_written + t; table     */
/* rows -1 padded; query_start_loc prefix sums; context_lens kv_written + new;  */
/* logits index = the item's last token, or -1 for a prefill chunk that does    */
/* not sample) with the validation of src/model/model_runner.h:102-171 (query   */
/* lengths > 0 and 1 for decode items, qsl[B] == T, positions >= 0,             */
/* 0 < ctx <= max_blocks_per_req * bs, max_blocks_per_req * bs <= max_slots)    */
/* and the translator's own bound (an item needs ceil(ctx / bs) blocks,         */
/* batch_translator.cpp:196-211); block ids must lie in [0, num_cache_blocks).  */
/* ------------------------------------------------------------------------- */
static int32_t clamp_i32(int64_t v) { return (int32_t)(v < 0x7fffffff ? v : 0x7fffffff); }

int orc_build_batch_metadata(const int32_t* item_kv_written, const int32_t* item_new_tokens,
                             const int32_t* item_flags, const int32_t* item_block_start,
                             const int32_t* blocks, int batch_size, int num_tokens,
                             int total_blocks, int max_blocks_per_req, int block_size,
                             int num_cache_blocks,
                             int32_t* positions, int32_t* slot_mapping, int32_t* block_table,
                             int32_t* query_start_loc, int32_t* context_lens,
                             int32_t* logits_indices) {
    const int B = batch_size, T = num_tokens, mbpr = max_blocks_per_req, bs = block_size;
    int status = 0;
    if (mbpr > num_cache_blocks) status = 6;
    int64_t offset = 0;
    for (int i = 0; i < B; ++i) {
        const int len = item_new_tokens[i];
        const int kvw = item_kv_written[i];
        const int flags = item_flags[i];
        const int64_t ctx = (int64_t)kvw + len;
        const int b0 = item_block_start[i];
        const int b1 = item_block_start[i + 1];
        int nblk = b1 - b0;
        if (b0 < 0 || b1 < b0 || b1 > total_blocks) {
            status = 6;
            nblk = 0;
        }
        if (len <= 0) status = 6;
        if ((flags & ORC_ITEM_DECODE) && len != 1) status = 6;
        if (kvw < 0) status = 6;
        if (ctx <= 0 || ctx > (int64_t)mbpr * bs) status = 6;
        if (nblk > mbpr || (ctx > 0 && nblk < (ctx + bs - 1) / bs)) status = 6;

        const int n = len > 0 ? len : 0;
        /* offsets and lengths past INT_MAX (only in a failing batch) are stored as INT_MAX */
        query_start_loc[i] = clamp_i32(offset);
        context_lens[i] = clamp_i32(ctx);
        logits_indices[i] =
            (flags & (ORC_ITEM_DECODE | ORC_ITEM_SAMPLE)) ? clamp_i32(offset + n - 1) : -1;
        for (int t = 0; t < n; ++t) {
            const int64_t tok = offset + t;
            if (tok >= T) break;
            const int64_t pos = (int64_t)kvw + t;
            positions[tok] = (int32_t)pos;
            int32_t slot = -1;
            if (pos >= 0) {
                const int64_t bidx = pos / bs;
                if (bidx < nblk) {
                    const int blk = blocks[b0 + bidx];
                    if (blk >= 0 && blk < num_cache_blocks)
                        slot = (int32_t)((int64_t)blk * bs + pos % bs);
                    else
                        status = 6;
                }
            }
            slot_mapping[tok] = slot;
        }
        for (int b = 0; b < mbpr; ++b) {
            int32_t v = -1;
            if (b < nblk) {
                const int blk = blocks[b0 + b];
                if (blk >= 0 && blk < num_cache_blocks)
                    v = blk;
                else
                    status = 6;
            }
            block_table[(int64_t)i * mbpr + b] = v;
        }
        offset += n;
    }
    query_start_loc[B] = clamp_i32(offset);
    if (offset != T) status = 6;
    return status;
}

/* ------------------------------------------------------------------------- */
/* fp8 KV cache (no counterpart in the reference, whose cache is bf16 only;    */
/* src/base/traits.h:117-124 anticipates other KV profiles). OCP E4M3 ("fn": */
/* no infinities, 0x7f/0xff NaN, largest finite 448), round to nearest even.  */
/* Each cache row (slot, kv_head) is quantised with its own fp32 scale:        */
/*   amax = max |x|; scale = the smallest power of two P >= 2^-126 with         */
/*   amax <= 448 P; q = e4m3(clamp(x / P, +-448)) (scale 0 and q 0 for an       */
/*   all-zero row); value = q * scale.                                          */
/* Scales live in [slot / bs][kv_head][slot % bs] order, so the 16 scales of a  */
/* block's rows for one head are contiguous.                                   */
/* ------------------------------------------------------------------------- */
uint8_t orc_f32_to_e4m3(float x) {
    const uint8_t sign = signbit(x) ? 0x80 : 0x00;
    float a = fabsf(x);
    if (!(a == a)) return 0x7f;              /* NaN */
    if (a >= 448.0f) return sign | 0x7e;     /* saturate */
    if (a < 0.015625f) {                     /* below 2^-6: subnormal grid m * 2^-9 */
        const float m = nearbyintf(a * 512.0f);  /* exact scaling, RNE */
        return sign | (uint8_t)m;                /* m == 8 is the smallest normal 0x08 */
    }
    int e;
    const float f = frexpf(a, &e);           /* a = f * 2^e, f in [0.5, 1) */
    e -= 1;                                  /* a = (2f) * 2^e, 2f in [1, 2) */
    float m = nearbyintf((2.0f * f - 1.0f) * 8.0f);  /* exact: 2f has <= 24 bits */
    if (m == 8.0f) {
        m = 0.0f;
        e += 1;
    }
    if (e > 8 || (e == 8 && m > 6.0f)) return sign | 0x7e;
    return sign | (uint8_t)(((e + 7) << 3) | (int)m);
}

float orc_e4m3_to_f32(uint8_t b) {
    const int e = (b >> 3) & 15, m = b & 7;
    float v;
    if ((b & 0x7f) == 0x7f) return NAN;
    if (e == 0)
        v = ldexpf((float)m, -9);
    else
        v = ldexpf(1.0f + m / 8.0f, e - 7);
    return (b & 0x80) ? -v : v;
}

int64_t orc_fp8_scale_index(int slot, int kv_head, int num_kv_heads, int block_size) {
    return ((int64_t)(slot / block_size) * num_kv_heads + kv_head) * block_size +
           slot % block_size;
}

float orc_fp8_row_scale(float amax) {
    if (!(amax > 0.0f)) return 0.0f;
    /* a row holding an infinity: 2^126, so inf * 2^-126 clamps to 448 and finite elements
       store as zeros (kv_fp8.hip fp8_row_scale) */
    if (isinf(amax)) return ldexpf(1.0f, 126);
    /* smallest p with amax <= 448 * 2^p, by search (448 * 2^p is exact in float) */
    int p = -126;
    while (p < 127 && amax > ldexpf(448.0f, p)) ++p;
    return ldexpf(1.0f, p);
}

void orc_quantize_row_fp8(const uint16_t* x, int n, uint8_t* q, float* scale) {
    float amax = 0.0f;
    for (int d = 0; d < n; ++d) {
        const float a = fabsf(orc_bf16_to_f32(x[d]));
        if (a > amax) amax = a;
    }
    *scale = orc_fp8_row_scale(amax);
    const float inv = amax > 0.0f ? 1.0f / *scale : 0.0f;
    for (int d = 0; d < n; ++d) {
        float v = orc_bf16_to_f32(x[d]) * inv;
        v = v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v);
        q[d] = orc_f32_to_e4m3(v);
    }
}

void orc_write_kv_cache_fp8(const uint16_t* k_new, const uint16_t* v_new, uint8_t* k_cache,
                            uint8_t* v_cache, float* k_scale, float* v_scale,
                            const int32_t* slot_mapping, int total_tokens, int n_kv_heads,
                            int head_dim, int max_slots, int block_size) {
    for (int t = 0; t < total_tokens; ++t) {
        const int slot = slot_mapping[t];
        if (slot < 0 || slot >= max_slots) continue;
        for (int h = 0; h < n_kv_heads; ++h) {
            const int64_t src = ((int64_t)t * n_kv_heads + h) * head_dim;
            const int64_t dst = ((int64_t)slot * n_kv_heads + h) * head_dim;
            const int64_t si = orc_fp8_scale_index(slot, h, n_kv_heads, block_size);
            orc_quantize_row_fp8(k_new + src, head_dim, k_cache + dst, k_scale + si);
            orc_quantize_row_fp8(v_new + src, head_dim, v_cache + dst, v_scale + si);
        }
    }
}

/* Decode over the fp8 cache: the reference decode (attend_one) with each K/V element read
 * as e4m3 value * row scale. */
static float e4m3_lut[256];

typedef struct {
    const uint16_t* q;
    const uint8_t *k, *v;
    const float *ks, *vs;
    const int32_t *bt, *ctx;
    float* out;
    int B, mbpr, hq, hkv, d, bs;
} decode_fp8_ctx;

static void decode_one_fp8(int64_t i, void* p, float* scores, int64_t* bases) {
    const decode_fp8_ctx* c = (const decode_fp8_ctx*)p;
    const int req = (int)(i / c->hq), qh = (int)(i % c->hq);
    float* o = c->out + ((int64_t)req * c->hq + qh) * c->d;
    const int ctx = c->ctx[req];
    const int nb = ctx > 0 ? (ctx + c->bs - 1) / c->bs : 0;
    for (int d = 0; d < c->d; ++d) o[d] = 0.0f;
    if (ctx <= 0 || nb > c->mbpr) return;
    const int kvh = qh / (c->hq / c->hkv);
    const uint16_t* qv = c->q + ((int64_t)req * c->hq + qh) * c->d;
    const int32_t* rb = c->bt + (int64_t)req * c->mbpr;
    const float scale = 1.0f / sqrtf((float)c->d);
    float mx = -INFINITY;
    int any = 0;
    for (int pos = 0; pos < ctx; ++pos) {
        const int blk = rb[pos / c->bs];
        if (blk < 0) {
            bases[pos] = -1;
            continue;
        }
        const int slot = blk * c->bs + pos % c->bs;
        bases[pos] = slot;
        const int64_t row = ((int64_t)slot * c->hkv + kvh) * c->d;
        const float ks = c->ks[orc_fp8_scale_index(slot, kvh, c->hkv, c->bs)];
        float s = 0.0f;
        for (int d = 0; d < c->d; ++d)
            s += orc_bf16_to_f32(qv[d]) * (e4m3_lut[c->k[row + d]] * ks);
        s *= scale;
        scores[pos] = s;
        if (s > mx) mx = s;
        any = 1;
    }
    if (!any) return;
    float denom = 0.0f;
    for (int pos = 0; pos < ctx; ++pos) {
        if (bases[pos] < 0) continue;
        scores[pos] = expf(scores[pos] - mx);
        denom += scores[pos];
    }
    const float inv = 1.0f / (denom + 1e-6f);
    for (int pos = 0; pos < ctx; ++pos) {
        if (bases[pos] < 0) continue;
        const int slot = (int)bases[pos];
        const int64_t row = ((int64_t)slot * c->hkv + kvh) * c->d;
        const float vs = c->vs[orc_fp8_scale_index(slot, kvh, c->hkv, c->bs)];
        const float w = scores[pos] * inv;
        for (int d = 0; d < c->d; ++d) o[d] += w * (e4m3_lut[c->v[row + d]] * vs);
    }
}

void orc_decode_attention_fp8(const uint16_t* q, const uint8_t* k_cache, const uint8_t* v_cache,
                              const float* k_scale, const float* v_scale,
                              const int32_t* block_table, const int32_t* context_lens,
                              float* out, int batch_size, int max_blocks_per_req,
                              int num_q_heads, int num_kv_heads, int head_dim,
                              int cache_block_size, int nthreads) {
    for (int b = 0; b < 256; ++b) e4m3_lut[b] = orc_e4m3_to_f32((uint8_t)b);  /* before workers */
    decode_fp8_ctx c = {q, k_cache, v_cache, k_scale, v_scale, block_table, context_lens, out,
                        batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
                        cache_block_size};
    run_parallel(decode_one_fp8, &c, (int64_t)batch_size * num_q_heads, nthreads,
                 max_ctx_of(context_lens, batch_size));
}

/* Prefill over the fp8 cache: orc_prefill_attention's request lookup and causal range
 * (prefill_attn.cu:80-241) with each K/V element read as e4m3 value * row scale. */
typedef struct {
    const uint16_t* q;
    const uint8_t *k, *v;
    const float *ks, *vs;
    const int32_t *bt, *qsl, *ctx;
    float* out;
    int B, T, mbpr, hq, hkv, d, bs;
} prefill_fp8_ctx;

static void prefill_one_fp8(int64_t i, void* p, float* scores, int64_t* bases) {
    const prefill_fp8_ctx* c = (const prefill_fp8_ctx*)p;
    const int g = (int)(i / c->hq), qh = (int)(i % c->hq);
    int req = 0;
    while (req + 1 < c->B && c->qsl[req + 1] <= g) ++req;
    const int qbeg = c->qsl[req];
    const int qlen = c->qsl[req + 1] - qbeg;
    const int local = g - qbeg;
    if (qlen <= 0 || local < 0 || local >= qlen) return;
    const int context_len = c->ctx[req];
    const int prefix = context_len - qlen;
    if (prefix < 0) return;
    const int visible = prefix + local + 1;
    if (visible <= 0 || visible > context_len) return;
    const int kvh = qh / (c->hq / c->hkv);
    const float scale = 1.0f / sqrtf((float)c->d);
    const uint16_t* qv = c->q + ((int64_t)g * c->hq + qh) * c->d;
    const int32_t* rb = c->bt + (int64_t)req * c->mbpr;
    float* o = c->out + ((int64_t)g * c->hq + qh) * c->d;
    float mx = -INFINITY;
    int any = 0;
    for (int pos = 0; pos < visible; ++pos) {
        const int lb = pos / c->bs;
        const int blk = lb < c->mbpr ? rb[lb] : -1;
        if (blk < 0) {
            bases[pos] = -1;
            continue;
        }
        const int slot = blk * c->bs + pos % c->bs;
        bases[pos] = slot;
        const int64_t row = ((int64_t)slot * c->hkv + kvh) * c->d;
        const float ks = c->ks[orc_fp8_scale_index(slot, kvh, c->hkv, c->bs)];
        float s = 0.0f;
        for (int d = 0; d < c->d; ++d)
            s += orc_bf16_to_f32(qv[d]) * (e4m3_lut[c->k[row + d]] * ks);
        s *= scale;
        scores[pos] = s;
        if (s > mx) mx = s;
        any = 1;
    }
    for (int d = 0; d < c->d; ++d) o[d] = 0.0f;
    if (!any) return;
    float denom = 0.0f;
    for (int pos = 0; pos < visible; ++pos) {
        if (bases[pos] < 0) continue;
        scores[pos] = expf(scores[pos] - mx);
        denom += scores[pos];
    }
    const float inv = 1.0f / denom;
    for (int pos = 0; pos < visible; ++pos) {
        if (bases[pos] < 0) continue;
        const int slot = (int)bases[pos];
        const int64_t row = ((int64_t)slot * c->hkv + kvh) * c->d;
        const float vs = c->vs[orc_fp8_scale_index(slot, kvh, c->hkv, c->bs)];
        const float w = scores[pos] * inv;
        for (int d = 0; d < c->d; ++d) o[d] += w * (e4m3_lut[c->v[row + d]] * vs);
    }
}

void orc_prefill_attention_fp8(const uint16_t* q, const uint8_t* k_cache, const uint8_t* v_cache,
                               const float* k_scale, const float* v_scale,
                               const int32_t* block_table, const int32_t* query_start_loc,
                               const int32_t* context_lens, float* out, int batch_size,
                               int total_query_tokens, int max_blocks_per_req, int num_q_heads,
                               int num_kv_heads, int head_dim, int cache_block_size,
                               int nthreads) {
    for (int b = 0; b < 256; ++b) e4m3_lut[b] = orc_e4m3_to_f32((uint8_t)b);  /* before workers */
    prefill_fp8_ctx c = {q, k_cache, v_cache, k_scale, v_scale, block_table, query_start_loc,
                         context_lens, out, batch_size, total_query_tokens, max_blocks_per_req,
                         num_q_heads, num_kv_heads, head_dim, cache_block_size};
    run_parallel(prefill_one_fp8, &c, (int64_t)total_query_tokens * num_q_heads, nthreads,
                 max_ctx_of(context_lens, batch_size));
}
