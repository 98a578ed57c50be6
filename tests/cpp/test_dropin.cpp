// C++ drop-in layer test: the reference-signature launchers (kernel/hip_kernels.h) and the
// CRTP backend (backend/hip_backend.h), as src/executor-style callers would use them.
//   test_dropin cpu  -- validation paths only (no device needed)
//   test_dropin gpu  -- also runs write/decode/prefill through HipBackend and through the
//                       launchers and checks both give bit-identical results, plus a closed
//                       form (uniform scores -> mean of V).
// Mirrors tests/kernel/test_{decode_attn,prefill_attn,write_kv_cache}.cu of the reference
// (NullPointers / RejectsNullPointers / NullPointerReturnsError and the readback checks).
#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "backend/hip_backend.h"
#include "ccinfer_attn.h"
#include "kernel/hip_kernels.h"

using namespace ccinfer;

static int g_fail = 0;
#define CHECK(cond)                                                         \
    do {                                                                    \
        if (!(cond)) {                                                      \
            std::fprintf(stderr, "CHECK failed %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            ++g_fail;                                                       \
        }                                                                   \
    } while (0)

struct FakeBackend : DeviceBackend<FakeBackend> {
    int calls = 0;
    template <typename T> Result<void> prefill_attention_impl(const PrefillAttnParams&) { ++calls; return {}; }
    template <typename T> Result<void> decode_attention_impl(const DecodeAttnParams&) { ++calls; return {}; }
    template <typename T> Result<void> write_kv_cache_impl(const WriteKVCacheParams&) { ++calls; return {}; }
};

static void cpu_checks() {
    FakeBackend fb;
    int dummy = 0;
    void* p = &dummy;
    const int32_t* ip = &dummy;
    auto r = fb.decode_attention<__hip_bfloat16>(DecodeAttnParams{
        .q_ = nullptr, .k_cache_ = nullptr, .v_cache_ = nullptr, .block_table_ = nullptr,
        .context_lens_ = nullptr, .output_ = nullptr, .batch_size_ = 1,
        .max_blocks_per_req_ = 1, .num_q_heads_ = 4, .num_kv_heads_ = 4, .head_dim_ = 64,
        .cache_block_size_ = 16});
    CHECK(!r.has_value() && r.error() == ErrorCode::InvalidArgument);
    r = fb.decode_attention<__hip_bfloat16>(DecodeAttnParams{
        .q_ = p, .k_cache_ = p, .v_cache_ = p, .block_table_ = ip, .context_lens_ = ip,
        .output_ = p, .batch_size_ = 1, .max_blocks_per_req_ = 1, .num_q_heads_ = 6,
        .num_kv_heads_ = 4, .head_dim_ = 64, .cache_block_size_ = 16});
    CHECK(!r.has_value() && r.error() == ErrorCode::InvalidArgument);  // 6 % 4 != 0
    r = fb.decode_attention<__hip_bfloat16>(DecodeAttnParams{
        .q_ = p, .k_cache_ = p, .v_cache_ = p, .block_table_ = ip, .context_lens_ = ip,
        .output_ = p, .batch_size_ = 1, .max_blocks_per_req_ = 1, .num_q_heads_ = 8,
        .num_kv_heads_ = 4, .head_dim_ = 64, .cache_block_size_ = 16});
    CHECK(r.has_value() && fb.calls == 1);
    int32_t start_loc[2] = {0, 0};
    r = fb.prefill_attention<__hip_bfloat16>(PrefillAttnParams{
        .q_ = nullptr, .k_cache_ = nullptr, .v_cache_ = nullptr, .block_table_ = nullptr,
        .query_start_loc_ = start_loc, .context_lens_ = nullptr, .output_ = nullptr,
        .batch_size_ = 1, .max_blocks_per_req_ = 1, .num_q_heads_ = 4, .num_kv_heads_ = 4,
        .head_dim_ = 64, .cache_block_size_ = 16});
    CHECK(!r.has_value() && r.error() == ErrorCode::InvalidArgument);
    r = fb.write_kv_cache<__hip_bfloat16>(WriteKVCacheParams{
        .k_new_ = nullptr, .v_new_ = nullptr, .k_cache_ = nullptr, .v_cache_ = nullptr,
        .slot_mapping_ = nullptr, .total_tokens_ = 1, .num_kv_heads_ = 1, .head_dim_ = 1,
        .max_slots_ = 64});
    CHECK(!r.has_value() && r.error() == ErrorCode::InvalidArgument);
    CHECK(fb.calls == 1);

    // Launchers reject before touching a device.
    auto d = launch_decode_attention(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, 1,
                                     4, 4, 64, 16, nullptr);
    CHECK(!d.has_value() && d.error() == ErrorCode::InvalidArgument);
    auto pf = launch_prefill_attention(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                       nullptr, 1, 1, 1, 4, 4, 64, 16, nullptr);
    CHECK(!pf.has_value() && pf.error() == ErrorCode::InvalidArgument);
    auto w = launch_write_kv_cache(nullptr, nullptr, nullptr, nullptr, nullptr, 1, 1, 1, 64,
                                   nullptr);
    CHECK(!w.has_value() && w.error() == ErrorCode::InvalidArgument);
    CHECK(error_message(ErrorCode::InvalidArgument) == "invalid argument");

    // Workspace reservation sizes (host-only arithmetic over the C ABI size queries).
    CHECK(attn_workspace_bytes(AttnWorkspaceLimits{}) == 0);
    CHECK(attn_workspace_bytes(AttnWorkspaceLimits{.max_batch_size = 4, .max_query_tokens = 64,
                                                    .max_blocks_per_req = 8, .num_q_heads = 6,
                                                    .num_kv_heads = 4, .head_dim = 64}) == 0);
    const AttnWorkspaceLimits lim{.max_batch_size = 64, .max_query_tokens = 4096,
                                  .max_blocks_per_req = 256, .num_q_heads = 16,
                                  .num_kv_heads = 8, .head_dim = 128};
    const size_t res = attn_workspace_bytes(lim);
    CHECK(res > 0);
    // every shape within the limits fits the reservation
    for (int b : {1, 2, 3, 4, 5, 8, 9, 31, 64})
        for (int mb : {1, 16, 255, 256}) {
            CHECK(ccinfer_decode_workspace_size(b, mb, 16, 8, 128, 16) <= res);
            for (int t : {b, 1000, 4096})
                CHECK(ccinfer_prefill_workspace_size(b, t, mb, 16, 8, 128, 16) <= res);
        }
}

static uint16_t bf(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}
static float fb16(uint16_t h) {
    uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

template <typename T>
static T* dev_upload(const std::vector<T>& h) {
    T* d = nullptr;
    CHECK(hipMalloc(&d, h.size() * sizeof(T)) == hipSuccess);
    CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) == hipSuccess);
    return d;
}
template <typename T>
static std::vector<T> dev_download(const T* d, size_t n) {
    std::vector<T> h(n);
    CHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost) == hipSuccess);
    return h;
}

static void gpu_checks() {
    auto br = HipBackend::create(0);
    CHECK(br.has_value());
    if (!br.has_value()) return;
    HipBackend& be = **br;
    const int B = 3, HQ = 16, HKV = 8, D = 128, MBPR = 64, NBLK = 200, BS = 16;
    std::vector<uint16_t> hq(B * HQ * D), hk(NBLK * BS * HKV * D), hv(hk.size());
    uint32_t s = 12345u;
    auto rnd = [&]() { s = s * 1664525u + 1013904223u; return ((s >> 9) & 0xffff) / 32768.0f - 1.0f; };
    for (auto& x : hq) x = bf(rnd());
    for (auto& x : hk) x = bf(rnd());
    for (auto& x : hv) x = bf(rnd());
    std::vector<int32_t> bt(B * MBPR, -1), ctx = {37, 1000, 513};
    for (int b = 0; b < B; ++b)
        for (int i = 0; i < (ctx[b] + 15) / 16; ++i) bt[b * MBPR + i] = (b * 67 + i * 3) % NBLK;
    auto* q = dev_upload(hq);
    auto* k = dev_upload(hk);
    auto* v = dev_upload(hv);
    auto* dbt = dev_upload(bt);
    auto* dctx = dev_upload(ctx);
    __hip_bfloat16 *o1 = nullptr, *o2 = nullptr;
    CHECK(hipMalloc(&o1, hq.size() * 2) == hipSuccess);
    CHECK(hipMalloc(&o2, hq.size() * 2) == hipSuccess);
    auto bq = reinterpret_cast<const __hip_bfloat16*>(q);
    auto bk = reinterpret_cast<const __hip_bfloat16*>(k);
    auto bv = reinterpret_cast<const __hip_bfloat16*>(v);

    const DecodeAttnParams dp{
        .q_ = q, .k_cache_ = k, .v_cache_ = v, .block_table_ = dbt, .context_lens_ = dctx,
        .output_ = o1, .batch_size_ = B, .max_blocks_per_req_ = MBPR, .num_q_heads_ = HQ,
        .num_kv_heads_ = HKV, .head_dim_ = D, .cache_block_size_ = BS};
    // No reservation yet: the ops reject instead of allocating.
    CHECK(ccinfer_decode_workspace_size(B, MBPR, HQ, HKV, D, BS) > 0);
    auto r = be.decode_attention<__hip_bfloat16>(dp);
    CHECK(!r.has_value() && r.error() == ErrorCode::InvalidArgument);
    auto l = launch_decode_attention(bq, bk, bv, dbt, dctx, o2, B, MBPR, HQ, HKV, D, BS, nullptr);
    CHECK(!l.has_value() && l.error() == ErrorCode::InvalidArgument);

    // Reserve once (initialisation), then run.
    const AttnWorkspaceLimits lim{.max_batch_size = B, .max_query_tokens = 128,
                                  .max_blocks_per_req = MBPR, .num_q_heads = HQ,
                                  .num_kv_heads = HKV, .head_dim = D, .cache_block_size = BS};
    CHECK(be.reserve_workspace(lim).has_value());
    CHECK(be.reserved_workspace_bytes() == attn_workspace_bytes(lim));
    CHECK(reserve_launcher_workspace(nullptr, lim).has_value());

    // A shape beyond the reservation is rejected before any launch (the size check runs
    // first; the buffers here are far too small for the shape, so a launch would fault).
    const int BIG_B = 4096, BIG_MBPR = 4096;
    const size_t big = ccinfer_decode_workspace_size(BIG_B, BIG_MBPR, HQ, HKV, D, BS);
    CHECK(big > be.reserved_workspace_bytes());
    if (big > be.reserved_workspace_bytes()) {
        DecodeAttnParams bp = dp;
        bp.batch_size_ = BIG_B;
        bp.max_blocks_per_req_ = BIG_MBPR;
        r = be.decode_attention<__hip_bfloat16>(bp);
        CHECK(!r.has_value() && r.error() == ErrorCode::InvalidArgument);
        l = launch_decode_attention(bq, bk, bv, dbt, dctx, o2, BIG_B, BIG_MBPR, HQ, HKV, D, BS,
                                    nullptr);
        CHECK(!l.has_value() && l.error() == ErrorCode::InvalidArgument);
    }

    // Decode: backend (own stream + workspace) vs reference-signature launcher.
    r = be.decode_attention<__hip_bfloat16>(dp);
    CHECK(r.has_value());
    CHECK(be.synchronize().has_value());
    l = launch_decode_attention(bq, bk, bv, dbt, dctx, o2, B, MBPR, HQ, HKV, D, BS, nullptr);
    CHECK(l.has_value());
    CHECK(hipDeviceSynchronize() == hipSuccess);
    CHECK(dev_download(reinterpret_cast<uint16_t*>(o1), hq.size()) ==
          dev_download(reinterpret_cast<uint16_t*>(o2), hq.size()));

    // The backend decode captured in a HIP graph (its ops allocate nothing): every replay,
    // with eager work and synchronisations between, equals the eager result bit for bit.
    {
        const auto want = dev_download(reinterpret_cast<uint16_t*>(o1), hq.size());
        __hip_bfloat16* og = nullptr;
        CHECK(hipMalloc(&og, hq.size() * 2) == hipSuccess);
        DecodeAttnParams gp = dp;
        gp.output_ = og;
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        CHECK(hipStreamBeginCapture(be.stream(), hipStreamCaptureModeGlobal) == hipSuccess);
        r = be.decode_attention<__hip_bfloat16>(gp);
        CHECK(r.has_value());
        CHECK(hipStreamEndCapture(be.stream(), &graph) == hipSuccess);
        CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess);
        for (int rep = 0; rep < 3; ++rep) {
            CHECK(hipMemset(og, 0xff, hq.size() * 2) == hipSuccess);
            CHECK(hipGraphLaunch(exec, be.stream()) == hipSuccess);
            CHECK(be.synchronize().has_value());
            CHECK(dev_download(reinterpret_cast<uint16_t*>(og), hq.size()) == want);
            // eager work between replays, on the same stream and workspace
            CHECK(be.decode_attention<__hip_bfloat16>(dp).has_value());
            CHECK(be.synchronize().has_value());
        }
        CHECK(hipGraphExecDestroy(exec) == hipSuccess);
        CHECK(hipGraphDestroy(graph) == hipSuccess);
        CHECK(hipFree(og) == hipSuccess);
    }

    // Prefill of 3 requests (qlen 20, 1, 64) both ways.
    std::vector<int32_t> qsl = {0, 20, 21, 85}, pctx = {60, 700, 64};
    const int T = 85;
    std::vector<uint16_t> pq(T * HQ * D);
    for (auto& x : pq) x = bf(rnd());
    auto* dq = dev_upload(pq);
    auto* dqsl = dev_upload(qsl);
    auto* dpctx = dev_upload(pctx);
    __hip_bfloat16 *p1 = nullptr, *p2 = nullptr;
    CHECK(hipMalloc(&p1, pq.size() * 2) == hipSuccess);
    CHECK(hipMalloc(&p2, pq.size() * 2) == hipSuccess);
    r = be.prefill_attention<__hip_bfloat16>(PrefillAttnParams{
        .q_ = dq, .k_cache_ = k, .v_cache_ = v, .block_table_ = dbt, .query_start_loc_ = dqsl,
        .context_lens_ = dpctx, .output_ = p1, .num_tokens_ = T, .batch_size_ = B,
        .max_blocks_per_req_ = MBPR, .num_q_heads_ = HQ, .num_kv_heads_ = HKV, .head_dim_ = D,
        .cache_block_size_ = BS});
    CHECK(r.has_value());
    CHECK(be.synchronize().has_value());
    l = launch_prefill_attention(reinterpret_cast<const __hip_bfloat16*>(dq), bk, bv, dbt, dqsl,
                                 dpctx, p2, B, T, MBPR, HQ, HKV, D, BS, nullptr);
    CHECK(l.has_value());
    CHECK(hipDeviceSynchronize() == hipSuccess);
    CHECK(dev_download(reinterpret_cast<uint16_t*>(p1), pq.size()) ==
          dev_download(reinterpret_cast<uint16_t*>(p2), pq.size()));

    // Write KV (test_write_kv_cache.cu KAT shape) then a uniform-score decode: out == 0.2.
    std::vector<uint16_t> kn(4 * 2 * 4), vn(4 * 2 * 4);
    for (int t = 0; t < 4; ++t)
        for (int h = 0; h < 2; ++h)
            for (int dd = 0; dd < 4; ++dd) {
                kn[(t * 2 + h) * 4 + dd] = bf(float(t * 100 + h * 10 + dd));
                vn[(t * 2 + h) * 4 + dd] = bf(float(t * 200 + h * 10 + dd));
            }
    std::vector<int32_t> slots = {5, 17, 0, 63};
    std::vector<uint16_t> zeros(64 * 2 * 4, 0);
    auto* dkn = dev_upload(kn);
    auto* dvn = dev_upload(vn);
    auto* dsl = dev_upload(slots);
    auto* kc = dev_upload(zeros);
    auto* vc = dev_upload(zeros);
    r = be.write_kv_cache<__hip_bfloat16>(WriteKVCacheParams{
        .k_new_ = dkn, .v_new_ = dvn, .k_cache_ = kc, .v_cache_ = vc, .slot_mapping_ = dsl,
        .total_tokens_ = 4, .num_kv_heads_ = 2, .head_dim_ = 4, .max_slots_ = 64});
    CHECK(r.has_value());
    CHECK(be.synchronize().has_value());
    auto kh = dev_download(kc, zeros.size());
    for (int t = 0; t < 4; ++t)
        CHECK(std::memcmp(&kh[slots[t] * 8], &kn[t * 8], 16) == 0);
    CHECK(kh[8] == 0);

    std::vector<uint16_t> uq(2 * 4 * 64, bf(0.1f)), uk(32 * 4 * 64, bf(0.1f)), uv(uk.size(), bf(0.2f));
    std::vector<int32_t> ubt = {0, 1, 0, 1}, uctx = {32, 32};
    auto* duq = dev_upload(uq);
    auto* duk = dev_upload(uk);
    auto* duv = dev_upload(uv);
    auto* dubt = dev_upload(ubt);
    auto*ductx = dev_upload(uctx);
    __hip_bfloat16* uo = nullptr;
    CHECK(hipMalloc(&uo, uq.size() * 2) == hipSuccess);
    // another head shape on the same stream: the reservation grows to cover it
    CHECK(reserve_launcher_workspace(
              nullptr, AttnWorkspaceLimits{.max_batch_size = 2, .max_query_tokens = 2,
                                           .max_blocks_per_req = 2, .num_q_heads = 4,
                                           .num_kv_heads = 4, .head_dim = 64})
              .has_value());
    l = launch_decode_attention(reinterpret_cast<const __hip_bfloat16*>(duq),
                                reinterpret_cast<const __hip_bfloat16*>(duk),
                                reinterpret_cast<const __hip_bfloat16*>(duv), dubt, ductx, uo, 2,
                                2, 4, 4, 64, 16, nullptr);
    CHECK(l.has_value());
    CHECK(hipDeviceSynchronize() == hipSuccess);
    for (uint16_t x : dev_download(reinterpret_cast<uint16_t*>(uo), uq.size()))
        CHECK(std::fabs(fb16(x) - fb16(bf(0.2f))) < 2e-3f);
    release_launcher_workspaces();
    for (void* ptr : {(void*)q, (void*)k, (void*)v, (void*)dbt, (void*)dctx, (void*)o1, (void*)o2,
                      (void*)dq, (void*)dqsl, (void*)dpctx, (void*)p1, (void*)p2, (void*)dkn,
                      (void*)dvn, (void*)dsl, (void*)kc, (void*)vc, (void*)duq, (void*)duk,
                      (void*)duv, (void*)dubt, (void*)ductx, (void*)uo})
        CHECK(hipFree(ptr) == hipSuccess);
}

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
    cpu_checks();
    if (gpu) gpu_checks();
    std::printf("test_dropin %s: %s (%d failure(s))\n", gpu ? "gpu" : "cpu",
                g_fail ? "FAIL" : "ok", g_fail);
    return g_fail ? 1 : 0;
}
