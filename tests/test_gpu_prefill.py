"""Paged causal prefill attention on the GPU against the CPU oracle.

Reference behaviour: src/kernel/attention/prefill_attn.cu:43-242 and the causal contract of
src/backend/params.h:140-146; reference tests: tests/kernel/test_prefill_attn.cu:24-105
(paged prefill == dense causal attention for prefix 0 and an identity table, max-abs < 0.02),
tests/integration/test_prefix_cache_e2e.cpp (shared prefix blocks drive prefill).
Bar: max-abs <= 2e-2 and mean-abs <= 2e-3 against the fp32 oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import (decode_attention, prefill_attention, prefill_workspace_size,
                         write_kv_cache)
from ccinfer_amd import workloads as W
from tests._util import assert_attn_close, f32, from_u16, say, u16

pytestmark = pytest.mark.gpu


def run_prefill(w, dev, out=None, block_size=16, total=None):
    meta = w.device_meta(dev)
    q = w.q if total is None else w.q[:total]
    if out is not None and total is not None:
        out = out[:total]
    o = prefill_attention(q, w.k_cache, w.v_cache, meta["block_table"],
                          meta["query_start_loc"], meta["context_lens"], output=out,
                          cache_block_size=block_size)
    torch.cuda.synchronize()
    return o


def oracle_prefill(w, pairs=None, block_size=16, out=None, total=None):
    q = u16(w.q) if total is None else u16(w.q[:total])
    return oracle.prefill(q, u16(w.k_cache), u16(w.v_cache), w.block_table,
                          w.query_start_loc, w.context_lens, block_size=block_size,
                          pairs=pairs, out=out)


def write_new(w, dev):
    write_kv_cache(w.k_new, w.v_new, w.k_cache, w.v_cache,
                   torch.from_numpy(w.slot_mapping).to(dev))


def sample_pairs(w, n, seed):
    rng = np.random.default_rng(seed)
    t = int(w.query_start_loc[-1])
    rows = np.concatenate([rng.integers(0, t, n), w.query_start_loc[:-1],
                           w.query_start_loc[1:] - 1])
    heads = np.concatenate([rng.integers(0, w.hq, n), np.zeros(w.batch, np.int64),
                            np.full(w.batch, w.hq - 1)])
    return np.stack([rows, heads], 1).astype(np.int32)


def test_reference_single_request_matches_dense(gpu):
    """test_prefill_attn.cu:24-105 with the LCG fill of test_naive_attn.cu:67-74."""
    say("prefill KAT single request vs dense causal")
    t, h, d = 32, 4, 64
    q = oracle.lcg_fill(t * h * d, 1).reshape(t, h, d)
    kc = oracle.lcg_fill(4 * 16 * h * d, 2).reshape(64, h, d)
    vc = oracle.lcg_fill(4 * 16 * h * d, 3).reshape(64, h, d)
    w = W.PagedWorkload("kat", h, h, d, np.array([t], np.int32), np.array([[0, 1]], np.int32),
                        4, from_u16(q, gpu), from_u16(kc, gpu), from_u16(vc, gpu),
                        query_start_loc=np.array([0, t], np.int32))
    got = f32(run_prefill(w, gpu))
    dense = oracle.naive(q, kc[:t], vc[:t])
    mx, _ = assert_attn_close(got, dense, "vs dense")
    assert mx < 0.02
    assert_attn_close(got, oracle_prefill(w), "vs paged oracle")


def test_config3_prefix_cached(gpu):
    say("prefill config3 8x(512+1536), shared prefix (sampled rows)")
    w = W.prefill_prefix(device=gpu)
    write_new(w, gpu)
    got = f32(run_prefill(w, gpu))
    pairs = sample_pairs(w, 384, 3)
    want = oracle_prefill(w, pairs=pairs)
    r, h = pairs[:, 0], pairs[:, 1]
    assert_attn_close(got[r, h], want[r, h], "config3")
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("prefix,new,sharers", [
    (64, 100, (1,)), (1024, [300, 77, 513, 129], (1, 2, 3))])
def test_shared_prefix_equals_private_copy(gpu, prefix, new, sharers):
    """Sequences listing the same prefix blocks (with equal or unequal new-token lengths) ==
    the same batch with private copies of those blocks."""
    say(f"prefill shared prefix == private copy (prefix {prefix}, new {new})")
    n = 3 if np.isscalar(new) else len(new)
    w = W.prefill_prefix(device=gpu, seed=8, n_seqs=n, prefix=prefix, new=new, hq=16, hkv=8,
                         share_pairs=tuple((s, 0) for s in sharers))
    write_new(w, gpu)
    shared = u16(run_prefill(w, gpu))
    # Give the sharers private copies of their (shared) prefix blocks in fresh pool blocks.
    pblk = prefix // 16
    extra = w.num_blocks
    kc = torch.cat([w.k_cache, torch.empty((len(sharers) * pblk * 16,) + w.k_cache.shape[1:],
                                           dtype=w.k_cache.dtype, device=gpu)])
    vc = torch.cat([w.v_cache, torch.empty_like(kc[:len(sharers) * pblk * 16])])
    bt = w.block_table.copy()
    for si, seq in enumerate(sharers):
        assert np.array_equal(w.block_table[0, :pblk], w.block_table[seq, :pblk])
        for i in range(pblk):
            src, dst = int(bt[seq, i]), extra + si * pblk + i
            kc[dst * 16:(dst + 1) * 16] = w.k_cache[src * 16:(src + 1) * 16]
            vc[dst * 16:(dst + 1) * 16] = w.v_cache[src * 16:(src + 1) * 16]
            bt[seq, i] = dst
    extra += len(sharers) * pblk
    w2 = W.PagedWorkload("copy", w.hq, w.hkv, w.d, w.context_lens, bt, extra, w.q, kc, vc,
                         query_start_loc=w.query_start_loc)
    private = u16(run_prefill(w2, gpu))
    assert np.array_equal(shared, private)


def test_mixed_chunked_prefill_and_decode(gpu):
    say("prefill mixed 4x512 chunks + 128 decodes (sampled rows)")
    w = W.mixed_step(device=gpu)
    write_new(w, gpu)
    got = f32(run_prefill(w, gpu))
    pairs = sample_pairs(w, 256, 4)
    want = oracle_prefill(w, pairs=pairs)
    r, h = pairs[:, 0], pairs[:, 1]
    assert_attn_close(got[r, h], want[r, h], "mixed")
    # Decode items through prefill == the decode operator on the same rows.
    nc = w.info["n_chunks"]
    rows = torch.from_numpy(w.query_start_loc[nc:-1].astype(np.int64)).to(gpu)
    meta = w.device_meta(gpu)
    dec = decode_attention(w.q[rows].contiguous(), w.k_cache, w.v_cache,
                           meta["block_table"][nc:].contiguous(),
                           meta["context_lens"][nc:].contiguous())
    assert_attn_close(got[w.query_start_loc[nc:-1]], f32(dec), "mixed decode items")


def test_plan_with_thousands_of_requests(gpu):
    # 2600 requests: the planner's scans take several entries per thread, its histogram
    # sorts 1100 query tiles, and 1500 single-token requests become decode items
    say("prefill plan 1100 chunks + 1500 decodes (sampled rows)")
    w = W.mixed_step(device=gpu, seed=9, n_chunks=1100, chunk=16, prefix_hi=96,
                     n_decode=1500, dec_lo=16, dec_hi=400)
    write_new(w, gpu)
    got = f32(run_prefill(w, gpu))
    pairs = sample_pairs(w, 512, 9)
    want = oracle_prefill(w, pairs=pairs)
    r, h = pairs[:, 0], pairs[:, 1]
    assert_attn_close(got[r, h], want[r, h], "many requests")


@pytest.mark.parametrize("hq,hkv,d,new,prefix", [
    (16, 8, 128, 200, 48), (4, 4, 128, 70, 0), (16, 4, 128, 130, 32), (8, 8, 64, 90, 16),
    (16, 8, 256, 75, 32), (6, 2, 128, 40, 16), (16, 8, 96, 37, 16), (4, 2, 80, 33, 0),
    (32, 2, 128, 20, 16), (32, 1, 128, 100, 16), (17, 1, 64, 70, 0), (48, 2, 96, 60, 32)])
def test_head_shapes_and_ragged_lengths(gpu, hq, hkv, d, new, prefix):
    say(f"prefill shape hq={hq} hkv={hkv} d={d} new={new} prefix={prefix}")
    w = W.prefill_prefix(device=gpu, seed=hq + d + new, n_seqs=3, prefix=prefix, new=new,
                         share_pairs=(), hq=hq, hkv=hkv, d=d)
    write_new(w, gpu)
    assert_attn_close(f32(run_prefill(w, gpu)), oracle_prefill(w), f"hq{hq}/hkv{hkv}/d{d}")


def test_varlen_batch_edge_cases(gpu):
    """qlen 1..3 items, prefix < 0 rows left untouched, holes and table overflow."""
    say("prefill varlen edge cases")
    rng = np.random.default_rng(12)
    hq, hkv, d = 16, 8, 128
    qlen = np.array([2, 1, 3, 5, 130, 1, 64], np.int32)
    ctx = np.array([40, 17, 3, 2, 200, 1, 300], np.int32)   # seq 3: prefix < 0 (untouched)
    mbpr = 16
    pool = 128
    perm = rng.permutation(pool).astype(np.int32)
    bt = perm[:len(qlen) * mbpr].reshape(len(qlen), mbpr).copy()
    bt[4, 3] = -1                      # hole inside a long prefill
    bt[6, 15] = -1
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    total = int(qsl[-1])
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    q = W.randn_bf16((total, hq, d), g, gpu)
    kc = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    vc = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    w = W.PagedWorkload("edge", hq, hkv, d, ctx, bt, pool, q, kc, vc, query_start_loc=qsl)
    sentinel = torch.full_like(q, 7.0)
    got = f32(run_prefill(w, gpu, out=sentinel.clone()))
    want = oracle_prefill(w, out=np.full((total, hq, d), 7.0, np.float32))
    untouched = slice(qsl[3], qsl[4])
    assert np.all(got[untouched] == 7.0)
    assert_attn_close(got, want, "edge")


def test_rows_past_total_tokens_not_processed(gpu):
    say("prefill total_query_tokens < query_start_loc[B]")
    w = W.prefill_prefix(device=gpu, seed=30, n_seqs=2, prefix=16, new=80, share_pairs=(),
                         hq=8, hkv=4, d=128)
    write_new(w, gpu)
    total = 120
    out = torch.full_like(w.q, 3.0)
    got = f32(run_prefill(w, gpu, out=out, total=total))
    want = oracle_prefill(w, total=total, out=np.full((total, w.hq, w.d), 3.0, np.float32))
    assert_attn_close(got, want, "clipped")


def test_block_size_8(gpu):
    """Non-16 cache blocks (accepted by the reference prefill launcher) on the any-layout
    tile kernel."""
    say("prefill block_size 8")
    rng = np.random.default_rng(3)
    hq, hkv, d, bs = 8, 4, 128, 8
    qlen, ctx, mbpr, pool = np.array([20, 9], np.int32), np.array([50, 9], np.int32), 8, 20
    bt = rng.permutation(pool)[:16].reshape(2, 8).astype(np.int32)
    qsl = np.array([0, 20, 29], np.int32)
    g = torch.Generator(device=gpu)
    g.manual_seed(2)
    q = W.randn_bf16((29, hq, d), g, gpu)
    kc = W.randn_bf16((pool * bs, hkv, d), g, gpu)
    vc = W.randn_bf16((pool * bs, hkv, d), g, gpu)
    w = W.PagedWorkload("bs8", hq, hkv, d, ctx, bt, pool, q, kc, vc, query_start_loc=qsl)
    got = f32(run_prefill(w, gpu, block_size=bs))
    assert_attn_close(got, oracle_prefill(w, block_size=bs), "bs8")


def test_deterministic(gpu):
    say("prefill determinism")
    w = W.prefill_prefix(device=gpu, seed=4, n_seqs=2, prefix=32, new=300, share_pairs=())
    write_new(w, gpu)
    assert np.array_equal(u16(run_prefill(w, gpu)), u16(run_prefill(w, gpu)))


def test_mixed_batch_under_graph_capture(gpu):
    """The decode items run on the caller's side stream, forked from the caller's stream and
    joined back; that fork/join must capture into a graph and replay to the eager result."""
    from ccinfer_amd import SideStream
    say("prefill mixed batch captured in a graph")
    # 42 requests: at least 32, so the decode items take the side stream
    w = W.mixed_step(device=gpu, n_chunks=2, chunk=128, n_decode=40, dec_hi=4096)
    write_new(w, gpu)
    meta = w.device_meta(gpu)
    eager = run_prefill(w, gpu).clone()
    out = torch.zeros_like(w.q)
    n = prefill_workspace_size(w.batch, w.q.shape[0], w.mbpr, w.hq, w.hkv, w.d)
    ws = torch.zeros(max(1, n), dtype=torch.uint8, device=gpu)
    side = SideStream(gpu)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        prefill_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                          meta["query_start_loc"], meta["context_lens"], output=out,
                          workspace=ws, overlap=side)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_concurrent_mixed_prefills_on_two_streams(gpu):
    """Two mixed batches launched concurrently on two streams, each with its own workspace
    and side stream, give the same bits as the same calls run one after the other: the
    library holds no state shared between calls."""
    from ccinfer_amd import SideStream
    say("prefill concurrent mixed batches on two streams")
    ws_a = W.mixed_step(device=gpu, seed=41, n_chunks=2, chunk=256, n_decode=48, dec_hi=8192)
    ws_b = W.mixed_step(device=gpu, seed=42, n_chunks=3, chunk=128, n_decode=36, dec_hi=6000)
    for w in (ws_a, ws_b):
        write_new(w, gpu)
    serial = [run_prefill(w, gpu).clone() for w in (ws_a, ws_b)]
    outs = [torch.zeros_like(w.q) for w in (ws_a, ws_b)]
    metas = [w.device_meta(gpu) for w in (ws_a, ws_b)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    sides = [SideStream(gpu), SideStream(gpu)]
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        for w, m, o, st, sd in zip((ws_a, ws_b), metas, outs, streams, sides):
            with torch.cuda.stream(st):
                prefill_attention(w.q, w.k_cache, w.v_cache, m["block_table"],
                                  m["query_start_loc"], m["context_lens"], output=o, overlap=sd)
        torch.cuda.synchronize()
        for o, want in zip(outs, serial):
            assert torch.equal(o, want)


@pytest.mark.parametrize("which", ["q", "k_cache", "output"])
def test_two_byte_aligned_views(gpu, which):
    """A q or output view that is only 2-byte aligned runs the MFMA kernels on workspace
    copies of its rows (bit-equal to the aligned call); a cache that is only 2-byte aligned
    runs the any-layout tile kernel."""
    say(f"prefill with a 2-byte aligned {which}")
    w = W.prefill_prefix(device=gpu, seed=19, n_seqs=3, prefix=32, new=90, share_pairs=(),
                         hq=8, hkv=4, d=128)
    write_new(w, gpu)

    def shifted(t):
        flat = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
        v = flat[1:].view(t.shape)
        v.copy_(t)
        return v

    meta = w.device_meta(gpu)
    q, kc, out = w.q, w.k_cache, None
    if which == "q":
        q = shifted(w.q)
    elif which == "k_cache":
        kc = shifted(w.k_cache)
    else:
        out = shifted(torch.zeros_like(w.q))
    got = prefill_attention(q, kc, w.v_cache, meta["block_table"], meta["query_start_loc"],
                            meta["context_lens"], output=out)
    torch.cuda.synchronize()
    assert_attn_close(f32(got), oracle_prefill(w), f"misaligned {which}")
    if which != "k_cache":
        assert torch.equal(got, run_prefill(w, gpu))


def test_two_byte_aligned_output_keeps_unwritten_rows(gpu):
    """The staged output starts as a copy of the caller's rows, so rows the kernels do not
    write (a request whose context is shorter than its query) come back unchanged; a mixed
    batch's decode items write through the staged rows too."""
    say("prefill staged output: untouched rows and decode items")
    rng = np.random.default_rng(31)
    hq, hkv, d = 16, 8, 128
    qlen = np.array([70, 1, 3, 1, 5, 200], np.int32)
    ctx = np.array([90, 300, 2, 17, 40, 200], np.int32)   # request 2: prefix < 0
    mbpr, pool = 24, 160
    bt = rng.permutation(pool)[:len(qlen) * mbpr].reshape(len(qlen), mbpr).astype(np.int32)
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    total = int(qsl[-1])
    g = torch.Generator(device=gpu)
    g.manual_seed(6)
    q = W.randn_bf16((total, hq, d), g, gpu)
    kc = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    vc = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    w = W.PagedWorkload("staged", hq, hkv, d, ctx, bt, pool, q, kc, vc, query_start_loc=qsl)
    flat = torch.full((total * hq * d + 9,), 7.0, dtype=torch.bfloat16, device=gpu)
    ov = flat[3:3 + total * hq * d].view(total, hq, d)
    meta = w.device_meta(gpu)
    prefill_attention(q, kc, vc, meta["block_table"], meta["query_start_loc"],
                      meta["context_lens"], output=ov)
    torch.cuda.synchronize()
    got = f32(ov)
    want = oracle_prefill(w, out=np.full((total, hq, d), 7.0, np.float32))
    assert np.all(got[qsl[2]:qsl[3]] == 7.0)
    assert torch.all(flat[:3] == 7.0) and torch.all(flat[3 + total * hq * d:] == 7.0)
    assert_attn_close(got, want, "staged edge")
    aligned = run_prefill(w, gpu, out=torch.full_like(q, 7.0))
    assert torch.equal(ov, aligned)


@pytest.mark.parametrize("bs,hq,hkv,d", [(32, 16, 8, 128), (64, 8, 8, 64), (256, 32, 4, 128),
                                         (48, 16, 8, 96)])
def test_block_sizes_multiple_of_16_on_mfma_path(gpu, bs, hq, hkv, d):
    """Cache blocks of 16·k tokens run the MFMA prefill through a 16-token table built in the
    workspace: bit-equal to the same call with that table written out on the host, and
    within the tolerance of the oracle at block size bs. The batch mixes prompt chunks over
    cached prefixes with decode items."""
    say(f"prefill block size {bs} hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(bs + d)
    qlen = np.array([300, 1, 77, 1, 1, 129, 40], np.int32)
    prefix = np.array([0, 900, 250, 31, 2047, 600, 5], np.int32)
    ctx = prefix + qlen
    mbpr = int((ctx.max() + bs - 1) // bs) + 1
    pool = len(qlen) * mbpr
    bt = rng.permutation(pool).reshape(len(qlen), mbpr).astype(np.int32)
    k = bs // 16
    bt16 = (bt[:, :, None] * k + np.arange(k)[None, None, :]).reshape(len(qlen), mbpr * k)
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    total = int(qsl[-1])
    g = torch.Generator(device=gpu)
    g.manual_seed(bs)
    q = W.randn_bf16((total, hq, d), g, gpu)
    kc = W.randn_bf16((pool * bs, hkv, d), g, gpu)
    vc = W.randn_bf16((pool * bs, hkv, d), g, gpu)
    w = W.PagedWorkload(f"bs{bs}", hq, hkv, d, ctx, bt, pool, q, kc, vc, query_start_loc=qsl)
    w16 = W.PagedWorkload("bs16", hq, hkv, d, ctx, bt16.astype(np.int32), pool * k, q, kc, vc,
                          query_start_loc=qsl)
    got = run_prefill(w, gpu, block_size=bs)
    assert torch.equal(got, run_prefill(w16, gpu))
    pairs = sample_pairs(w, 400, bs)
    want = oracle_prefill(w, pairs=pairs, block_size=bs)
    r, h = pairs[:, 0], pairs[:, 1]
    assert_attn_close(f32(got)[r, h], want[r, h], f"bs{bs}")


def test_more_than_4096_requests(gpu):
    """The planner keeps per-request arrays in LDS up to 4096 requests and in the workspace
    beyond; the reference launcher has no batch limit."""
    say("prefill 5200 requests: 4700 prompt chunks + 500 decodes (sampled rows)")
    w = W.mixed_step(device=gpu, seed=23, n_chunks=4700, chunk=4, prefix_hi=64, n_decode=500,
                     dec_lo=8, dec_hi=200)
    write_new(w, gpu)
    assert w.batch > 4096
    got = f32(run_prefill(w, gpu))
    pairs = sample_pairs(w, 512, 23)
    want = oracle_prefill(w, pairs=pairs)
    r, h = pairs[:, 0], pairs[:, 1]
    assert_attn_close(got[r, h], want[r, h], "5200 requests")


def test_table_row_longer_than_4096_blocks(gpu):
    """A 70K-token context (4400 blocks per table row) stays on the MFMA path: block ids are
    read from the table row in global memory, not staged in LDS."""
    say("prefill 1 x (70144 cached + 300 new) (sampled rows)")
    w = W.prefill_prefix(device=gpu, seed=24, n_seqs=1, prefix=70144, new=300, share_pairs=(),
                         hq=16, hkv=8, d=128)
    write_new(w, gpu)
    assert w.mbpr > 4096
    got = f32(run_prefill(w, gpu))
    pairs = sample_pairs(w, 48, 24)
    want = oracle_prefill(w, pairs=pairs)
    r, h = pairs[:, 0], pairs[:, 1]
    assert_attn_close(got[r, h], want[r, h], "long table")


def test_mixed_batch_with_600_decode_items(gpu):
    """600 single-token requests of 100..3000 positions in a prefill call: the decode items
    run the flat plan's index with snapped ranges (4816 wavefronts), reaching requests
    through the item list. Unused slots poisoned; every decode row against the oracle."""
    from tests.test_gpu_random_shapes import _poison_unused
    say("prefill mixed 2x64 chunks + 600 decodes of 100..3000 positions (all decode rows)")
    w = W.mixed_step(device=gpu, seed=31, n_chunks=2, chunk=64, prefix_hi=256, n_decode=600,
                     dec_lo=100, dec_hi=3000)
    write_new(w, gpu)
    _poison_unused(w, gpu)
    got = f32(run_prefill(w, gpu))
    assert np.all(np.isfinite(got))
    nc = w.info["n_chunks"]
    rows = w.query_start_loc[nc:-1]
    ref = oracle.decode(u16(w.q)[rows], u16(w.k_cache), u16(w.v_cache), w.block_table[nc:],
                        w.context_lens[nc:])
    assert_attn_close(got[rows], ref, "600 decode items")


@pytest.mark.parametrize("n_req,mbpr", [(40, 24), (40, 136), (257, 24)])
def test_mixed_batch_same_bits_serial_and_forked(gpu, n_req, mbpr):
    """A mixed batch gives the same bits whether its decode items run after the tiles or,
    with a side stream (32+ requests), beside them: the planner lists the decode items in
    request order, so their split plan does not depend on timing. Every row must also
    match the oracle: ragged prompts, single-token items, empty and malformed (prefix < 0)
    requests, a table hole. 40 requests with 24-block rows run the decode items inside the
    tile launch (with or without the side stream); with 136-block rows (past 2048
    positions) they take the decode kernels; 257 requests take the decode plan's index
    kernel."""
    from ccinfer_amd import SideStream
    say(f"prefill mixed batch serial vs forked, {n_req} requests, {mbpr} blocks per row")
    rng = np.random.default_rng(900 + n_req)
    hq, hkv, d = 16, 8, 128
    qlen = rng.choice([0, 1, 1, 2, 7, 33, 129], size=n_req).astype(np.int32)
    prefix = rng.integers(0, 200, n_req).astype(np.int32)
    ctx = np.minimum(qlen + prefix, mbpr * 16).astype(np.int32)
    ctx[::17] = np.maximum(qlen[::17] - 1, 0)      # prefix < 0: rows left untouched
    pool = n_req * mbpr
    bt = rng.permutation(pool).astype(np.int32).reshape(n_req, mbpr)
    bt[5, 2] = -1                                  # a hole
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    total = int(qsl[-1])
    g = torch.Generator(device=gpu)
    g.manual_seed(n_req)
    q = W.randn_bf16((total, hq, d), g, gpu)
    kc = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    vc = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    w = W.PagedWorkload("mixed_fork", hq, hkv, d, ctx, bt, pool, q, kc, vc, query_start_loc=qsl)
    m = w.device_meta(gpu)
    outs = []
    for side in (None, SideStream(gpu)):
        o = torch.full_like(q, 7.0)
        prefill_attention(q, kc, vc, m["block_table"], m["query_start_loc"],
                          m["context_lens"], output=o, overlap=side)
        torch.cuda.synchronize()
        outs.append(o)
    want = oracle_prefill(w, out=np.full((total, hq, d), 7.0, np.float32))
    if not torch.equal(outs[0], outs[1]):
        a, b = f32(outs[0]), f32(outs[1])
        bad = np.nonzero((a != b).any(axis=(1, 2)))[0]
        req = np.searchsorted(qsl, bad, side="right") - 1
        for r, rq in list(zip(bad, req))[:12]:
            ea = np.abs(a[r] - want[r]).max()
            eb = np.abs(b[r] - want[r]).max()
            print(f"row {r} req {rq} qlen {qlen[rq]} ctx {ctx[rq]} err serial {ea:.3e} "
                  f"fork {eb:.3e} heads {np.nonzero((a[r] != b[r]).any(axis=1))[0]}")
        print("bad rows", len(bad), "requests", np.unique(req))
    assert_attn_close(f32(outs[1]), want, f"forked {n_req}")
    assert_attn_close(f32(outs[0]), want, f"serial {n_req}")
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 1, 80), (8, 8, 64), (64, 2, 128)])
def test_single_token_requests_inside_the_tile_launch(gpu, hq, hkv, d):
    """Batches of up to 256 (request, kv head) groups with table rows of up to 2048 positions
    run their single-token requests as extra workgroups of the tile launch (no decode
    launches). Every row against the oracle: single-token requests with 1..2048 positions,
    prompts, empty and malformed (prefix < 0) requests, a table hole, rows past
    total_query_tokens, virtual kv heads (G = 32) and padded head dims; the side stream
    changes nothing."""
    from ccinfer_amd import SideStream
    say(f"prefill single-token requests in the tile launch hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(hq * 100 + d)
    n_req, mbpr = 24, 128
    qlen = rng.choice([0, 1, 1, 1, 2, 33, 129], size=n_req).astype(np.int32)
    prefix = rng.integers(0, 2048, n_req).astype(np.int32)
    ctx = np.minimum(qlen + prefix, mbpr * 16).astype(np.int32)
    ctx[1], qlen[1] = 2048, 1                      # a full-length single-token row
    ctx[7] = np.maximum(qlen[7] - 1, 0)            # prefix < 0: rows left untouched
    pool = n_req * mbpr
    bt = rng.permutation(pool).astype(np.int32).reshape(n_req, mbpr)
    bt[3, 5] = -1                                  # a hole
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    total = int(qsl[-1])
    clip = total - 1 if qlen[-1] == 1 else total   # the last request's row past the end
    g = torch.Generator(device=gpu)
    g.manual_seed(hq + d)
    q = W.randn_bf16((total, hq, d), g, gpu)
    kc = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    vc = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    w = W.PagedWorkload("fused_dec", hq, hkv, d, ctx, bt, pool, q, kc, vc, query_start_loc=qsl)
    m = w.device_meta(gpu)
    outs = []
    for side in (None, SideStream(gpu)):
        o = torch.full_like(q, 7.0)
        prefill_attention(q[:clip], kc, vc, m["block_table"], m["query_start_loc"],
                          m["context_lens"], output=o[:clip], overlap=side)
        torch.cuda.synchronize()
        outs.append(o)
    want = oracle_prefill(w, total=clip, out=np.full((clip, hq, d), 7.0, np.float32))
    got = f32(outs[0])
    assert_attn_close(got[:clip], want, f"fused decode items hq{hq}/hkv{hkv}/d{d}")
    assert np.all(got[clip:] == 7.0)
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("d", [48, 160, 192, 224])
def test_single_token_requests_at_wide_head_dims(gpu, d):
    """Head dims off the decode entry's list with single-token requests of up to 3000
    positions (past the fused route's 2048): those run the decode kernels (192 in its own
    tile, 160 / 224 padded to 256, 48 padded to 64) beside the tile kernel; every row
    against the oracle."""
    say(f"prefill mixed batch d={d}")
    w = W.mixed_step(device=gpu, seed=d, n_chunks=2, chunk=64, prefix_hi=512, n_decode=12,
                     dec_lo=100, dec_hi=3000, hq=8, hkv=4, d=d)
    write_new(w, gpu)
    assert_attn_close(f32(run_prefill(w, gpu)), oracle_prefill(w), f"mixed d{d}")
