"""A whole decode step captured in a HIP graph: the device-built batch metadata, the fused
prologue (split QKV + q/k RMSNorm + RoPE + KV write) and decode attention, as a serving loop
would replay it. Each replay, with eager work and synchronisations between replays, must
reproduce the eager step bit for bit (no host syncs, memsets or allocations inside the step).
"""
import numpy as np
import pytest
import torch

from ccinfer_amd import (ITEM_DECODE, build_batch_metadata, decode_attention,
                         decode_workspace_size, qkv_prologue)
from ccinfer_amd import workloads as W
from tests._util import say

pytestmark = pytest.mark.gpu
BS = 16


def test_decode_step_under_graph_capture(gpu):
    say("decode step (metadata + prologue + decode) captured in a graph")
    rng = np.random.default_rng(31)
    g = torch.Generator(device=gpu)
    g.manual_seed(31)
    b, hq, hkv, d, pool = 24, 16, 8, 128, 2048
    kvw = rng.integers(20, 900, b).astype(np.int32)           # tokens already cached
    nblk = (kvw + 1 + BS - 1) // BS
    perm = rng.permutation(pool).astype(np.int32)
    start = np.zeros(b + 1, np.int32)
    start[1:] = np.cumsum(nblk)
    assert start[-1] <= pool
    blocks = perm[:start[-1]]
    mbpr = int(nblk.max())
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    items = [dev(kvw), dev(np.ones(b, np.int32)), dev(np.full(b, ITEM_DECODE, np.int32)),
             dev(start), dev(blocks)]
    k_cache = W.randn_bf16((pool * BS, hkv, d), g, gpu)
    v_cache = W.randn_bf16((pool * BS, hkv, d), g, gpu)
    qkv = W.randn_bf16((b, (hq + 2 * hkv) * d), g, gpu)
    qn = (1.0 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(torch.bfloat16)
    rope = W.rope_cache_table(4096, d, 1e6, gpu)
    meta = build_batch_metadata(*items, num_tokens=b, max_blocks_per_req=mbpr,
                                num_cache_blocks=pool)
    q = torch.empty((b, hq, d), dtype=torch.bfloat16, device=gpu)
    out = torch.empty_like(q)
    ws = torch.empty(max(1, decode_workspace_size(b, mbpr, hq, hkv, d)), dtype=torch.uint8,
                     device=gpu)

    def step():
        build_batch_metadata(*items, num_tokens=b, max_blocks_per_req=mbpr,
                             num_cache_blocks=pool, out=meta)
        qkv_prologue(qkv, qn, kn, meta["positions"], rope, meta["slot_mapping"], k_cache,
                     v_cache, hq, q_out=q)
        decode_attention(q, k_cache, v_cache, meta["block_table"], meta["context_lens"],
                         output=out, workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # eager; the step is idempotent (it rewrites the same new K/V rows)
    torch.cuda.synchronize()
    assert int(meta["status"].item()) == 0
    eager = out.clone()
    eager_k = k_cache.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step()
    for rep in range(3):
        out.zero_()
        meta["slot_mapping"].fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        assert torch.equal(k_cache, eager_k), rep
        assert int(meta["status"].item()) == 0
    # the eager step matches decode over the cache it wrote (positions = kvw, ctx = kvw + 1)
    assert np.array_equal(meta["positions"].cpu().numpy(), kvw)
    assert np.array_equal(meta["context_lens"].cpu().numpy(), kvw + 1)


def _replay_matches(graph, outs, eager, between):
    """Replays `graph` three times with eager work (`between`) and synchronisations between
    the replays; every replay must reproduce the eager results bit for bit."""
    for rep in range(3):
        between()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), rep


def test_mixed_prefill_under_graph_capture(gpu):
    """KV write + prefill of a mixed batch (chunked prefills and decode items through the
    planner, tile kernel and decode-item launches) captured with a preallocated workspace."""
    from ccinfer_amd import prefill_attention, prefill_workspace_size, write_kv_cache
    say("mixed prefill (planner + tiles + decode items) captured in a graph")
    w = W.mixed_step(device=gpu, seed=41, n_chunks=3, chunk=200, prefix_hi=512, n_decode=40,
                     dec_lo=16, dec_hi=3000)
    meta = w.device_meta(gpu)
    out = torch.empty_like(w.q)
    ws = torch.empty(max(1, prefill_workspace_size(w.batch, w.q.shape[0], w.mbpr, w.hq, w.hkv,
                                                   w.d)), dtype=torch.uint8, device=gpu)

    def step():
        write_kv_cache(w.k_new, w.v_new, w.k_cache, w.v_cache, meta["slot_mapping"])
        prefill_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                          meta["query_start_loc"], meta["context_lens"], output=out,
                          workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    eager = [out.clone(), w.k_cache.clone()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step()

    def between():
        out.zero_()
        ws.fill_(0xA5)  # stale workspace contents must not matter
    _replay_matches(graph, [out, w.k_cache], eager, between)


def test_decode_with_kv_write_and_fp8_under_graph_capture(gpu):
    """The decode step with its KV write in the launch, and the fp8 write + fp8 decode,
    captured with preallocated workspaces."""
    from ccinfer_amd import (decode_attention_fp8, decode_attention_write_kv, fp8_scale_numel,
                             write_kv_cache_fp8)
    say("decode with fused KV write, and fp8 write + decode, captured in a graph")
    w = W.decode_batched(device=gpu, seed=42, batch=48, ctx_lo=100, ctx_hi=3000,
                         with_write=True)
    meta = w.device_meta(gpu)
    slots = w.k_cache.shape[0]
    out = torch.empty_like(w.q)
    out8 = torch.empty_like(w.q)
    ws = torch.empty(max(1, decode_workspace_size(w.batch, w.mbpr, w.hq, w.hkv, w.d)),
                     dtype=torch.uint8, device=gpu)
    ws8 = torch.empty_like(ws)
    kc = torch.zeros((slots, w.hkv, w.d), dtype=torch.uint8, device=gpu)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(fp8_scale_numel(slots, w.hkv), dtype=torch.float32, device=gpu)
    vs = torch.zeros_like(ks)
    all_slots = torch.arange(slots, dtype=torch.int32, device=gpu)
    write_kv_cache_fp8(w.k_cache, w.v_cache, kc, vc, ks, vs, all_slots)

    def step():
        decode_attention_write_kv(w.q, w.k_new, w.v_new, w.k_cache, w.v_cache,
                                  meta["block_table"], meta["context_lens"], output=out,
                                  workspace=ws)
        write_kv_cache_fp8(w.k_new, w.v_new, kc, vc, ks, vs, meta["slot_mapping"])
        decode_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"], meta["context_lens"],
                             output=out8, workspace=ws8)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    eager = [out.clone(), out8.clone(), w.k_cache.clone(), kc.clone(), ks.clone()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step()

    def between():
        out.zero_()
        out8.zero_()
        ws.fill_(0x5A)
        ws8.fill_(0x5A)
    _replay_matches(graph, [out, out8, w.k_cache, kc, ks], eager, between)
