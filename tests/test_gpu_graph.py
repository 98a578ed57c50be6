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
