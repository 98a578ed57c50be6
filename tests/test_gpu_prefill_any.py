"""Prefill on the any-layout route: the MFMA tile kernel with element-wise staging, for the
shapes the reference prefill accepts beyond the native kernels' layout -- cache blocks of
any size, head dims up to 256 that are not a multiple of 8 (or of 16 above 128), and k / v
caches that are only 2-byte aligned (src/kernel/attention/prefill_attn.cu:246-279 takes any
cache_block_size and head_dim <= 256). Mixed batches: single-token requests run as one-row
tiles on this route.

Every cache slot that no request may read is poisoned (K = NaN, V = Inf), so a wrong gather
shows up as a non-finite or far-off row. All rows are compared with the CPU oracle at the
attention bar (max-abs 2e-2, mean-abs 2e-3); rows of a request whose context is shorter
than its query keep the output's prior contents.
"""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import prefill_attention
from ccinfer_amd import workloads as W
from tests._util import assert_attn_close, f32, say, u16

pytestmark = pytest.mark.gpu

POISON_K, POISON_V = 0x7FC0, 0x7F80  # bf16 NaN, +Inf


def _offset_copy(t, elems):
    flat = torch.empty(t.numel() + elems, dtype=t.dtype, device=t.device)
    v = flat[elems:elems + t.numel()].view(t.shape)
    v.copy_(t)
    return v


def _case(dev, seed, bs, hq, hkv, d, qlen, prefix):
    rng = np.random.default_rng(seed)
    qlen = np.asarray(qlen, np.int32)
    ctx = (np.asarray(prefix, np.int32) + qlen).astype(np.int32)
    ctx[2] = qlen[2] - 1                       # request 2: context shorter than its query
    nb = (np.maximum(ctx, 1) + bs - 1) // bs
    mbpr = int(nb.max()) + 1
    pool = int(nb.sum()) + 8
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((len(qlen), mbpr), -1, np.int32)
    cur = 0
    for b in range(len(qlen)):
        bt[b, :nb[b]] = perm[cur:cur + nb[b]]
        cur += nb[b]
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    total = int(qsl[-1])
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = W.randn_bf16((total, hq, d), g, dev)
    k = W.randn_bf16((pool * bs, hkv, d), g, dev)
    v = W.randn_bf16((pool * bs, hkv, d), g, dev)
    # poison every slot no request may read
    used = np.zeros(pool * bs, bool)
    for b in range(len(qlen)):
        if ctx[b] < qlen[b]:
            continue
        pos = np.arange(ctx[b])
        used[bt[b, pos // bs] * bs + pos % bs] = True
    bad = torch.from_numpy(np.nonzero(~used)[0]).to(dev)
    k.view(torch.int16)[bad] = POISON_K
    v.view(torch.int16)[bad] = torch.tensor(POISON_V, dtype=torch.int16, device=dev)
    return q, k, v, bt, qsl, ctx


@pytest.mark.parametrize("bs,hq,hkv,d,offset", [
    (8, 16, 8, 128, 0),      # 8-token blocks
    (24, 8, 4, 64, 0),       # 24-token blocks
    (16, 16, 8, 100, 0),     # head dim not a multiple of 8
    (16, 16, 8, 128, 1),     # caches offset by one element
    (8, 32, 4, 250, 3),      # head dim 250 (the 256 tile), offset caches, 8-token blocks
    (1, 8, 8, 72, 0),        # one-token blocks
    (40, 64, 2, 120, 5),     # 32 q-heads per kv head, 40-token blocks, offset caches
])
def test_any_layout_matches_oracle(gpu, bs, hq, hkv, d, offset):
    say(f"any-layout prefill bs={bs} hq={hq} hkv={hkv} d={d} offset={offset}")
    qlen = [300, 1, 5, 1, 77, 1, 129, 40]
    prefix = [0, 900, 0, 31, 250, 2047, 600, 5]
    q, k, v, bt, qsl, ctx = _case(gpu, bs * 7 + d, bs, hq, hkv, d, qlen, prefix)
    want = oracle.prefill(u16(q), u16(k), u16(v), bt, qsl, ctx, block_size=bs,
                          out=np.full(q.shape, 3.0, np.float32))
    kc, vc = (_offset_copy(k, offset), _offset_copy(v, offset)) if offset else (k, v)
    out = torch.full_like(q, 3.0)
    got = prefill_attention(q, kc, vc, torch.from_numpy(bt).to(gpu),
                            torch.from_numpy(qsl).to(gpu), torch.from_numpy(ctx).to(gpu),
                            output=out, cache_block_size=bs)
    torch.cuda.synchronize()
    got = f32(got)
    assert np.all(got[qsl[2]:qsl[3]] == 3.0)   # context shorter than the query: untouched
    assert_attn_close(got, want, f"bs{bs} d{d}")
    again = prefill_attention(q, kc, vc, torch.from_numpy(bt).to(gpu),
                              torch.from_numpy(qsl).to(gpu), torch.from_numpy(ctx).to(gpu),
                              output=torch.full_like(q, 3.0), cache_block_size=bs)
    torch.cuda.synchronize()
    assert np.array_equal(u16(again), u16(out))


def test_any_layout_workspace_size(gpu):
    """The size query covers the any-layout route; a smaller workspace is rejected before
    anything is launched."""
    from ccinfer_amd import _lib
    say("any-layout prefill workspace")
    q, k, v, bt, qsl, ctx = _case(gpu, 5, 8, 16, 8, 64, [64, 1, 3, 1, 9, 1, 20, 4],
                                  [0, 50, 0, 7, 30, 90, 10, 2])
    lib = _lib.load()
    n = lib.ccinfer_prefill_workspace_size(len(ctx), q.shape[0], bt.shape[1], 16, 8, 64, 8)
    assert n > 0
    ws = torch.zeros(n, dtype=torch.uint8, device=gpu)
    out = torch.empty_like(q)
    m = {k_: torch.from_numpy(a).to(gpu) for k_, a in (("bt", bt), ("qsl", qsl), ("ctx", ctx))}
    s = torch.cuda.current_stream().cuda_stream
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), m["bt"].data_ptr(), m["qsl"].data_ptr(),
            m["ctx"].data_ptr(), out.data_ptr(), len(ctx), q.shape[0], bt.shape[1], 16, 8, 64,
            8, ws.data_ptr()]
    assert lib.ccinfer_prefill_attention(*args, n - 1, s) == 6
    assert lib.ccinfer_prefill_attention(*args, n, s) == 0
    torch.cuda.synchronize()


def test_any_layout_under_graph_capture(gpu):
    """The any-layout route (planner + tile kernel, no host work between them) captures into
    a HIP graph; every replay, with eager work and synchronisations between, equals the
    eager call."""
    say("any-layout prefill captured in a graph")
    q, k, v, bt, qsl, ctx = _case(gpu, 9, 8, 16, 8, 128, [200, 1, 5, 1, 64, 1, 33, 7],
                                  [0, 700, 0, 30, 100, 1500, 64, 3])
    m = [torch.from_numpy(a).to(gpu) for a in (bt, qsl, ctx)]
    eager = prefill_attention(q, k, v, *m, output=torch.full_like(q, 3.0),
                              cache_block_size=8).clone()
    from ccinfer_amd import prefill_workspace_size
    n = prefill_workspace_size(len(ctx), q.shape[0], bt.shape[1], 16, 8, 128, 8)
    ws = torch.zeros(max(1, n), dtype=torch.uint8, device=gpu)
    out = torch.full_like(q, 3.0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        prefill_attention(q, k, v, *m, output=out, cache_block_size=8, workspace=ws)
    for _ in range(3):
        out.fill_(3.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_any_layout_rows_past_total_tokens(gpu):
    """total_query_tokens below query_start_loc[B]: rows past it are neither read nor
    written (src/kernel/attention/prefill_attn.cu launches total_query_tokens rows)."""
    say("any-layout prefill with total_query_tokens < query_start_loc[B]")
    q, k, v, bt, qsl, ctx = _case(gpu, 11, 8, 16, 8, 100, [40, 1, 5, 1, 90, 1, 60, 30],
                                  [10, 300, 0, 20, 50, 700, 0, 9])
    total = int(qsl[5]) + 17                  # stops inside request 6
    out = torch.full_like(q, 3.0)
    got = prefill_attention(q[:total], k, v, torch.from_numpy(bt).to(gpu),
                            torch.from_numpy(qsl).to(gpu), torch.from_numpy(ctx).to(gpu),
                            output=out[:total], cache_block_size=8)
    torch.cuda.synchronize()
    want = oracle.prefill(u16(q[:total]), u16(k), u16(v), bt, qsl, ctx, block_size=8,
                          out=np.full((total,) + tuple(q.shape[1:]), 3.0, np.float32))
    assert_attn_close(f32(got), want, "clipped")
    assert torch.all(out[total:] == 3.0)


def test_any_layout_more_than_4096_requests(gpu):
    """The planner's per-request arrays move to the workspace past 4096 requests; on this
    route single-token requests are tiles too. Sampled rows against the oracle."""
    say("any-layout prefill with 5000 requests (24-token blocks)")
    rng = np.random.default_rng(13)
    n = 5000
    qlen = np.where(rng.random(n) < 0.4, 1, rng.integers(2, 6, n)).astype(np.int32)
    prefix = rng.integers(0, 60, n).astype(np.int32)
    q, k, v, bt, qsl, ctx = _case(gpu, 13, 24, 8, 4, 64, qlen, prefix)
    got = f32(prefill_attention(q, k, v, torch.from_numpy(bt).to(gpu),
                                torch.from_numpy(qsl).to(gpu), torch.from_numpy(ctx).to(gpu),
                                output=torch.full_like(q, 3.0), cache_block_size=24))
    torch.cuda.synchronize()
    rows = np.concatenate([qsl[:-1][::97], qsl[1:][::89] - 1])
    pairs = np.stack([rows, rows % 8], 1).astype(np.int32)
    want = oracle.prefill(u16(q), u16(k), u16(v), bt, qsl, ctx, block_size=24, pairs=pairs,
                          out=np.full(q.shape, 3.0, np.float32))
    r, h = pairs[:, 0], pairs[:, 1]
    assert_attn_close(got[r, h], want[r, h], "5000 requests")
