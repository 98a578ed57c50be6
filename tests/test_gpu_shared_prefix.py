"""Shared-prefix decode (ccinfer_decode_attention_shared_prefix) against the CPU oracle of
the reference decode (tests/kernel/test_decode_attn.cu:24-86, decode_attn.cu:364-473), on
batches whose table rows start with the same block ids -- the prefix-cache hits that the
reference's KVCacheManager::lookup_prefix_cache hands out (src/cache/kv_cache_manager.cpp:
93-173, BlockTable::shared_count, src/cache/block.h:85-97).

Every cache slot no request may read is poisoned (K = NaN, V = Inf), so a prefix read from
a wrong block, row or head makes the output non-finite. Bar: max-abs 2e-2, mean-abs 2e-3 on
all rows; a batch with nothing shared must give plain decode's bits."""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import decode_attention, decode_attention_shared_prefix
from ccinfer_amd import workloads as W
from tests._util import assert_attn_close, f32, say, u16
from tests.test_gpu_fullsize import poison_unused

pytestmark = pytest.mark.gpu


def oracle_decode(w):
    return oracle.decode(u16(w.q), u16(w.k_cache), u16(w.v_cache), w.block_table,
                         w.context_lens)


def run(fn, w, dev):
    meta = w.device_meta(dev)
    out = fn(w.q, w.k_cache, w.v_cache, meta["block_table"], meta["context_lens"])
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("batch,prefix,lo,hi,groups,hq,hkv,d", [
    (64, 2048, 128, 1024, 1, 16, 8, 128),    # the 64-way shared system prompt
    (64, 2048, 128, 1024, 3, 16, 8, 128),    # three prompts, uneven group sizes
    (37, 512, 1, 300, 5, 32, 8, 128),        # G = 4 (4 members per tile), 1-token suffixes
    (20, 1024, 40, 700, 2, 8, 8, 64),        # G = 1 (16 members per tile)
    (24, 768, 10, 200, 4, 64, 8, 128),       # G = 8 (2 members per tile)
    (30, 256, 5, 90, 3, 16, 8, 96),          # head dim 96 tile
    (30, 256, 5, 90, 3, 16, 8, 80),          # padded head dim
    (30, 256, 5, 90, 3, 8, 4, 192),          # head dim 192 tile
    (300, 512, 1, 400, 7, 16, 8, 128),       # past 256 requests: the indexed flat plan
    (3, 1024, 100, 300, 1, 16, 8, 128),      # 3 requests: the fixed split plan
])
def test_shared_prefix_matches_oracle(gpu, batch, prefix, lo, hi, groups, hq, hkv, d):
    say(f"shared-prefix decode b={batch} prefix={prefix} priv=[{lo},{hi}] groups={groups} "
        f"hq={hq} hkv={hkv} d={d}")
    w = W.decode_shared_prefix(device=gpu, seed=batch + prefix + groups, batch=batch,
                               prefix=prefix, priv_lo=lo, priv_hi=hi, groups=groups, hq=hq,
                               hkv=hkv, d=d)
    poison_unused(w, gpu)
    got = f32(run(decode_attention_shared_prefix, w, gpu))
    assert_attn_close(got, oracle_decode(w), w.name)


def test_nothing_shared_gives_plain_decode_bits(gpu):
    for name, w in [("configs[1]", W.decode_batched(device=gpu, seed=61, with_write=False)),
                    ("b300", W.decode_batched(device=gpu, seed=62, batch=300, ctx_hi=2000,
                                              with_write=False)),
                    ("b2", W.decode_batched(device=gpu, seed=63, batch=2, ctx_lo=600,
                                            ctx_hi=900, with_write=False))]:
        say(f"shared-prefix decode, nothing shared: {name}")
        a = run(decode_attention_shared_prefix, w, gpu)
        b = run(decode_attention, w, gpu)
        assert torch.equal(a, b), name


def test_edge_rows(gpu):
    """Members whose context ends inside the common prefix, invalid rows (zeros), a hole in
    a prefix, an unshared request whose first block matches nothing, and identical rows."""
    say("shared-prefix decode edge rows")
    hq, hkv, d = 16, 8, 128
    rng = np.random.default_rng(71)
    pool = 600
    perm = rng.permutation(pool).astype(np.int32)
    mbpr = 96
    B = 12
    bt = np.full((B, mbpr), -1, np.int32)
    common = perm[:64]                       # a 1024-token prefix
    cur = 64
    ctx = np.array([1300, 1025, 700, 1100, 0, 1200, 1200, 900, 50, 1300, 1300, 1024], np.int32)
    for b in range(B):
        nb = (ctx[b] + 15) // 16
        if b in (8,):                        # unshared request
            bt[b, :nb] = perm[cur:cur + nb]
            cur += nb
            continue
        bt[b, :min(nb, 64)] = common[:min(nb, 64)]
        if nb > 64:
            bt[b, 64:nb] = perm[cur:cur + nb - 64]
            cur += nb - 64
    bt[5] = bt[6]                            # rows 5 and 6: the same table and context
    bt[9, 10] = bt[10, 10] = -1              # a shared hole (equal in both rows)
    bt[9, 11:64] = bt[10, 11:64]
    ctx[4] = 0                               # invalid: zeros
    g = torch.Generator(device=gpu)
    g.manual_seed(72)
    q = W.randn_bf16((B, hq, d), g, gpu)
    k = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    v = W.randn_bf16((pool * 16, hkv, d), g, gpu)
    w = W.PagedWorkload("edge", hq, hkv, d, ctx, bt, pool, q, k, v)
    poison_unused(w, gpu)
    got = f32(run(decode_attention_shared_prefix, w, gpu))
    want = oracle_decode(w)
    assert np.all(got[4] == 0)
    assert_attn_close(got, want, "edge")


def test_repeatable(gpu):
    """Members join their subgroups in arrival order; the output must not depend on it."""
    say("shared-prefix decode repeatability")
    w = W.decode_shared_prefix(device=gpu, seed=81, batch=50, prefix=1024, priv_lo=20,
                               priv_hi=500, groups=3)
    first = run(decode_attention_shared_prefix, w, gpu).clone()
    for _ in range(3):
        assert torch.equal(run(decode_attention_shared_prefix, w, gpu), first)
