"""Seeded random layouts through every route of the C ABI, against the CPU oracle.

Each case draws a batch (request count, query lengths, cached prefixes), a head layout
(query/KV heads, head dim), a cache block size and pointer offsets for q, output and the
caches, so that the native MFMA paths, the row copies, the expanded tables, the 2-byte
decode loads and the any-layout prefill tiles are all exercised together with mixed
batches. Every cache slot no request may read is poisoned (K = NaN, V = Inf). Bar: max-abs
2e-2, mean-abs 2e-3 on every row (reference tests: tests/kernel/test_decode_attn.cu,
tests/kernel/test_prefill_attn.cu use max-abs 2e-2 against their CPU references).
"""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import decode_attention, prefill_attention
from ccinfer_amd import workloads as W
from tests._util import assert_attn_close, f32, say, u16

pytestmark = pytest.mark.gpu

HEADS = [(16, 8), (32, 8), (8, 8), (64, 2), (12, 4), (28, 4)]
DECODE_DIMS = [32, 64, 80, 96, 112, 120, 128, 192, 256]
PREFILL_DIMS = DECODE_DIMS + [72, 100, 200, 250]


def _view(t, offset):
    if offset == 0:
        return t
    flat = torch.empty(t.numel() + offset + 8, dtype=t.dtype, device=t.device)
    v = flat[offset:offset + t.numel()].view(t.shape)
    v.copy_(t)
    return v


def _build(dev, rng, batch, bs, hq, hkv, d, qlen, ctx):
    nb = (np.maximum(ctx, 1) + bs - 1) // bs
    mbpr = int(nb.max()) + int(rng.integers(0, 3))
    pool = int(nb.sum()) + 4
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((batch, mbpr), -1, np.int32)
    cur = 0
    for b in range(batch):
        bt[b, :nb[b]] = perm[cur:cur + nb[b]]
        cur += nb[b]
    g = torch.Generator(device=dev)
    g.manual_seed(int(rng.integers(1 << 30)))
    total = int(qlen.sum())
    q = W.randn_bf16((total, hq, d), g, dev)
    k = W.randn_bf16((pool * bs, hkv, d), g, dev)
    v = W.randn_bf16((pool * bs, hkv, d), g, dev)
    used = np.zeros(pool * bs, bool)
    for b in range(batch):
        if ctx[b] < qlen[b]:
            continue
        pos = np.arange(ctx[b])
        used[bt[b, pos // bs] * bs + pos % bs] = True
    bad = torch.from_numpy(np.nonzero(~used)[0]).to(dev)
    k.view(torch.int16)[bad] = 0x7FC0   # NaN
    v.view(torch.int16)[bad] = 0x7F80   # +Inf
    return q, k, v, bt


@pytest.mark.parametrize("seed", range(12))
def test_random_layout_decode(gpu, seed):
    rng = np.random.default_rng(1000 + seed)
    batch = int(rng.integers(1, 80))
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    d = int(rng.choice(DECODE_DIMS))
    ctx = rng.integers(1, 1500, batch).astype(np.int32)
    offs = [int(rng.choice([0, 0, 1, 3])) for _ in range(4)]   # q, k, v, output
    say(f"random decode seed={seed} B={batch} hq={hq} hkv={hkv} d={d} offsets={offs}")
    q, k, v, bt = _build(gpu, rng, batch, 16, hq, hkv, d, np.ones(batch, np.int32), ctx)
    want = oracle.decode(u16(q), u16(k), u16(v), bt, ctx)
    out = _view(torch.zeros_like(q), offs[3])
    got = decode_attention(_view(q, offs[0]), _view(k, offs[1]), _view(v, offs[2]),
                           torch.from_numpy(bt).to(gpu), torch.from_numpy(ctx).to(gpu),
                           output=out)
    torch.cuda.synchronize()
    assert_attn_close(f32(got), want, f"decode seed {seed}")


@pytest.mark.parametrize("seed", range(16))
def test_random_layout_prefill(gpu, seed):
    rng = np.random.default_rng(2000 + seed)
    batch = int(rng.integers(1, 24))
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    d = int(rng.choice(PREFILL_DIMS))
    bs = int(rng.choice([16, 16, 8, 32, 48, 24]))
    kinds = rng.integers(0, 3, batch)        # 0 prompt chunk, 1 single token, 2 short chunk
    qlen = np.where(kinds == 1, 1, np.where(kinds == 0, rng.integers(2, 300, batch),
                                            rng.integers(2, 9, batch))).astype(np.int32)
    prefix = rng.integers(0, 800, batch).astype(np.int32)
    ctx = (prefix + qlen).astype(np.int32)
    if batch > 2:
        ctx[rng.integers(batch)] = 0         # a request with nothing to attend: untouched
    offs = [int(rng.choice([0, 0, 1, 3])) for _ in range(4)]   # q, k, v, output
    say(f"random prefill seed={seed} B={batch} hq={hq} hkv={hkv} d={d} bs={bs} offsets={offs}")
    q, k, v, bt = _build(gpu, rng, batch, bs, hq, hkv, d, qlen, ctx)
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    want = oracle.prefill(u16(q), u16(k), u16(v), bt, qsl, ctx, block_size=bs,
                          out=np.full(q.shape, 3.0, np.float32))
    out = _view(torch.full_like(q, 3.0), offs[3])
    got = prefill_attention(_view(q, offs[0]), _view(k, offs[1]), _view(v, offs[2]),
                            torch.from_numpy(bt).to(gpu), torch.from_numpy(qsl).to(gpu),
                            torch.from_numpy(ctx).to(gpu), output=out, cache_block_size=bs)
    torch.cuda.synchronize()
    assert_attn_close(f32(got), want, f"prefill seed {seed}")
