"""Seeded synthetic paged-attention workloads (the five benchmark configurations).

Metadata (context lengths, block pools, block tables, slot mappings) comes from numpy's
PCG64 (`np.random.default_rng(seed)`); Q/K/V values are N(0,1) drawn with a seeded torch
generator on the target device and rounded to bf16. Block tables follow the reference's
contract (src/worker/batch_translator.cpp:213-293): int32 [batch][max_blocks_per_req],
-1 padded; slot = block_id * 16 + pos % 16; context_lens include the new tokens.

Every generator takes `scale` knobs so tests can build the same shape family small.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

BLOCK = 16
QWEN3_06B = dict(hq=16, hkv=8, d=128)
QWEN3_8B = dict(hq=32, hkv=8, d=128)


@dataclass
class PagedWorkload:
    """One batch over a paged KV cache. Device tensors live on `device`."""
    name: str
    hq: int
    hkv: int
    d: int
    context_lens: np.ndarray          # [B] int32
    block_table: np.ndarray           # [B, MBPR] int32, -1 padded
    num_blocks: int
    q: torch.Tensor                   # [rows, Hq, D] bf16
    k_cache: torch.Tensor             # [num_blocks * 16, Hkv, D] bf16
    v_cache: torch.Tensor
    query_start_loc: Optional[np.ndarray] = None   # [B+1] (prefill / mixed)
    k_new: Optional[torch.Tensor] = None           # [T_new, Hkv, D] tokens to write
    v_new: Optional[torch.Tensor] = None
    slot_mapping: Optional[np.ndarray] = None      # [T_new] int32
    info: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.context_lens.size)

    @property
    def mbpr(self) -> int:
        return int(self.block_table.shape[1])

    def device_meta(self, device) -> dict:
        """int32 metadata tensors on `device`."""
        out = {
            "block_table": torch.from_numpy(self.block_table).to(device),
            "context_lens": torch.from_numpy(self.context_lens).to(device),
        }
        if self.query_start_loc is not None:
            out["query_start_loc"] = torch.from_numpy(self.query_start_loc).to(device)
        if self.slot_mapping is not None:
            out["slot_mapping"] = torch.from_numpy(self.slot_mapping).to(device)
        return out

    def kv_bytes(self) -> int:
        """Algorithmic decode bytes: K+V of every context position, once per (seq, kv_head)."""
        return int(np.sum(self.context_lens.astype(np.int64))) * self.hkv * self.d * 2 * 2


def randn_bf16(shape, gen: torch.Generator, device) -> torch.Tensor:
    """N(0,1) rounded to bf16, generated in chunks to bound the fp32 temporary."""
    n = int(np.prod(shape))
    out = torch.empty(n, dtype=torch.bfloat16, device=device)
    step = 1 << 26
    for s in range(0, n, step):
        e = min(n, s + step)
        out[s:e] = torch.randn(e - s, generator=gen, device=device, dtype=torch.float32)
    return out.view(*shape)


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _tables(rng: np.random.Generator, blocks_per_seq, pool_blocks: int,
            shared: Optional[dict] = None) -> np.ndarray:
    """Assigns distinct pool blocks (drawn without replacement from a shuffled pool).

    shared: {seq: (src_seq, n_blocks)} makes seq's first n_blocks equal src_seq's.
    """
    perm = rng.permutation(pool_blocks).astype(np.int32)
    mbpr = int(max(blocks_per_seq))
    bt = np.full((len(blocks_per_seq), mbpr), -1, np.int32)
    cur = 0
    shared = shared or {}
    for b, n in enumerate(blocks_per_seq):
        start = 0
        if b in shared:
            src, ns = shared[b]
            bt[b, :ns] = bt[src, :ns]
            start = ns
        take = n - start
        bt[b, start:n] = perm[cur:cur + take]
        cur += take
    assert cur <= pool_blocks
    return bt


def _pool_size(distinct_blocks: int, slack: float = 1.1) -> int:
    return int(math.ceil(distinct_blocks * slack))


def _cache(pool_blocks: int, hkv: int, d: int, gen, device):
    k = randn_bf16((pool_blocks * BLOCK, hkv, d), gen, device)
    v = randn_bf16((pool_blocks * BLOCK, hkv, d), gen, device)
    return k, v


def decode_single(device="cpu", seed: int = 1, ctx: int = 512, pool_blocks: int = 256,
                  hq: int = 16, hkv: int = 8, d: int = 128) -> PagedWorkload:
    """Config 1: batch 1, ctx 512 in 32 blocks, table = first blocks of a permuted pool."""
    rng = np.random.default_rng(seed)
    nblk = -(-ctx // BLOCK)
    perm = rng.permutation(pool_blocks).astype(np.int32)
    bt = perm[:nblk].reshape(1, nblk).copy()
    g = _gen(seed, device)
    q = randn_bf16((1, hq, d), g, device)
    k, v = _cache(pool_blocks, hkv, d, g, device)
    return PagedWorkload("decode_b1_ctx512", hq, hkv, d, np.array([ctx], np.int32), bt,
                         pool_blocks, q, k, v)


def decode_batched(device="cpu", seed: int = 2, batch: int = 64, ctx_lo: int = 128,
                   ctx_hi: int = 4096, hq: int = 16, hkv: int = 8, d: int = 128,
                   with_write: bool = True) -> PagedWorkload:
    """Config 2: ragged contexts U[ctx_lo, ctx_hi]; new token of each seq written first."""
    rng = np.random.default_rng(seed)
    ctx = rng.integers(ctx_lo, ctx_hi + 1, size=batch).astype(np.int32)
    nblk = (ctx + BLOCK - 1) // BLOCK
    pool = _pool_size(int(nblk.sum()))
    bt = _tables(rng, nblk.tolist(), pool)
    g = _gen(seed, device)
    q = randn_bf16((batch, hq, d), g, device)
    k, v = _cache(pool, hkv, d, g, device)
    w = PagedWorkload(f"decode_b{batch}_ctx{ctx_lo}-{ctx_hi}", hq, hkv, d, ctx, bt, pool, q, k, v)
    if with_write:
        pos = ctx - 1
        w.slot_mapping = (bt[np.arange(batch), pos // BLOCK] * BLOCK + pos % BLOCK).astype(np.int32)
        w.k_new = randn_bf16((batch, hkv, d), g, device)
        w.v_new = randn_bf16((batch, hkv, d), g, device)
    return w


def decode_shared_prefix(device="cpu", seed: int = 7, batch: int = 64, prefix: int = 2048,
                         priv_lo: int = 128, priv_hi: int = 1024, groups: int = 1,
                         hq: int = 16, hkv: int = 8, d: int = 128) -> PagedWorkload:
    """Decode over shared cached prompts: request b belongs to prefix group b % groups; the
    group's prefix (`prefix` tokens, whole blocks) sits in blocks every member's table row
    starts with (prefix-cache hits), followed by U[priv_lo, priv_hi] private tokens."""
    assert prefix % BLOCK == 0 and 1 <= groups <= batch
    rng = np.random.default_rng(seed)
    priv = rng.integers(priv_lo, priv_hi + 1, size=batch)
    ctx = (prefix + priv).astype(np.int32)
    nblk = (ctx + BLOCK - 1) // BLOCK
    pblk = prefix // BLOCK
    shared = {b: (b % groups, pblk) for b in range(groups, batch)}
    distinct = int(nblk.sum()) - len(shared) * pblk
    pool = _pool_size(distinct)
    bt = _tables(rng, nblk.tolist(), pool, shared)
    g = _gen(seed, device)
    q = randn_bf16((batch, hq, d), g, device)
    k, v = _cache(pool, hkv, d, g, device)
    w = PagedWorkload(f"decode_b{batch}_shared{groups}x{prefix}+{priv_lo}-{priv_hi}", hq, hkv,
                      d, ctx, bt, pool, q, k, v)
    w.info["prefix"] = prefix
    w.info["groups"] = groups
    # bytes of distinct K/V positions: each group's prefix once, every private suffix
    w.info["unique_kv_bytes"] = (groups * prefix + int(priv.sum())) * hkv * d * 2 * 2
    return w


def decode_long(device="cpu", seed: int = 5, batch: int = 32, ctx: int = 32768,
                hq: int = 32, hkv: int = 8, d: int = 128) -> PagedWorkload:
    """Config 5: every context `ctx` tokens, blocks scattered across a shuffled pool."""
    rng = np.random.default_rng(seed)
    nblk = -(-ctx // BLOCK)
    pool = _pool_size(batch * nblk)
    bt = _tables(rng, [nblk] * batch, pool)
    g = _gen(seed, device)
    q = randn_bf16((batch, hq, d), g, device)
    k, v = _cache(pool, hkv, d, g, device)
    return PagedWorkload(f"decode_b{batch}_ctx{ctx}_gqa{hq // hkv}", hq, hkv, d,
                         np.full(batch, ctx, np.int32), bt, pool, q, k, v)


def prefill_prefix(device="cpu", seed: int = 3, n_seqs: int = 8, prefix: int = 512,
                   new=1536, share_pairs=((1, 0),), hq: int = 16, hkv: int = 8,
                   d: int = 128) -> PagedWorkload:
    """Config 3: n_seqs x (cached prefix + new prompt tokens), causal; seq 1 shares seq 0's
    prefix blocks. `new` is one length for every sequence or one per sequence. The new
    tokens' K/V are returned in k_new/v_new + slot_mapping (to be written before attention)."""
    assert prefix % BLOCK == 0
    rng = np.random.default_rng(seed)
    news = np.full(n_seqs, new, np.int64) if np.isscalar(new) else np.asarray(new, np.int64)
    assert news.shape == (n_seqs,) and np.all(news > 0)
    ctx = prefix + news
    nblk = -(-ctx // BLOCK)
    pblk = prefix // BLOCK
    shared = {dst: (src, pblk) for dst, src in share_pairs}
    distinct = int(nblk.sum()) - len(shared) * pblk
    pool = _pool_size(distinct)
    bt = _tables(rng, nblk.tolist(), pool, shared)
    g = _gen(seed, device)
    qsl = np.concatenate([[0], np.cumsum(news)]).astype(np.int32)
    total = int(qsl[-1])
    q = randn_bf16((total, hq, d), g, device)
    k, v = _cache(pool, hkv, d, g, device)
    seq = np.repeat(np.arange(n_seqs), news)
    pos = prefix + np.arange(total) - qsl[seq]
    slot = (bt[seq, pos // BLOCK] * BLOCK + pos % BLOCK).astype(np.int32)
    label = f"{int(news[0])}" if np.all(news == news[0]) else f"{int(news.min())}..{int(news.max())}"
    w = PagedWorkload(f"prefill_{n_seqs}x({prefix}+{label})", hq, hkv, d, ctx.astype(np.int32),
                      bt, pool, q, k, v, query_start_loc=qsl)
    w.slot_mapping = slot
    w.k_new = randn_bf16((total, hkv, d), g, device)
    w.v_new = randn_bf16((total, hkv, d), g, device)
    w.info["prefix"] = prefix
    w.info["new"] = int(news[0]) if np.all(news == news[0]) else news.tolist()
    return w


def mixed_step(device="cpu", seed: int = 4, n_chunks: int = 4, chunk: int = 512,
               prefix_hi: int = 2048, n_decode: int = 128, dec_lo: int = 1024,
               dec_hi: int = 32768, hq: int = 16, hkv: int = 8, d: int = 128) -> PagedWorkload:
    """Config 4: chunked-prefill items (prefix ~ U[0, prefix_hi], multiple of 16) followed
    by single-token decode items (ctx ~ logU[dec_lo, dec_hi]) over one block table."""
    rng = np.random.default_rng(seed)
    pre = rng.integers(0, prefix_hi // BLOCK + 1, size=n_chunks) * BLOCK
    dctx = np.floor(np.exp(rng.uniform(np.log(dec_lo), np.log(dec_hi), size=n_decode)))
    ctx = np.concatenate([pre + chunk, dctx]).astype(np.int32)
    qlen = np.concatenate([np.full(n_chunks, chunk), np.ones(n_decode)]).astype(np.int32)
    nblk = (ctx + BLOCK - 1) // BLOCK
    pool = _pool_size(int(nblk.sum()))
    bt = _tables(rng, nblk.tolist(), pool)
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    total = int(qsl[-1])
    g = _gen(seed, device)
    q = randn_bf16((total, hq, d), g, device)
    k, v = _cache(pool, hkv, d, g, device)
    seq = np.repeat(np.arange(ctx.size), qlen)
    pos = (np.arange(total) - qsl[seq]) + (ctx - qlen)[seq]
    slot = (bt[seq, pos // BLOCK] * BLOCK + pos % BLOCK).astype(np.int32)
    w = PagedWorkload(f"mixed_{n_chunks}x{chunk}+{n_decode}dec", hq, hkv, d, ctx, bt, pool, q,
                      k, v, query_start_loc=qsl)
    w.slot_mapping = slot
    w.k_new = randn_bf16((total, hkv, d), g, device)
    w.v_new = randn_bf16((total, hkv, d), g, device)
    w.info["n_chunks"] = n_chunks
    w.info["n_decode"] = n_decode
    return w


def prefill_flops(w: PagedWorkload) -> int:
    """Algorithmic prefill FLOPs: 4 * D * Hq per visible (query, key) pair, masked work not
    counted, single-token (decode) items excluded."""
    qsl = w.query_start_loc
    total = 0
    for b in range(w.batch):
        ql = int(qsl[b + 1] - qsl[b])
        if ql <= 1:
            continue
        pre = int(w.context_lens[b]) - ql
        total += ql * pre + ql * (ql + 1) // 2
    return 4 * w.d * w.hq * total


def decode_items_kv_bytes(w: PagedWorkload) -> int:
    """K+V bytes of the single-token items of a mixed batch (once per seq, kv_head)."""
    qsl = w.query_start_loc
    ql = qsl[1:] - qsl[:-1]
    return int(np.sum(w.context_lens[ql == 1].astype(np.int64))) * w.hkv * w.d * 4


@dataclass
class PrologueWorkload:
    """One layer's attention prologue input: the packed QKV projection of `tokens` tokens,
    q/k RMSNorm weights, positions, a (cos, sin) table and the slots of a paged KV cache."""
    name: str
    hq: int
    hkv: int
    d: int
    qkv: torch.Tensor            # [tokens, (hq + 2 hkv) d] bf16
    q_norm_w: torch.Tensor       # [d] bf16
    k_norm_w: torch.Tensor       # [d] bf16
    positions: torch.Tensor      # [tokens] int32
    rope_cache: torch.Tensor     # [max_position, d / 2, 2] float32
    slot_mapping: torch.Tensor   # [tokens] int32
    k_cache: torch.Tensor        # [slots, hkv, d] bf16
    v_cache: torch.Tensor
    q_out: torch.Tensor          # [tokens, hq, d] bf16

    @property
    def tokens(self) -> int:
        return self.qkv.shape[0]

    def bytes(self) -> int:
        """Algorithmic HBM bytes: the QKV rows read once, q written, K and V written to the
        cache, one (cos, sin) row, position and slot per token, and the two weight rows."""
        per_token = ((self.hq + 2 * self.hkv) * self.d * 2 + self.hq * self.d * 2
                     + 2 * self.hkv * self.d * 2 + (self.d // 2) * 8 + 8)
        return self.tokens * per_token + 2 * self.d * 2


def rope_cache_table(max_position: int, rotary_dim: int, theta: float, device) -> torch.Tensor:
    """(cos, sin) of pos * theta^(-2p / rotary_dim) in float32, [max_position, rotary_dim/2, 2]
    (the table src/model/rope/rope_cache.cpp builds on the host)."""
    half = rotary_dim // 2
    p = torch.arange(half, dtype=torch.float32)
    inv = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float32), p * 2.0 / rotary_dim)
    ang = torch.arange(max_position, dtype=torch.float32)[:, None] * inv[None, :]
    return torch.stack([torch.cos(ang), torch.sin(ang)], -1).contiguous().to(device)


def prologue(device="cpu", seed: int = 6, tokens: int = 64, hq: int = 16, hkv: int = 8,
             d: int = 128, max_position: int = 40960, theta: float = 1e6,
             cache_slots: Optional[int] = None) -> PrologueWorkload:
    """Decode-side prologue of one layer: `tokens` new tokens (one per sequence for a decode
    batch) at random positions, written to distinct random slots of the cache."""
    rng = np.random.default_rng(seed)
    slots = cache_slots or max(4 * tokens, 1024)
    g = _gen(seed, device)
    qkv = randn_bf16((tokens, (hq + 2 * hkv) * d), g, device)
    qn = randn_bf16((d,), g, device)
    kn = randn_bf16((d,), g, device)
    pos = torch.from_numpy(rng.integers(0, max_position, tokens).astype(np.int32)).to(device)
    sm = torch.from_numpy(rng.permutation(slots)[:tokens].astype(np.int32)).to(device)
    kc = torch.zeros((slots, hkv, d), dtype=torch.bfloat16, device=device)
    return PrologueWorkload(f"prologue_t{tokens}", hq, hkv, d, qkv, qn, kn, pos,
                            rope_cache_table(max_position, d, theta, device), sm, kc,
                            torch.zeros_like(kc),
                            torch.empty((tokens, hq, d), dtype=torch.bfloat16, device=device))
