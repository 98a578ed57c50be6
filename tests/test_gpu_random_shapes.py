"""Seeded random shapes across every decode and prefill path against the CPU oracle.

Each case draws a head dim from the reference's decode list (native MFMA sizes and the ones
padded to 64 / 128 / 256), a query-group size from 1 to 32 (above 16: virtual kv heads),
a batch size and context range that select the group plan, the fixed split plan or the
balanced split plan, and optionally holes in the block table; every cache slot no request
may read is poisoned (K = NaN, V = Inf), so a gather outside the visible positions shows as
a non-finite output. Decode cases also run the decode step with the new tokens' KV write
in the launch and check it bit-equal to write_kv_cache + decode_attention. Reference
behaviour: src/kernel/attention/decode_attn.cu:364-473, prefill_attn.cu:80-241,
write_kv_cache.cu:12-34. Bar: max-abs <= 2e-2, mean-abs <= 2e-3 on every row. The fp8 cases
(no reference counterpart) poison unused slots with the E4M3 NaN code; mixed batches run
chunked prefills and decode items in one prefill call.
"""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import (decode_attention, decode_attention_fp8, decode_attention_write_kv,
                         prefill_attention, prefill_attention_fp8, write_kv_cache)
from ccinfer_amd import workloads as W
from tests._util import assert_attn_close, f32, from_u16, say, u16
from tests.test_gpu_fp8 import _dequant_bf16, quantised_cache

pytestmark = pytest.mark.gpu

HEAD_DIMS = (32, 64, 80, 96, 112, 120, 128, 192, 256)
GROUPS = (1, 2, 3, 4, 5, 8, 16, 24, 32)


def _unused_rows(w, dev):
    used = np.zeros(w.num_blocks * 16, bool)
    for b in range(w.batch):
        n = min(int(w.context_lens[b]), w.mbpr * 16)
        pos = np.arange(n)
        blk = w.block_table[b, pos // 16]
        ok = blk >= 0
        used[blk[ok] * 16 + pos[ok] % 16] = True
    return torch.from_numpy(np.nonzero(~used)[0]).to(dev)


def _poison_unused(w, dev):
    rows = _unused_rows(w, dev)
    if rows.numel():
        w.k_cache[rows] = float("nan")
        w.v_cache[rows] = float("inf")


def _decode_case(seed):
    rng = np.random.default_rng(seed)
    d = int(rng.choice(HEAD_DIMS))
    g = int(rng.choice(GROUPS))
    hkv = int(rng.choice((1, 2, 4, 8)))
    plan = int(rng.integers(0, 3))  # 0: group, 1: fixed split, 2: balanced split
    if plan == 0:
        batch, lo, hi = 1, 1, 500
        hkv = max(1, min(hkv, 16 // g)) if g <= 16 else 1
    elif plan == 1:
        batch, lo, hi = int(rng.integers(1, 4)), 1, int(rng.integers(600, 5000))
    else:
        batch, lo, hi = int(rng.integers(4, 70)), 1, int(rng.integers(100, 3000))
    hkv = max(1, min(hkv, 64 // g))  # at most 64 q-heads (keeps the CPU oracle quick)
    return d, g * hkv, hkv, batch, lo, hi, bool(rng.integers(0, 2))


@pytest.mark.parametrize("seed", range(24))
def test_random_decode(gpu, seed):
    d, hq, hkv, batch, lo, hi, holes = _decode_case(seed)
    say(f"random decode seed={seed} d={d} hq={hq} hkv={hkv} B={batch} ctx=[{lo},{hi}] "
        f"holes={holes}")
    w = W.decode_batched(device=gpu, seed=1000 + seed, batch=batch, ctx_lo=lo, ctx_hi=hi,
                         hq=hq, hkv=hkv, d=d, with_write=True)
    if holes and w.mbpr > 2:
        bt = w.block_table.copy()
        rng = np.random.default_rng(seed)
        for b in range(0, batch, 2):
            nb = int(np.count_nonzero(bt[b] >= 0))
            if nb > 2:
                bt[b, int(rng.integers(0, nb - 1))] = -1   # never the last block
        w.block_table = bt
    kc, vc = w.k_cache.clone(), w.v_cache.clone()
    meta = w.device_meta(gpu)
    write_kv_cache(w.k_new, w.v_new, kc, vc, meta["slot_mapping"])
    want = decode_attention(w.q, kc, vc, meta["block_table"], meta["context_lens"])
    got = decode_attention_write_kv(w.q, w.k_new, w.v_new, w.k_cache, w.v_cache,
                                    meta["block_table"], meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(w.k_cache, kc) and torch.equal(w.v_cache, vc)
    assert torch.equal(got, want)
    _poison_unused(w, gpu)
    got = decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                           meta["context_lens"])
    torch.cuda.synchronize()
    ref = oracle.decode(u16(w.q), u16(w.k_cache), u16(w.v_cache), w.block_table,
                        w.context_lens)
    assert_attn_close(f32(got), ref, f"seed {seed}")


def _prefill_case(seed):
    rng = np.random.default_rng(10_000 + seed)
    d = int(rng.choice(HEAD_DIMS[:-1] + (256,)))
    g = int(rng.choice(GROUPS))
    hkv = int(rng.choice((1, 2, 4)))
    n = int(rng.integers(1, 6))
    prefix = int(rng.integers(0, 40)) * 16
    new = [int(x) for x in rng.integers(1, 400, size=n)]
    hkv = max(1, min(hkv, 64 // g))
    return d, g * hkv, hkv, n, prefix, new, bool(rng.integers(0, 2))


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill(gpu, seed):
    d, hq, hkv, n, prefix, new, share = _prefill_case(seed)
    say(f"random prefill seed={seed} d={d} hq={hq} hkv={hkv} n={n} prefix={prefix} "
        f"new={new} share={share}")
    w = W.prefill_prefix(device=gpu, seed=2000 + seed, n_seqs=n, prefix=prefix, new=new,
                         share_pairs=((1, 0),) if share and n > 1 and prefix > 0 else (),
                         hq=hq, hkv=hkv, d=d)
    meta = w.device_meta(gpu)
    write_kv_cache(w.k_new, w.v_new, w.k_cache, w.v_cache, meta["slot_mapping"])
    _poison_unused(w, gpu)
    got = prefill_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                            meta["query_start_loc"], meta["context_lens"])
    torch.cuda.synchronize()
    ref = oracle.prefill(u16(w.q), u16(w.k_cache), u16(w.v_cache), w.block_table,
                         w.query_start_loc, w.context_lens)
    assert_attn_close(f32(got), ref, f"seed {seed}")


FP8_DIMS = (64, 128, 256)


@pytest.mark.parametrize("seed", range(12))
def test_random_decode_fp8(gpu, seed):
    """fp8 cache (native head dims): every plan and group size, unused slots holding the
    E4M3 NaN code (0x7f), against the oracle's decode over the same fp8 cache."""
    d, hq, hkv, batch, lo, hi, _ = _decode_case(500 + seed)
    if d not in FP8_DIMS:
        d = FP8_DIMS[seed % 3]
    say(f"random fp8 decode seed={seed} d={d} hq={hq} hkv={hkv} B={batch} ctx=[{lo},{hi}]")
    w = W.decode_batched(device=gpu, seed=3000 + seed, batch=batch, ctx_lo=lo, ctx_hi=hi,
                         hq=hq, hkv=hkv, d=d, with_write=False)
    kc, vc, ks, vs = quantised_cache(gpu, w, hkv, d)
    rows = _unused_rows(w, gpu)
    if rows.numel():
        kc[rows] = 0x7F
        vc[rows] = 0x7F
    meta = w.device_meta(gpu)
    got = decode_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"], meta["context_lens"])
    torch.cuda.synchronize()
    ref = oracle.decode_fp8(u16(w.q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                            vs.cpu().numpy(), w.block_table, w.context_lens)
    assert_attn_close(f32(got), ref, f"fp8 seed {seed}")


@pytest.mark.parametrize("seed", range(8))
def test_random_prefill_fp8(gpu, seed):
    """fp8 prefill (head dims 64 / 128): bit-identical to the bf16 prefill over the
    dequantised cache, with every unused slot poisoned in both caches."""
    d, hq, hkv, n, prefix, new, share = _prefill_case(600 + seed)
    d = (64, 128)[seed % 2]
    say(f"random fp8 prefill seed={seed} d={d} hq={hq} hkv={hkv} n={n} prefix={prefix} "
        f"new={new}")
    w = W.prefill_prefix(device=gpu, seed=4000 + seed, n_seqs=n, prefix=prefix, new=new,
                         share_pairs=((1, 0),) if share and n > 1 and prefix > 0 else (),
                         hq=hq, hkv=hkv, d=d)
    meta = w.device_meta(gpu)
    write_kv_cache(w.k_new, w.v_new, w.k_cache, w.v_cache, meta["slot_mapping"])
    kc, vc, ks, vs = quantised_cache(gpu, w, hkv, d)
    kb = from_u16(_dequant_bf16(kc.cpu().numpy(), ks.cpu().numpy(), hkv), gpu)
    vb = from_u16(_dequant_bf16(vc.cpu().numpy(), vs.cpu().numpy(), hkv), gpu)
    rows = _unused_rows(w, gpu)
    if rows.numel():
        kc[rows] = 0x7F
        vc[rows] = 0x7F
        kb[rows] = float("nan")
        vb[rows] = float("inf")
    out8 = prefill_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"],
                                 meta["query_start_loc"], meta["context_lens"])
    out16 = prefill_attention(w.q, kb, vb, meta["block_table"], meta["query_start_loc"],
                              meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(out8, out16)
    assert bool(torch.isfinite(out8).all())


@pytest.mark.parametrize("seed", range(8))
def test_random_mixed(gpu, seed):
    """Mixed batches (chunked prefills + single-token decode items) over every head dim and
    group size, with 2..48 decode items (group plan or split plan for them), unused slots
    poisoned, against the oracle."""
    rng = np.random.default_rng(7000 + seed)
    d = int(rng.choice(HEAD_DIMS))
    g = int(rng.choice(GROUPS))
    hkv = max(1, min(int(rng.choice((1, 2, 4))), 64 // g))
    n_chunks = int(rng.integers(1, 4))
    chunk = int(rng.integers(2, 300))
    n_decode = int(rng.integers(2, 49))
    dec_hi = int(rng.choice((400, 3000)))
    say(f"random mixed seed={seed} d={d} hq={g * hkv} hkv={hkv} chunks={n_chunks}x{chunk} "
        f"decodes={n_decode} dec_hi={dec_hi}")
    w = W.mixed_step(device=gpu, seed=8000 + seed, n_chunks=n_chunks, chunk=chunk,
                     prefix_hi=512, n_decode=n_decode, dec_lo=1, dec_hi=dec_hi, hq=g * hkv,
                     hkv=hkv, d=d)
    meta = w.device_meta(gpu)
    write_kv_cache(w.k_new, w.v_new, w.k_cache, w.v_cache, meta["slot_mapping"])
    _poison_unused(w, gpu)
    got = prefill_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                            meta["query_start_loc"], meta["context_lens"])
    torch.cuda.synchronize()
    ref = oracle.prefill(u16(w.q), u16(w.k_cache), u16(w.v_cache), w.block_table,
                         w.query_start_loc, w.context_lens)
    assert_attn_close(f32(got), ref, f"mixed seed {seed}")


@pytest.mark.parametrize("seed", range(9))
def test_random_large_batch_decode(gpu, seed):
    """Batches of 257-1200 requests (the flat plan's index kernel, equal, snapped or
    whole-request ranges) over every decode head dim and group size, holes in the table and
    unread slots poisoned: every output finite, a sample of rows against the oracle."""
    rng = np.random.default_rng(900 + seed)
    d = HEAD_DIMS[seed]
    g = int(rng.choice(GROUPS))
    hkv = max(1, min(int(rng.choice((1, 2, 4, 8))), 32 // g))
    batch = int(rng.integers(257, 1201))
    hi = int(rng.integers(200, 3001))
    say(f"random large decode seed={seed} d={d} hq={g * hkv} hkv={hkv} B={batch} "
        f"ctx=[1,{hi}]")
    w = W.decode_batched(device=gpu, seed=9000 + seed, batch=batch, ctx_lo=1, ctx_hi=hi,
                         hq=g * hkv, hkv=hkv, d=d, with_write=False)
    bt = w.block_table.copy()
    for b in range(0, batch, 5):
        nb = int(np.count_nonzero(bt[b] >= 0))
        if nb > 2:
            bt[b, int(rng.integers(0, nb - 1))] = -1
    w.block_table = bt
    _poison_unused(w, gpu)
    meta = w.device_meta(gpu)
    got = f32(decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                               meta["context_lens"]))
    assert np.all(np.isfinite(got))
    rows = np.unique(np.r_[0:16, rng.integers(0, batch, size=48), batch - 8:batch])
    ref = oracle.decode(u16(w.q)[rows], u16(w.k_cache), u16(w.v_cache), w.block_table[rows],
                        w.context_lens[rows])
    assert_attn_close(got[rows], ref, f"large seed {seed}")
