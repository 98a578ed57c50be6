"""Full-size parity: every (row, head) of configs[2], configs[3] and configs[4] against the
CPU oracle, with every cache slot that no request may read poisoned (K = NaN, V = Inf).

The poison turns block-table indexing into an exact check on the fast paths: a gather that
leaves the visible positions (a wrong block id, row, head or tile offset) makes the output
non-finite, and any other mistake in a tile, head or row shows up against the oracle, which
reads only the visible positions. Reference behaviour: src/kernel/attention/prefill_attn.cu
:80-241 and decode_attn.cu:364-473; reference tests: tests/kernel/test_prefill_attn.cu:24-105,
tests/integration/test_prefix_cache_e2e.cpp:19-171, tests/kernel/test_decode_attn.cu:229-311.
Bar: max-abs <= 2e-2 and mean-abs <= 2e-3 on all rows.
"""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import (decode_attention, fp8_scale_numel, prefill_attention,
                         prefill_attention_fp8, write_kv_cache, write_kv_cache_fp8)
from ccinfer_amd import workloads as W
from tests._util import assert_attn_close, f32, say, u16

pytestmark = pytest.mark.gpu


def used_slots(w) -> np.ndarray:
    """Boolean mask over cache slots: slots some request's visible positions map to."""
    used = np.zeros(w.num_blocks * 16, bool)
    for b in range(w.batch):
        n = min(int(w.context_lens[b]), w.mbpr * 16)
        pos = np.arange(n)
        blk = w.block_table[b, pos // 16]
        ok = blk >= 0
        used[blk[ok] * 16 + pos[ok] % 16] = True
    return used


def poison_unused(w, dev):
    rows = torch.from_numpy(np.nonzero(~used_slots(w))[0]).to(dev)
    assert rows.numel() > 0
    w.k_cache[rows] = float("nan")
    w.v_cache[rows] = float("inf")
    return rows.numel()


def run_prefill(w, dev):
    meta = w.device_meta(dev)
    out = prefill_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                            meta["query_start_loc"], meta["context_lens"])
    torch.cuda.synchronize()
    return out


def oracle_prefill(w):
    return oracle.prefill(u16(w.q), u16(w.k_cache), u16(w.v_cache), w.block_table,
                          w.query_start_loc, w.context_lens)


def write_new(w, dev):
    write_kv_cache(w.k_new, w.v_new, w.k_cache, w.v_cache,
                   torch.from_numpy(w.slot_mapping).to(dev))


def test_config3_prefill_all_rows_poisoned(gpu):
    say("full-size configs[2] prefill 8x(512+1536), all rows, unused slots poisoned")
    w = W.prefill_prefix(device=gpu)
    write_new(w, gpu)
    n = poison_unused(w, gpu)
    got = f32(run_prefill(w, gpu))
    want = oracle_prefill(w)
    assert_attn_close(got, want, f"configs[2] ({n} poisoned slots)")


def test_config4_mixed_all_rows_poisoned(gpu):
    say("full-size configs[3] mixed 4x512 + 128 decodes, all rows, unused slots poisoned")
    w = W.mixed_step(device=gpu)
    write_new(w, gpu)
    n = poison_unused(w, gpu)
    got = f32(run_prefill(w, gpu))
    want = oracle_prefill(w)
    assert_attn_close(got, want, f"configs[3] ({n} poisoned slots)")


def test_config5_decode_all_rows_poisoned(gpu):
    say("full-size configs[4] decode b32 ctx32768 gqa4, all rows, unused slots poisoned")
    w = W.decode_long(device=gpu)
    n = poison_unused(w, gpu)
    meta = w.device_meta(gpu)
    got = f32(decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                               meta["context_lens"]))
    want = oracle.decode(u16(w.q), u16(w.k_cache), u16(w.v_cache), w.block_table,
                         w.context_lens)
    assert_attn_close(got, want, f"configs[4] ({n} poisoned slots)")


@pytest.mark.parametrize("hq,hkv,d,prefix,new,holes", [
    (16, 8, 128, 512, 300, False), (16, 8, 128, 96, 700, True), (32, 8, 128, 64, 257, False),
    (8, 8, 64, 128, 400, True), (16, 8, 256, 48, 200, True),
    # head dims below 64 / 128 / 256 run those kernels padded with zeros
    (16, 8, 80, 208, 300, True), (8, 2, 32, 128, 400, False), (8, 4, 192, 64, 250, True),
    (16, 4, 112, 96, 333, False), (4, 4, 120, 512, 129, True), (8, 8, 72, 64, 200, False)])
def test_prefill_poisoned_shapes(gpu, hq, hkv, d, prefix, new, holes):
    """Ragged tiles, a shared prefix and (optionally) table holes, on every head shape's
    fast path, with all unreadable slots poisoned."""
    say(f"prefill poison hq={hq} hkv={hkv} d={d} prefix={prefix} new={new} holes={holes}")
    w = W.prefill_prefix(device=gpu, seed=hq + d + new, n_seqs=4, prefix=prefix, new=new,
                         share_pairs=((1, 0),), hq=hq, hkv=hkv, d=d)
    write_new(w, gpu)
    if holes:
        bt = w.block_table.copy()
        bt[2, 1] = -1          # a hole inside the cached prefix
        bt[3, bt.shape[1] // 2] = -1
        w.block_table = bt
    poison_unused(w, gpu)
    assert_attn_close(f32(run_prefill(w, gpu)), oracle_prefill(w), "poisoned prefill")


@pytest.mark.parametrize("d,hq,hkv,dec_hi", [(96, 8, 4, 3000), (192, 8, 4, 3000),
                                            (128, 32, 1, 3000),
                                            (128, 32, 1, 300), (80, 16, 8, 300)])
def test_mixed_padded_head_dim_or_wide_group_poisoned(gpu, d, hq, hkv, dec_hi):
    """A mixed batch (chunked prefills + decode items) at a padded head dim, or with 32
    query heads per KV head; rows of at most 512 positions send the decode items to the
    one-launch group kernel, longer ones to the split kernel + merge."""
    say(f"mixed batch d={d} hq={hq} hkv={hkv} dec_hi={dec_hi}, unused slots poisoned")
    short = dec_hi <= 512
    w = W.mixed_step(device=gpu, seed=d + hq, n_chunks=3, chunk=100 if short else 200,
                     prefix_hi=128 if short else 512, n_decode=40, dec_lo=16, dec_hi=dec_hi,
                     hq=hq, hkv=hkv, d=d)
    if short:
        assert w.mbpr * 16 <= 512
    write_new(w, gpu)
    poison_unused(w, gpu)
    assert_attn_close(f32(run_prefill(w, gpu)), oracle_prefill(w), f"mixed d{d}")


def test_prefill_fp8_poisoned(gpu):
    """fp8 cache: unreadable slots hold NaN bytes (0x7f) and NaN row scales."""
    say("fp8 prefill with poisoned unused slots and scales")
    hq, hkv, d = 16, 8, 128
    w = W.prefill_prefix(device=gpu, seed=77, n_seqs=4, prefix=256, new=333,
                         share_pairs=((1, 0),), hq=hq, hkv=hkv, d=d)
    write_new(w, gpu)
    slots = w.num_blocks * 16
    kc = torch.empty((slots, hkv, d), dtype=torch.uint8, device=gpu)
    vc = torch.empty_like(kc)
    ks = torch.empty(fp8_scale_numel(slots, hkv), dtype=torch.float32, device=gpu)
    vs = torch.empty_like(ks)
    write_kv_cache_fp8(w.k_cache, w.v_cache, kc, vc, ks, vs,
                       torch.arange(slots, dtype=torch.int32, device=gpu))
    unused = np.nonzero(~used_slots(w))[0]
    rows = torch.from_numpy(unused).to(gpu)
    kc[rows] = 0x7F
    vc[rows] = 0xFF
    sidx = oracle.fp8_scale_index(unused[:, None], np.arange(hkv)[None, :], hkv).reshape(-1)
    sidx = torch.from_numpy(sidx.astype(np.int64)).to(gpu)
    ks[sidx] = float("nan")
    vs[sidx] = float("inf")
    meta = w.device_meta(gpu)
    out = prefill_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"],
                                meta["query_start_loc"], meta["context_lens"])
    torch.cuda.synchronize()
    want = oracle.prefill_fp8(u16(w.q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                              vs.cpu().numpy(), w.block_table, w.query_start_loc, w.context_lens)
    assert_attn_close(f32(out), want, "poisoned fp8 prefill")
