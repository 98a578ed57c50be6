"""Paged decode attention on the GPU against the CPU oracle (and closed forms).

Reference behaviour: src/kernel/attention/decode_attn.cu:364-473; reference tests:
tests/kernel/test_decode_attn.cu (SingleDecodeStep :88-163, GQA :165-227,
RandomPagedGQAMatchesCpuReference :229-311, NullPointers :313-325).
Bar: max-abs <= 2e-2 and mean-abs <= 2e-3 against the fp32 oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import CcinferError, decode_attention, write_kv_cache
from ccinfer_amd import workloads as W
from tests._util import assert_attn_close, f32, from_u16, say, u16

pytestmark = pytest.mark.gpu


def run_decode(w: W.PagedWorkload, dev, block_size=16):
    meta = w.device_meta(dev)
    out = decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                           meta["context_lens"], cache_block_size=block_size)
    torch.cuda.synchronize()
    return out


def oracle_decode(w: W.PagedWorkload, pairs=None, block_size=16):
    return oracle.decode(u16(w.q), u16(w.k_cache), u16(w.v_cache), w.block_table,
                         w.context_lens, block_size=block_size, pairs=pairs)


def _kat(dev):
    b, hq, hkv, d, nphys = 2, 8, 2, 64, 3
    qi = np.arange(b * hq * d)
    ki = np.arange(nphys * 16 * hkv * d)
    q = oracle.f32_to_bf16((((qi * 17) % 23 - 11) * 0.03125).astype(np.float32))
    k = oracle.f32_to_bf16((((ki * 13) % 29 - 14) * 0.025).astype(np.float32))
    v = oracle.f32_to_bf16((((ki * 7) % 31 - 15) * 0.02).astype(np.float32))
    return W.PagedWorkload(
        "kat", hq, hkv, d, np.array([31, 17], np.int32),
        np.array([[2, 0, 1], [1, 2, -1]], np.int32), nphys,
        from_u16(q.reshape(b, hq, d), dev), from_u16(k.reshape(-1, hkv, d), dev),
        from_u16(v.reshape(-1, hkv, d), dev))


def test_reference_kat_random_paged_gqa(gpu):
    say("decode KAT RandomPagedGQAMatchesCpuReference")
    w = _kat(gpu)
    got = f32(run_decode(w, gpu))
    want = oracle_decode(w)
    mx, _ = assert_attn_close(got, want, "KAT")
    assert mx < 0.01  # the reference test's own bound


def test_uniform_scores_give_mean_v(gpu):
    say("decode closed form Q=K=0.1 V=0.2")
    b, hq, hkv, d = 2, 4, 4, 64
    q = torch.full((b, hq, d), 0.1, dtype=torch.bfloat16, device=gpu)
    k = torch.full((32, hkv, d), 0.1, dtype=torch.bfloat16, device=gpu)
    v = torch.full((32, hkv, d), 0.2, dtype=torch.bfloat16, device=gpu)
    bt = torch.tensor([[0, 1], [0, 1]], dtype=torch.int32, device=gpu)
    cl = torch.tensor([32, 32], dtype=torch.int32, device=gpu)
    out = f32(decode_attention(q, k, v, bt, cl))
    vbf = float(torch.tensor(0.2, dtype=torch.bfloat16))
    assert np.allclose(out, vbf, atol=2e-3)
    assert np.array_equal(out[0], out[1])


def test_gqa_heads_equal(gpu):
    say("decode GQA heads equal")
    q = torch.full((1, 8, 64), 0.1, dtype=torch.bfloat16, device=gpu)
    kv = torch.full((16, 2, 64), 0.1, dtype=torch.bfloat16, device=gpu)
    out = f32(decode_attention(q, kv, kv, torch.zeros((1, 1), dtype=torch.int32, device=gpu),
                               torch.tensor([16], dtype=torch.int32, device=gpu)))
    assert np.abs(out - out[:, :1]).max() < 1e-2


def test_config1_single_sequence(gpu):
    say("decode config1 b1 ctx512")
    w = W.decode_single(device=gpu)
    assert_attn_close(f32(run_decode(w, gpu)), oracle_decode(w), "config1")


def test_config2_batched_with_write(gpu):
    say("decode config2 b64 ctx U[128,4096] + write")
    w = W.decode_batched(device=gpu)
    meta = w.device_meta(gpu)
    write_kv_cache(w.k_new, w.v_new, w.k_cache, w.v_cache, meta["slot_mapping"])
    got = f32(run_decode(w, gpu))
    assert_attn_close(got, oracle_decode(w), "config2")


def test_config5_long_context_sampled(gpu):
    say("decode config5 b32 ctx32768 gqa4 (sampled rows)")
    w = W.decode_long(device=gpu)
    got = f32(run_decode(w, gpu))
    rng = np.random.default_rng(11)
    pairs = np.stack([rng.integers(0, w.batch, 48), rng.integers(0, w.hq, 48)], 1)
    pairs = np.concatenate([pairs, [[0, 0], [w.batch - 1, w.hq - 1]]]).astype(np.int32)
    want = oracle_decode(w, pairs=pairs)
    assert_attn_close(got[pairs[:, 0], pairs[:, 1]], want[pairs[:, 0], pairs[:, 1]], "config5")
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 64), (16, 8, 256), (8, 8, 128), (32, 8, 128),
                                      (64, 4, 128), (32, 1, 128),  # G=16, G=32 (2 x 16)
                                      (48, 2, 128), (17, 1, 64), (64, 1, 96),  # G=24, 17, 64
                                      (16, 8, 80), (12, 4, 96), (8, 2, 32), (8, 4, 192),
                                      (4, 2, 112), (4, 4, 120)])
def test_head_shapes(gpu, hq, hkv, d):
    say(f"decode shape hq={hq} hkv={hkv} d={d}")
    w = W.decode_batched(device=gpu, seed=hq * 1000 + hkv * 10 + d, batch=5, ctx_lo=1,
                         ctx_hi=700, hq=hq, hkv=hkv, d=d, with_write=False)
    assert_attn_close(f32(run_decode(w, gpu)), oracle_decode(w), f"hq{hq}/hkv{hkv}/d{d}")


@pytest.mark.parametrize("hq,hkv,d,batch,ctx_hi", [
    (16, 8, 80, 1, 500),      # one workgroup per (request, kv_head), parts merged in LDS
    (8, 2, 32, 1, 400),
    (8, 4, 192, 1, 300),      # head dim 192 tile
    (16, 8, 80, 2, 3000),     # fixed split plan + merge kernel
    (8, 2, 32, 3, 900),
    (8, 4, 192, 2, 2500),
    (16, 8, 96, 40, 5000),    # balanced split plan + merge kernel (head dim 96 tile)
    (16, 8, 96, 1, 500),      # head dim 96 tile: group plan
    (16, 8, 96, 2, 3000),     # head dim 96 tile: fixed split plan
    (64, 4, 96, 3, 700),      # head dim 96 tile, G = 16
    (8, 8, 120, 12, 4000),
    (8, 4, 192, 24, 3000),
    (16, 4, 112, 64, 2000),
    (8, 8, 32, 48, 6000)])
def test_padded_head_dims_every_plan(gpu, hq, hkv, d, batch, ctx_hi):
    """Head dims below 64 / 128 / 256 run the MFMA kernels padded with zeros (32, 96 and 192
    in tiles of their own); every decode plan (LDS-merged groups, balanced splits with the
    merge kernel) against the oracle."""
    say(f"decode padded d={d} hq={hq} hkv={hkv} batch={batch} ctx<={ctx_hi}")
    w = W.decode_batched(device=gpu, seed=d * 7 + batch, batch=batch, ctx_lo=1, ctx_hi=ctx_hi,
                         hq=hq, hkv=hkv, d=d, with_write=False)
    assert_attn_close(f32(run_decode(w, gpu)), oracle_decode(w), f"padded d{d} b{batch}")


def test_edge_cases_zero_ctx_overflow_and_holes(gpu):
    say("decode edge cases")
    w = W.decode_batched(device=gpu, seed=21, batch=6, ctx_lo=40, ctx_hi=300, with_write=False)
    ctx = w.context_lens.copy()
    bt = w.block_table.copy()
    ctx[0] = 0                                   # -> zeros
    ctx[1] = bt.shape[1] * 16 + 1                # more blocks than the row holds -> zeros
    ctx[2] = int(np.count_nonzero(bt[2] >= 0)) * 16
    bt[2, 1] = -1                                # hole: those 16 positions are skipped
    ctx[3] = 1                                   # single position
    w.context_lens, w.block_table = ctx.astype(np.int32), bt
    got = f32(run_decode(w, gpu))
    want = oracle_decode(w)
    assert np.all(got[0] == 0) and np.all(got[1] == 0)
    assert_attn_close(got, want, "edge")


def test_unwritten_slots_holding_nan_do_not_leak(gpu):
    say("decode NaN in unused slots")
    w = W.decode_batched(device=gpu, seed=5, batch=8, ctx_lo=17, ctx_hi=200, with_write=False)
    used = np.zeros(w.num_blocks * 16, bool)
    for b in range(w.batch):
        pos = np.arange(w.context_lens[b])
        used[w.block_table[b, pos // 16] * 16 + pos % 16] = True
    nan_rows = torch.from_numpy(np.nonzero(~used)[0]).to(gpu)
    w.k_cache[nan_rows] = float("nan")
    w.v_cache[nan_rows] = float("inf")
    got = f32(run_decode(w, gpu))
    assert np.all(np.isfinite(got))
    assert_attn_close(got, oracle_decode(w), "nan-slots")


def test_deterministic(gpu):
    say("decode determinism")
    w = W.decode_batched(device=gpu, seed=9, batch=16, with_write=False)
    a = u16(run_decode(w, gpu))
    b = u16(run_decode(w, gpu))
    assert np.array_equal(a, b)


def test_rejects_bad_arguments(gpu):
    say("decode argument errors")
    w = _kat(gpu)
    meta = w.device_meta(gpu)
    with pytest.raises(CcinferError) as e:
        decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"], meta["context_lens"],
                         cache_block_size=32)
    assert e.value.code == 6
    q7 = torch.zeros((2, 7, 64), dtype=torch.bfloat16, device=gpu)  # 7 % 2 != 0
    with pytest.raises(CcinferError):
        decode_attention(q7, w.k_cache, w.v_cache, meta["block_table"], meta["context_lens"])


def test_workspace_reuse_across_shapes(gpu):
    """One workspace (deliberately filled with garbage first) reused across calls with
    different contexts: the split-KV scratch needs no initialisation."""
    say("decode workspace reuse")
    from ccinfer_amd import decode_workspace_size
    w = W.decode_long(device=gpu, seed=31, batch=6, ctx=3000, hq=16, hkv=8)
    need = decode_workspace_size(w.batch, w.mbpr, w.hq, w.hkv, w.d)
    assert need > 0
    ws = torch.full((need,), 0x7f, dtype=torch.uint8, device=gpu)
    rng = np.random.default_rng(2)
    for it in range(4):
        w.context_lens = rng.integers(1, 3001, w.batch).astype(np.int32)
        meta = w.device_meta(gpu)
        out = decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                               meta["context_lens"], workspace=ws)
        torch.cuda.synchronize()
        assert_attn_close(f32(out), oracle_decode(w), f"reuse {it}")


def _offset_view(t: torch.Tensor, elems: int = 1) -> torch.Tensor:
    """A copy of `t` whose data pointer is `elems` bf16 elements past a 256-byte boundary."""
    flat = torch.empty(t.numel() + elems, dtype=t.dtype, device=t.device)
    v = flat[elems:].view(t.shape)
    v.copy_(t)
    return v


@pytest.mark.parametrize("which", ["q", "k_cache", "v_cache", "output"])
def test_two_byte_aligned_views(gpu, which):
    """The reference launchers take any bf16 view. A q or output view that is only 2-byte
    aligned runs the MFMA kernels on workspace copies of its rows; a cache that is only
    2-byte aligned runs them with 2-byte piece loads. Either way bit-equal to the aligned
    call."""
    say(f"decode with a 2-byte aligned {which}")
    w = W.decode_batched(device=gpu, seed=17, batch=6, ctx_lo=20, ctx_hi=600, with_write=False)
    meta = w.device_meta(gpu)
    args = {"q": w.q, "k_cache": w.k_cache, "v_cache": w.v_cache}
    out = None
    if which == "output":
        out = _offset_view(torch.zeros_like(w.q))
    else:
        args[which] = _offset_view(args[which])
    assert (args["q"].data_ptr() % 16 != 0) == (which == "q")
    got = decode_attention(args["q"], args["k_cache"], args["v_cache"], meta["block_table"],
                           meta["context_lens"], output=out)
    torch.cuda.synchronize()
    assert_attn_close(f32(got), oracle_decode(w), f"misaligned {which}")
    aligned = decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                               meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(got, aligned)


@pytest.mark.parametrize("batch,ctx_lo,ctx_hi,hq,hkv,d,offset", [
    (64, 128, 4096, 16, 8, 128, 1),   # configs[1]: flat plan with merge
    (1, 512, 512, 16, 8, 128, 3),     # group plan
    (2, 100, 3000, 16, 8, 256, 1),    # fixed split plan, head dim 256
    (300, 1, 400, 16, 8, 96, 5),      # indexed flat plan, head dim 96 tile
    (300, 1, 400, 16, 8, 80, 3),      # indexed flat plan, padded head dim
    (40, 50, 900, 8, 4, 192, 5),      # head dim 192 tile
    (40, 50, 900, 64, 2, 64, 7),      # 32 query heads per kv head (virtual heads)
    (64, 128, 4096, 16, 8, 128, 2),   # 4-byte aligned: word loads
    (1, 512, 512, 16, 8, 96, 6),      # 4-byte aligned, group plan, head dim 96 tile
])
def test_two_byte_aligned_caches_on_mfma_path(gpu, batch, ctx_lo, ctx_hi, hq, hkv, d, offset):
    """K and V caches offset by an odd number of elements (only 2-byte aligned): the MFMA
    kernels with 2-byte piece loads, bit-equal to the same call on aligned copies, every
    decode plan; the fused KV write falls back to its own launch and still writes the same
    rows."""
    from ccinfer_amd import decode_attention_write_kv
    say(f"decode 2-byte aligned caches B={batch} ctx=[{ctx_lo},{ctx_hi}] hq={hq} hkv={hkv} "
        f"d={d}")
    w = W.decode_batched(device=gpu, seed=batch + d + 1, batch=batch, ctx_lo=ctx_lo,
                         ctx_hi=ctx_hi, hq=hq, hkv=hkv, d=d, with_write=True)
    meta = w.device_meta(gpu)
    want = decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                            meta["context_lens"])
    kc, vc = _offset_view(w.k_cache, offset), _offset_view(w.v_cache, offset)
    got = decode_attention(w.q, kc, vc, meta["block_table"], meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # with the new token's write: same output and same cache rows as on the aligned caches
    ka, va = w.k_cache.clone(), w.v_cache.clone()
    want_w = decode_attention_write_kv(w.q, w.k_new, w.v_new, ka, va, meta["block_table"],
                                       meta["context_lens"])
    got_w = decode_attention_write_kv(w.q, w.k_new, w.v_new, kc, vc, meta["block_table"],
                                      meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(got_w, want_w)
    assert torch.equal(kc, ka) and torch.equal(vc, va)


@pytest.mark.parametrize("batch,ctx_lo,ctx_hi,hq,hkv,d,offset", [
    (64, 128, 4096, 16, 8, 128, 1),   # configs[1]: split plan with merge
    (1, 512, 512, 16, 8, 128, 3),     # group plan (one launch)
    (300, 1, 400, 16, 8, 96, 5),      # flat plan with index kernel, head dim 96 tile
])
def test_two_byte_aligned_q_and_output_on_mfma_path(gpu, batch, ctx_lo, ctx_hi, hq, hkv, d,
                                                    offset):
    """q and output both 2-byte aligned (offset by an odd number of elements), every decode
    plan: the staged call equals the aligned call bit for bit and leaves the bytes around
    the output view alone."""
    say(f"decode staged rows B={batch} ctx=[{ctx_lo},{ctx_hi}] hq={hq} hkv={hkv} d={d}")
    w = W.decode_batched(device=gpu, seed=batch + d, batch=batch, ctx_lo=ctx_lo, ctx_hi=ctx_hi,
                         hq=hq, hkv=hkv, d=d, with_write=False)
    meta = w.device_meta(gpu)
    want = decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                            meta["context_lens"])
    qv = _offset_view(w.q, offset)
    flat = torch.full((w.q.numel() + offset + 8,), 5.0, dtype=torch.bfloat16, device=gpu)
    ov = flat[offset:offset + w.q.numel()].view(w.q.shape)
    got = decode_attention(qv, w.k_cache, w.v_cache, meta["block_table"], meta["context_lens"],
                           output=ov)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.all(flat[:offset] == 5.0) and torch.all(flat[offset + w.q.numel():] == 5.0)


def _write_then_decode(w, dev, slot_mapping, k_cache, v_cache):
    meta = w.device_meta(dev)
    write_kv_cache(w.k_new, w.v_new, k_cache, v_cache,
                   torch.from_numpy(slot_mapping.astype(np.int32)).to(dev))
    return decode_attention(w.q, k_cache, v_cache, meta["block_table"], meta["context_lens"])


@pytest.mark.parametrize("batch,ctx_lo,ctx_hi,hq,hkv,d", [
    (64, 128, 4096, 16, 8, 128),   # configs[1]: balanced split plan + merge
    (1, 512, 512, 16, 8, 128),     # group plan (one launch)
    (2, 100, 3000, 16, 8, 128),    # fixed split plan
    (9, 1, 700, 16, 8, 96),        # padded head dim
    (6, 20, 900, 32, 1, 128),      # two virtual kv heads write the same row
    (300, 1, 400, 16, 8, 64),      # more than 256 requests
])
def test_fused_kv_write_equals_write_then_decode(gpu, batch, ctx_lo, ctx_hi, hq, hkv, d):
    """decode_attention_write_kv == write_kv_cache (slot of each request's last position)
    followed by decode_attention: output and both caches bit-equal."""
    from ccinfer_amd import decode_attention_write_kv
    say(f"fused write+decode B={batch} ctx=[{ctx_lo},{ctx_hi}] hq={hq} hkv={hkv} d={d}")
    w = W.decode_batched(device=gpu, seed=batch + d, batch=batch, ctx_lo=ctx_lo, ctx_hi=ctx_hi,
                         hq=hq, hkv=hkv, d=d, with_write=True)
    kc, vc = w.k_cache.clone(), w.v_cache.clone()
    want = _write_then_decode(w, gpu, w.slot_mapping, kc, vc)
    meta = w.device_meta(gpu)
    got = decode_attention_write_kv(w.q, w.k_new, w.v_new, w.k_cache, w.v_cache,
                                    meta["block_table"], meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(w.k_cache, kc) and torch.equal(w.v_cache, vc)
    assert torch.equal(got, want)
    assert_attn_close(f32(got), oracle_decode(w), "fused write+decode vs oracle")


def test_fused_kv_write_skips_rows_without_a_slot(gpu):
    """Rows with ctx 0, ctx past the table row, a hole at the last position or a slot past
    max_slots write nothing; the rest write. Also the separate-launch path (k_new only
    2-byte aligned) and the row copies of a q view that is only 2-byte aligned."""
    from ccinfer_amd import decode_attention_write_kv
    say("fused write+decode edge rows")
    w = W.decode_batched(device=gpu, seed=31, batch=8, ctx_lo=40, ctx_hi=300, with_write=True)
    ctx = w.context_lens.copy()
    bt = w.block_table.copy()
    ctx[0] = 0
    ctx[1] = bt.shape[1] * 16 + 1
    bt[2, (ctx[2] - 1) // 16] = -1
    w.context_lens, w.block_table = ctx.astype(np.int32), bt
    max_slots = int(w.k_cache.shape[0])
    pos = np.maximum(ctx - 1, 0)
    slots = (bt[np.arange(8), np.minimum(pos // 16, bt.shape[1] - 1)] * 16 + pos % 16)
    slots = slots.astype(np.int64)
    slots[[0, 1, 2]] = -1
    limit = int(slots[3])          # row 3's slot (and any above it) is past max_slots
    slots[slots >= limit] = -1
    assert limit < max_slots and (slots >= 0).sum() >= 2
    for variant in ("fused", "split_write", "staged_q"):
        w2 = W.decode_batched(device=gpu, seed=31, batch=8, ctx_lo=40, ctx_hi=300,
                              with_write=True)
        w2.context_lens, w2.block_table = w.context_lens, w.block_table
        kc, vc = w2.k_cache.clone(), w2.v_cache.clone()
        want = _write_then_decode(w2, gpu, slots, kc, vc)
        meta = w2.device_meta(gpu)
        q, k_new, v_new = w2.q, w2.k_new, w2.v_new
        if variant == "split_write":
            k_new = _offset_view(k_new)
            v_new = _offset_view(v_new)
        if variant == "staged_q":
            q = _offset_view(q)
        got = decode_attention_write_kv(q, k_new, v_new, w2.k_cache, w2.v_cache,
                                        meta["block_table"], meta["context_lens"],
                                        max_slots=limit)
        torch.cuda.synchronize()
        assert torch.equal(w2.k_cache, kc) and torch.equal(w2.v_cache, vc), variant
        assert torch.equal(got, want), variant



def _poison_unread_slots(w, gpu):
    """NaN K / Inf V in every cache slot no request of w reads (rows with an invalid
    context read nothing)."""
    used = np.zeros(w.num_blocks * 16, bool)
    for b in range(w.batch):
        n = int(w.context_lens[b])
        if n <= 0 or (n + 15) // 16 > w.mbpr:
            continue
        pos = np.arange(n)
        blk = w.block_table[b, pos // 16]
        ok = blk >= 0
        used[blk[ok] * 16 + pos[ok] % 16] = True
    rows = torch.from_numpy(np.nonzero(~used)[0]).to(gpu)
    w.k_cache[rows] = float("nan")
    w.v_cache[rows] = float("inf")


def _invalidate_and_hole(w, seed, step):
    """Rows 3 (context 0) and 7 (longer than the table row) become invalid; every
    step-th row from 10 loses one block that is not its last."""
    rng = np.random.default_rng(seed)
    ctx = w.context_lens.copy()
    bt = w.block_table.copy()
    ctx[3] = 0
    ctx[7] = w.mbpr * 16 + 17
    for b in range(10, w.batch, step):
        nb = int(np.count_nonzero(bt[b] >= 0))
        if nb > 2:
            bt[b, int(rng.integers(0, nb - 1))] = -1
    w.context_lens = ctx
    w.block_table = bt


@pytest.mark.parametrize("batch,lo,hi,hq,hkv,seed", [
    (300, 100, 3000, 32, 8, 61),     # index, equal ranges
    (257, 4000, 4096, 32, 8, 63),    # index, equal ranges, long rows
    (1000, 1, 700, 32, 8, 62),       # index, snapped ranges (8000 wavefronts)
    (600, 100, 3000, 32, 8, 64),     # snapped, rows from under T to several T
    (200, 100, 3000, 32, 32, 65),    # snapped below the index's request limit
])
def test_flat_plan_index_for_large_batches(gpu, batch, lo, hi, hq, hkv, seed):
    """The flat plan's index kernel (more than 256 requests, or launches of many rounds of
    wavefronts, whose range starts snap to request boundaries): it writes the chunk and split
    prefixes and the range starts, and each wavefront walks its segments from them. Holes in
    the table, invalid contexts (0, longer than the table row) and every unused cache slot
    poisoned (NaN K, Inf V); every row against the oracle, and the fused KV write bit-equal
    to write + decode."""
    from ccinfer_amd import decode_attention_write_kv
    say(f"flat plan index: B={batch} ctx=[{lo},{hi}] hq={hq} hkv={hkv}")
    w = W.decode_batched(device=gpu, seed=seed, batch=batch, ctx_lo=lo, ctx_hi=hi, hq=hq,
                         hkv=hkv, with_write=True)
    _invalidate_and_hole(w, seed, 37)
    w.slot_mapping = w.slot_mapping.copy()
    w.slot_mapping[[3, 7]] = -1                  # invalid rows have no new-token slot
    meta = w.device_meta(gpu)
    kc, vc = w.k_cache.clone(), w.v_cache.clone()
    write_kv_cache(w.k_new, w.v_new, kc, vc, meta["slot_mapping"])
    want = decode_attention(w.q, kc, vc, meta["block_table"], meta["context_lens"])
    got = decode_attention_write_kv(w.q, w.k_new, w.v_new, w.k_cache, w.v_cache,
                                    meta["block_table"], meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(w.k_cache, kc) and torch.equal(w.v_cache, vc)
    _poison_unread_slots(w, gpu)
    out = run_decode(w, gpu)
    res = f32(out)
    assert np.all(res[3] == 0) and np.all(res[7] == 0)
    assert_attn_close(res, oracle_decode(w), f"B={batch}")


def test_flat_plan_snapped_fp8(gpu):
    """fp8 cache through the snapped index (600 requests, 4800 wavefronts), unused slots
    holding the E4M3 NaN code, against the oracle's fp8 decode."""
    from ccinfer_amd import decode_attention_fp8
    from tests.test_gpu_fp8 import quantised_cache
    from tests.test_gpu_random_shapes import _unused_rows
    say("flat plan snapped fp8: B=600 ctx=[100,3000]")
    w = W.decode_batched(device=gpu, seed=66, batch=600, ctx_lo=100, ctx_hi=3000,
                         with_write=False)
    kc, vc, ks, vs = quantised_cache(gpu, w, w.hkv, w.d)
    rows = _unused_rows(w, gpu)
    kc[rows] = 0x7F
    vc[rows] = 0x7F
    meta = w.device_meta(gpu)
    got = decode_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"], meta["context_lens"])
    torch.cuda.synchronize()
    ref = oracle.decode_fp8(u16(w.q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                            vs.cpu().numpy(), w.block_table, w.context_lens)
    assert_attn_close(f32(got), ref, "fp8 B=600")


@pytest.mark.parametrize("batch,lo,hi,hq,hkv,seed", [
    (2048, 100, 1000, 8, 8, 67),     # one range per request
    (2500, 2100, 2200, 4, 2, 68),    # requests of 66-69 chunks: two pieces each
])
def test_flat_plan_whole_rows(gpu, batch, lo, hi, hq, hkv, seed):
    """Launches whose longest request is short next to one resident wavefront's share: the
    index kernel gives each request its own ranges (pieces of at most 64 chunks) instead of
    equal ranges across requests. Every output finite and a sample of rows against the
    oracle, with invalid rows, table holes and every unread slot poisoned."""
    say(f"flat plan whole rows: B={batch} ctx=[{lo},{hi}] hq={hq} hkv={hkv}")
    w = W.decode_batched(device=gpu, seed=seed, batch=batch, ctx_lo=lo, ctx_hi=hi, hq=hq,
                         hkv=hkv, with_write=False)
    _invalidate_and_hole(w, seed, 29)
    _poison_unread_slots(w, gpu)
    res = f32(run_decode(w, gpu))
    assert np.all(np.isfinite(res))
    assert np.all(res[3] == 0) and np.all(res[7] == 0)
    rows = np.r_[0:64, 64:batch:23, batch - 5:batch]
    ref = oracle.decode(u16(w.q)[rows], u16(w.k_cache), u16(w.v_cache), w.block_table[rows],
                        w.context_lens[rows])
    assert_attn_close(res[rows], ref, f"B={batch}")


@pytest.mark.parametrize("batch,hkv", [(300, 8), (700, 8)])
def test_flat_plan_index_with_no_or_one_valid_row(gpu, batch, hkv):
    """The index kernel when the batch holds no chunks at all (every context 0 or too long
    for the table row: zeros everywhere), and when a single row holds them all."""
    say(f"flat plan index, degenerate batches: B={batch}")
    w = W.decode_batched(device=gpu, seed=69, batch=batch, ctx_lo=100, ctx_hi=3000,
                         hkv=hkv, with_write=False)
    full = w.context_lens.copy()
    ctx = np.zeros_like(full)
    ctx[1::2] = w.mbpr * 16 + 1                  # longer than the table row
    w.context_lens = ctx
    out = f32(run_decode(w, gpu))
    assert np.all(out == 0)
    ctx = np.zeros_like(full)
    ctx[batch // 2] = full[batch // 2]
    w.context_lens = ctx
    out = f32(run_decode(w, gpu))
    assert np.all(np.delete(out, batch // 2, axis=0) == 0)
    ref = oracle_decode(w)
    assert_attn_close(out, ref, "one valid row")
