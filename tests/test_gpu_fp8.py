"""fp8 (OCP E4M3) KV cache on the GPU against the oracle: the write is bit-exact (bytes and
scales); decode over the fp8 cache meets the attention bar (max-abs <= 2e-2, mean-abs <=
2e-3) against the oracle's fp32 decode over the same fp8 cache."""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import (decode_attention, decode_attention_fp8, fp8_scale_numel,
                         write_kv_cache_fp8)
from ccinfer_amd import workloads as W
from tests._util import assert_attn_close, f32, from_u16, say, u16

pytestmark = pytest.mark.gpu
BS = 16


def bf(x):
    """One float as a bf16 bit pattern (numpy scalar)."""
    return oracle.f32_to_bf16(np.array([x], np.float32))[0]


def rnd_bf16(rng, shape, scale=1.0):
    return oracle.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("hkv,d", [(8, 128), (3, 64), (2, 256), (1, 130)])
def test_write_bit_exact(gpu, hkv, d):
    say(f"fp8 write hkv={hkv} d={d}")
    rng = np.random.default_rng(d + hkv)
    t, slots = 37, 96
    k = rnd_bf16(rng, (t, hkv, d), 2.0)
    v = rnd_bf16(rng, (t, hkv, d), 1e-3)
    k[4] = 0                                       # all-zero rows: scale 0
    v[6, 0, 1] = bf(1e30)                          # one huge element
    v[12, 0, 2] = bf(np.inf)                       # infinities: scale 2^126, code 448
    v[13, :, 0] = bf(-np.inf)
    # scale boundaries: amax exactly 448 (scale 1), just above (scale 2), tiny (2^-126)
    k[7] = bf(0.5)
    k[7, :, 3] = bf(448.0)
    k[8] = bf(-1.0)
    k[8, :, 5] = bf(-450.0)
    k[10] = bf(2e-38)
    sm = rng.permutation(slots)[:t].astype(np.int32)
    sm[2], sm[9] = -1, slots + 4                   # skipped
    nsc = fp8_scale_numel(slots, hkv)
    kc0 = rng.integers(0, 256, (slots, hkv, d)).astype(np.uint8)
    vc0 = rng.integers(0, 256, (slots, hkv, d)).astype(np.uint8)
    ks0 = rng.standard_normal(nsc).astype(np.float32)
    vs0 = rng.standard_normal(nsc).astype(np.float32)
    want = [a.copy() for a in (kc0, vc0, ks0, vs0)]
    oracle.write_kv_cache_fp8(k, v, *want, sm)
    dev = [torch.from_numpy(a.copy()).to(gpu) for a in (kc0, vc0, ks0, vs0)]
    write_kv_cache_fp8(from_u16(k, gpu), from_u16(v, gpu), *dev, torch.from_numpy(sm).to(gpu))
    torch.cuda.synchronize()
    for name, g, w in zip(("k_cache", "v_cache", "k_scale", "v_scale"), dev, want):
        got = g.cpu().numpy()
        if got.dtype == np.float32:
            assert np.array_equal(got.view(np.uint32), w.view(np.uint32)), name
        else:
            assert np.array_equal(got, w), name


def quantised_cache(gpu, w, hkv, d):
    """The workload's bf16 cache quantised into an fp8 cache by the GPU write kernel."""
    slots = w.k_cache.shape[0]
    kc = torch.empty((slots, hkv, d), dtype=torch.uint8, device=gpu)
    vc = torch.empty_like(kc)
    ks = torch.empty(fp8_scale_numel(slots, hkv), dtype=torch.float32, device=gpu)
    vs = torch.empty_like(ks)
    write_kv_cache_fp8(w.k_cache, w.v_cache, kc, vc, ks, vs,
                       torch.arange(slots, dtype=torch.int32, device=gpu))
    return kc, vc, ks, vs


@pytest.mark.parametrize("name,make", [
    ("decode_b1_ctx512", lambda dev: W.decode_single(device=dev)),
    ("decode_b64_ctx128-4096", lambda dev: W.decode_batched(device=dev)),
    ("decode_b3_gqa4_long", lambda dev: W.decode_batched(device=dev, batch=3, ctx_lo=9000,
                                                         ctx_hi=20000, hq=32, hkv=8)),
])
def test_decode_fp8_matches_oracle(gpu, name, make):
    say(f"fp8 decode {name}")
    w = make(gpu)
    meta = w.device_meta(gpu)
    kc, vc, ks, vs = quantised_cache(gpu, w, w.hkv, w.d)
    out = decode_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"], meta["context_lens"])
    ref_bf16 = decode_attention(w.q, w.k_cache, w.v_cache, meta["block_table"],
                                meta["context_lens"])
    torch.cuda.synchronize()
    want = oracle.decode_fp8(u16(w.q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                             vs.cpu().numpy(), w.block_table, w.context_lens)
    assert_attn_close(f32(out), want, f"fp8 {name}")
    # quantisation error against the bf16 cache stays small (informative bound)
    err = np.abs(f32(out) - f32(ref_bf16))
    assert err.max() < 0.1 and err.mean() < 0.01, (err.max(), err.mean())


def test_decode_fp8_masks_holes_and_bad_rows(gpu):
    say("fp8 decode holes")
    rng = np.random.default_rng(5)
    b, hq, hkv, d, nblk = 4, 16, 8, 128, 64
    slots = nblk * BS
    w = W.decode_batched(device=gpu, batch=b, ctx_lo=100, ctx_hi=900)
    kc, vc, ks, vs = quantised_cache(gpu, w, hkv, d)
    bt = w.block_table.copy()
    bt[1, 2] = -1                  # a hole
    ctx = w.context_lens.copy()
    ctx[3] = 0                     # invalid row -> zeros
    out = decode_attention_fp8(w.q, kc, vc, ks, vs, torch.from_numpy(bt).to(gpu),
                               torch.from_numpy(ctx).to(gpu))
    torch.cuda.synchronize()
    want = oracle.decode_fp8(u16(w.q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                             vs.cpu().numpy(), bt, ctx)
    assert_attn_close(f32(out), want, "fp8 holes")
    assert np.all(f32(out)[3] == 0)
    assert rng is not None and slots > 0


def _dequant_bf16(kc, ks, hkv):
    """bf16(byte * row scale) of every cache row, rounded as the fp8 prefill's LDS pass does
    (float32 product, then round to nearest even bf16)."""
    slots = kc.shape[0]
    vals = oracle.e4m3_to_f32(kc.reshape(-1)).reshape(kc.shape).astype(np.float32)
    idx = oracle.fp8_scale_index(np.arange(slots)[:, None], np.arange(hkv)[None, :], hkv)
    return oracle.f32_to_bf16((vals * ks[idx][..., None]).astype(np.float32))


@pytest.mark.parametrize("hq,hkv,d,n_seqs,prefix,new", [
    (16, 8, 128, 3, 64, 200), (16, 4, 128, 2, 48, 130), (8, 8, 64, 3, 16, 90),
    (32, 1, 128, 2, 32, 100),  # 32 query heads per KV head
])
def test_prefill_fp8_equals_bf16_prefill_of_its_dequantised_cache(gpu, hq, hkv, d, n_seqs,
                                                                    prefix, new):
    """After staging, the fp8 prefill runs the bf16 pipeline on bf16(byte * scale) tiles:
    its output is bit-identical to the bf16 prefill over a cache holding those values."""
    from ccinfer_amd import prefill_attention, prefill_attention_fp8
    say(f"fp8 prefill exact hq={hq} hkv={hkv} d={d}")
    w = W.prefill_prefix(device=gpu, seed=hq + d + new, n_seqs=n_seqs, prefix=prefix, new=new,
                         hq=hq, hkv=hkv, d=d)
    meta = w.device_meta(gpu)
    kc, vc, ks, vs = quantised_cache(gpu, w, hkv, d)
    out8 = prefill_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"],
                                 meta["query_start_loc"], meta["context_lens"])
    kb = from_u16(_dequant_bf16(kc.cpu().numpy(), ks.cpu().numpy(), hkv), gpu)
    vb = from_u16(_dequant_bf16(vc.cpu().numpy(), vs.cpu().numpy(), hkv), gpu)
    out16 = prefill_attention(w.q, kb, vb, meta["block_table"], meta["query_start_loc"],
                              meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(out8, out16)
    want = oracle.prefill_fp8(u16(w.q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                              vs.cpu().numpy(), w.block_table, w.query_start_loc, w.context_lens)
    assert_attn_close(f32(out8), want, "fp8 prefill vs oracle")


@pytest.mark.parametrize("dec_hi,prefix_hi", [(4096, 2048), (2000, 1024)])
def test_prefill_fp8_mixed_batch_with_side_stream_decode_items(gpu, dec_hi, prefix_hi):
    """Rows past 2048 positions: the decode items take the fp8 decode kernels on the side
    stream; rows within 2048: they run inside the tile launch. Either way the oracle's
    bar, the same bits with and without the side stream, and the fp8 decode operator's
    result on the decode rows."""
    from ccinfer_amd import prefill_attention_fp8
    say(f"fp8 prefill mixed batch, decode rows up to {dec_hi}")
    w = W.mixed_step(device=gpu, n_chunks=2, chunk=128, n_decode=40, dec_hi=dec_hi,
                     dec_lo=min(1024, dec_hi), prefix_hi=prefix_hi)
    meta = w.device_meta(gpu)
    kc, vc, ks, vs = quantised_cache(gpu, w, w.hkv, w.d)
    from ccinfer_amd import SideStream
    out = prefill_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"],
                                meta["query_start_loc"], meta["context_lens"],
                                overlap=SideStream(gpu))
    torch.cuda.synchronize()
    want = oracle.prefill_fp8(u16(w.q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                              vs.cpu().numpy(), w.block_table, w.query_start_loc, w.context_lens)
    assert_attn_close(f32(out), want, "fp8 mixed")
    serial = prefill_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"],
                                   meta["query_start_loc"], meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(out, serial)  # the side stream changes the schedule, not the bits
    # the decode items equal the fp8 decode operator on the same rows
    nc = 2
    rows = torch.from_numpy(w.query_start_loc[nc:-1].astype(np.int64)).to(gpu)
    dec = decode_attention_fp8(w.q[rows].contiguous(), kc, vc, ks, vs,
                               meta["block_table"][nc:].contiguous(),
                               meta["context_lens"][nc:].contiguous())
    assert_attn_close(f32(out)[w.query_start_loc[nc:-1]], f32(dec), "fp8 mixed decode items")


def test_prefill_fp8_config3_equals_bf16_prefill_of_dequantised_cache(gpu):
    """Full configs[2] size (8 x (512 + 1536), shared prefix): bit-identical to the bf16
    prefill over the dequantised cache, whose own full-size parity is tested against the
    oracle on sampled rows."""
    from ccinfer_amd import prefill_attention, prefill_attention_fp8
    say("fp8 prefill config3 size vs bf16 over the dequantised cache")
    w = W.prefill_prefix(device=gpu)
    meta = w.device_meta(gpu)
    kc, vc, ks, vs = quantised_cache(gpu, w, w.hkv, w.d)
    out8 = prefill_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"],
                                 meta["query_start_loc"], meta["context_lens"])
    kb = from_u16(_dequant_bf16(kc.cpu().numpy(), ks.cpu().numpy(), w.hkv), gpu)
    vb = from_u16(_dequant_bf16(vc.cpu().numpy(), vs.cpu().numpy(), w.hkv), gpu)
    out16 = prefill_attention(w.q, kb, vb, meta["block_table"], meta["query_start_loc"],
                              meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(out8, out16)
    assert bool(torch.isfinite(out8.float()).all())


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 64), (16, 8, 256), (12, 4, 64),
                                      (32, 1, 128), (48, 2, 64)])  # G=32, G=24
def test_decode_fp8_other_head_dims(gpu, hq, hkv, d):
    say(f"fp8 decode hq={hq} hkv={hkv} d={d}")
    w = W.decode_batched(device=gpu, batch=12, ctx_lo=20, ctx_hi=1500, hq=hq, hkv=hkv, d=d)
    meta = w.device_meta(gpu)
    kc, vc, ks, vs = quantised_cache(gpu, w, hkv, d)
    out = decode_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"], meta["context_lens"])
    torch.cuda.synchronize()
    want = oracle.decode_fp8(u16(w.q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                             vs.cpu().numpy(), w.block_table, w.context_lens)
    assert_attn_close(f32(out), want, f"fp8 d={d}")


def test_prefill_fp8_holes_ragged_and_untouched_rows(gpu):
    """Table holes, a context longer than the table row, ragged tile ends and a prefix < 0
    row (left untouched): staging writes zero bytes for the slots it does not load, so
    stale LDS contents never reach the output."""
    from ccinfer_amd import prefill_attention_fp8
    say("fp8 prefill edge cases")
    rng = np.random.default_rng(13)
    hq, hkv, d, mbpr, pool = 16, 8, 128, 16, 160
    qlen = np.array([2, 1, 3, 5, 130, 1, 64, 90], np.int32)
    ctx = np.array([40, 17, 3, 2, 200, 1, 300, 250], np.int32)  # seq 3: prefix < 0
    bt = rng.permutation(pool)[:len(qlen) * mbpr].reshape(len(qlen), mbpr).astype(np.int32)
    bt[4, 3] = -1            # hole inside a long prefill
    bt[6, 15] = -1           # hole in the last block
    bt[7, 10:] = -1          # table row shorter than the visible range
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    total = int(qsl[-1])
    g = torch.Generator(device=gpu)
    g.manual_seed(6)
    q = W.randn_bf16((total, hq, d), g, gpu)
    w = W.PagedWorkload("edge8", hq, hkv, d, ctx, bt, pool, q,
                        W.randn_bf16((pool * BS, hkv, d), g, gpu),
                        W.randn_bf16((pool * BS, hkv, d), g, gpu), query_start_loc=qsl)
    kc, vc, ks, vs = quantised_cache(gpu, w, hkv, d)
    meta = w.device_meta(gpu)
    out = torch.full_like(q, 7.0)
    prefill_attention_fp8(q, kc, vc, ks, vs, meta["block_table"], meta["query_start_loc"],
                          meta["context_lens"], output=out)
    torch.cuda.synchronize()
    got = f32(out)
    want = oracle.prefill_fp8(u16(q), kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                              vs.cpu().numpy(), bt, qsl, ctx,
                              out=np.full((total, hq, d), 7.0, np.float32))
    assert np.all(got[qsl[3]:qsl[4]] == 7.0)
    assert np.all(np.isfinite(got))
    assert_attn_close(got, want, "fp8 edge")


def test_prefill_fp8_any_scale_equals_bf16_prefill_of_dequantised_cache(gpu):
    """Scales that are not powers of two (a caller's own quantiser) take the general
    conversion (float product, rounded to bf16); power-of-two rows of the same tiles take the
    one-instruction conversion. Both must equal the bf16 prefill over bf16(byte * scale)."""
    from ccinfer_amd import prefill_attention, prefill_attention_fp8
    say("fp8 prefill with arbitrary scales")
    hq, hkv, d = 16, 8, 128
    w = W.prefill_prefix(device=gpu, seed=77, n_seqs=3, prefix=96, new=150, hq=hq, hkv=hkv,
                         d=d)
    meta = w.device_meta(gpu)
    kc, vc, ks, vs = quantised_cache(gpu, w, hkv, d)
    rng = np.random.default_rng(3)
    for s in (ks, vs):
        f = rng.uniform(0.6, 1.9, s.numel()).astype(np.float32)
        f[rng.random(s.numel()) < 0.5] = 1.0      # about half the rows keep a power of two
        s.mul_(torch.from_numpy(f).to(gpu))
    sc = ks.cpu().numpy().view(np.uint32)
    assert 0.2 < np.mean((sc & 0x7FFFFF) == 0) < 0.8
    out8 = prefill_attention_fp8(w.q, kc, vc, ks, vs, meta["block_table"],
                                 meta["query_start_loc"], meta["context_lens"])
    kb = from_u16(_dequant_bf16(kc.cpu().numpy(), ks.cpu().numpy(), hkv), gpu)
    vb = from_u16(_dequant_bf16(vc.cpu().numpy(), vs.cpu().numpy(), hkv), gpu)
    out16 = prefill_attention(w.q, kb, vb, meta["block_table"], meta["query_start_loc"],
                              meta["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(out8, out16)
