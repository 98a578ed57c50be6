"""Pins the fp8 KV-cache functions of the oracle (OCP E4M3 bytes, one fp32 scale per cache
row). The reference has no fp8 cache, so there is no reference vector: the checks are an
independent library routine (torch.float8_e4m3fn) and closed forms.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

BS = 16


def test_e4m3_codes_match_torch_on_every_code():
    codes = np.arange(256, dtype=np.uint8)
    ours = oracle.e4m3_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan) and nan.sum() == 2  # 0x7f, 0xff
    np.testing.assert_array_equal(ours[~nan], ref[~nan])


def test_e4m3_rounding_matches_torch_on_all_bf16_values_in_range():
    bits = np.arange(65536, dtype=np.uint32) << 16
    x = bits.view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) <= 448)]
    ours = oracle.f32_to_e4m3(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, ref)


def test_e4m3_known_values_and_saturation():
    assert [int(v) for v in oracle.f32_to_e4m3([1.0, 448.0, -2.0, 2.0 ** -9, 0.0, -0.0])] == \
        [0x38, 0x7E, 0xC0, 0x01, 0x00, 0x80]
    # ties to even: 232 lies halfway between 224 (0x76) and 240 (0x77)
    assert int(oracle.f32_to_e4m3([232.0])[0]) == 0x76
    # beyond the largest finite value: saturates to +-448, never the NaN code
    assert [int(v) for v in oracle.f32_to_e4m3([1e6, -470.0])] == [0x7E, 0xFE]


def rnd_bf16(rng, shape, scale=1.0):
    return oracle.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def dequant(cache, scales, hkv):
    """Float value of every cache row: torch's E4M3 decoding times the row scale."""
    slots = cache.shape[0]
    vals = torch.from_numpy(cache.reshape(-1)).view(torch.float8_e4m3fn).float().numpy()
    vals = vals.reshape(cache.shape)
    idx = oracle.fp8_scale_index(np.arange(slots)[:, None], np.arange(hkv)[None, :], hkv)
    return vals * scales[idx][..., None]


def test_write_quantises_each_row_within_half_an_e4m3_step():
    rng = np.random.default_rng(1)
    t, hkv, d, slots = 20, 4, 128, 64
    k = rnd_bf16(rng, (t, hkv, d), 3.0)
    v = rnd_bf16(rng, (t, hkv, d), 0.01)
    k[3, 1] = 0  # an all-zero row
    sm = rng.permutation(slots)[:t].astype(np.int32)
    sm[5] = -1
    kc = np.full((slots, hkv, d), 0xAB, np.uint8)
    vc = kc.copy()
    ks = np.full(slots * hkv, -1.0, np.float32)
    vs = ks.copy()
    oracle.write_kv_cache_fp8(k, v, kc, vc, ks, vs, sm)
    kd, vd = dequant(kc, ks, hkv), dequant(vc, vs, hkv)
    for src, deq, sc in ((k, kd, ks), (v, vd, vs)):
        x = oracle.bf16_to_f32(src)
        for i in range(t):
            if sm[i] < 0:
                continue
            for h in range(hkv):
                row = x[i, h]
                amax = np.abs(row).max()
                s = sc[oracle.fp8_scale_index(sm[i], h, hkv)]
                if amax == 0:
                    assert s == 0 and np.all(deq[sm[i], h] == 0)
                    continue
                # the smallest power of two with amax <= 448 s
                assert s == 2.0 ** np.ceil(np.log2(np.float64(amax) / 448.0))
                assert amax <= 448 * s and amax > 224 * s
                # E4M3 spacing at |q| is 2^(floor(log2|q|) - 3) (2^-9 below 2^-6): the error
                # is at most half a step, times the scale
                q = np.abs(row) / s
                step = np.where(q < 2 ** -6, 2.0 ** -9, 2.0 ** (np.floor(np.log2(np.maximum(
                    q, 2 ** -6))) - 3))
                assert np.all(np.abs(deq[sm[i], h] - row) <= 0.5 * step * s * (1 + 1e-5) + 1e-30)
                assert np.max(np.abs(deq[sm[i], h])) == pytest.approx(amax, rel=2.0 ** -4)
    # skipped slot and untouched slots keep their bytes
    written = set(sm[sm >= 0].tolist())
    for sl in range(slots):
        if sl not in written:
            assert np.all(kc[sl] == 0xAB) and np.all(vc[sl] == 0xAB)


def test_scale_layout_groups_a_blocks_rows():
    # the 16 rows of block b for head h are scales [(b * Hkv + h) * 16, +16)
    hkv = 3
    idx = oracle.fp8_scale_index(np.arange(64), 2, hkv)
    assert list(idx[16:32]) == list(range((1 * hkv + 2) * 16, (1 * hkv + 2) * 16 + 16))


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8)])
def test_fp8_decode_equals_float64_attention_over_the_dequantised_cache(hq, hkv):
    rng = np.random.default_rng(hq)
    b, d, nblk = 3, 128, 40
    slots = nblk * BS
    ctx = np.array([1, 200, 523], np.int32)
    kc = rng.integers(0, 256, (slots, hkv, d)).astype(np.uint8)
    kc[(kc & 0x7F) == 0x7F] = 0x10  # no NaN codes
    vc = rng.integers(0, 256, (slots, hkv, d)).astype(np.uint8)
    vc[(vc & 0x7F) == 0x7F] = 0x22
    ks = rng.uniform(1e-3, 1e-2, slots * hkv).astype(np.float32)
    vs = rng.uniform(1e-3, 1e-2, slots * hkv).astype(np.float32)
    bt = np.full((b, 34), -1, np.int32)
    perm = rng.permutation(nblk)
    bt[0, 0] = perm[0]
    bt[1, :13] = perm[1:14]
    bt[2, :33] = perm[7:40]
    q = rnd_bf16(rng, (b, hq, d))
    got = oracle.decode_fp8(q, kc, vc, ks, vs, bt, ctx)
    kd, vd = dequant(kc, ks, hkv), dequant(vc, vs, hkv)
    g = hq // hkv
    for i in range(b):
        pos = np.arange(ctx[i])
        rows = bt[i, pos // BS] * BS + pos % BS
        for h in range(hq):
            qv = torch.from_numpy(oracle.bf16_to_f32(q[i, h]).astype(np.float64))[None, None]
            kk = torch.from_numpy(kd[rows, h // g].astype(np.float64))[None]
            vv = torch.from_numpy(vd[rows, h // g].astype(np.float64))[None]
            ref = F.scaled_dot_product_attention(qv, kk, vv)[0, 0].numpy()
            np.testing.assert_allclose(got[i, h], ref, rtol=2e-5, atol=2e-6)


def test_fp8_prefill_equals_bf16_prefill_on_an_exact_image():
    # fp8 bytes with scale 1/4 and a bf16 cache holding exactly their values: the two oracles
    # run the same float operations, so the outputs agree bit for bit
    rng = np.random.default_rng(21)
    hq, hkv, d, nblk = 8, 2, 64, 12
    slots = nblk * BS
    codes = rng.integers(0, 256, (slots, hkv, d)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x30
    kc8, vc8 = codes, np.roll(codes, 7)
    kb = oracle.f32_to_bf16(oracle.e4m3_to_f32(kc8) * np.float32(0.25))
    vb = oracle.f32_to_bf16(oracle.e4m3_to_f32(vc8) * np.float32(0.25))
    qsl = np.array([0, 20, 21, 40], np.int32)
    ctx = np.array([36, 60, 19], np.int32)
    bt = np.array([[0, 3, 5, 7], [1, 2, 4, 6], [8, 9, -1, -1]], np.int32)
    q = rnd_bf16(rng, (40, hq, d))
    quarter = np.full(slots * hkv, 0.25, np.float32)
    got = oracle.prefill_fp8(q, kc8, vc8, quarter, quarter, bt, qsl, ctx)
    want = oracle.prefill(q, kb, vb, bt, qsl, ctx)
    np.testing.assert_array_equal(got, want)


def test_fp8_prefill_equals_float64_causal_attention():
    rng = np.random.default_rng(22)
    hq, hkv, d, nblk = 4, 2, 128, 10
    slots = nblk * BS
    kc = rng.integers(0, 256, (slots, hkv, d)).astype(np.uint8)
    kc[(kc & 0x7F) == 0x7F] = 0x11
    vc = rng.integers(0, 256, (slots, hkv, d)).astype(np.uint8)
    vc[(vc & 0x7F) == 0x7F] = 0x23
    ks = rng.uniform(1e-3, 1e-2, slots * hkv).astype(np.float32)
    vs = rng.uniform(1e-3, 1e-2, slots * hkv).astype(np.float32)
    prefix, qlen = 40, 30
    bt = rng.permutation(nblk)[:5].astype(np.int32)[None]
    qsl = np.array([0, qlen], np.int32)
    ctx = np.array([prefix + qlen], np.int32)
    q = rnd_bf16(rng, (qlen, hq, d))
    got = oracle.prefill_fp8(q, kc, vc, ks, vs, bt, qsl, ctx)
    kd, vd = dequant(kc, ks, hkv), dequant(vc, vs, hkv)
    pos = np.arange(prefix + qlen)
    rows = bt[0, pos // BS] * BS + pos % BS
    for h in range(hq):
        qq = torch.from_numpy(oracle.bf16_to_f32(q[:, h]).astype(np.float64))[None]
        kk = torch.from_numpy(kd[rows, h // (hq // hkv)].astype(np.float64))[None]
        vv = torch.from_numpy(vd[rows, h // (hq // hkv)].astype(np.float64))[None]
        mask = pos[None, :] <= prefix + np.arange(qlen)[:, None]
        ref = F.scaled_dot_product_attention(qq, kk, vv,
                                             attn_mask=torch.from_numpy(mask)[None])[0].numpy()
        np.testing.assert_allclose(got[:, h], ref, rtol=2e-5, atol=2e-6)


def test_row_scale_boundaries():
    # amax exactly 448 * 2^k keeps scale 2^k; just above doubles it; tiny rows stop at 2^-126
    rows = [(448.0, 1.0), (450.0, 2.0), (224.0, 0.5), (1.0, 2.0 ** -8), (7.0, 2.0 ** -6),
            (2e-38, 2.0 ** -126), (3.0e38, 2.0 ** 120)]
    hkv, d = 1, 4
    for amax, want in rows:
        x = np.zeros((1, hkv, d), np.float32)
        x[0, 0, 1] = -amax
        k = oracle.f32_to_bf16(x)
        amax_b = float(np.abs(oracle.bf16_to_f32(k)).max())
        kc = np.zeros((16, hkv, d), np.uint8)
        ks = np.zeros(16 * hkv, np.float32)
        oracle.write_kv_cache_fp8(k, k, kc, kc.copy(), ks, ks.copy(), np.array([0], np.int32))
        assert ks[0] == want, (amax, ks[0])
        sc = float(ks[0])
        assert amax_b <= 448 * sc and (amax_b > 224 * sc or sc == 2.0 ** -126)


def test_row_with_an_infinity():
    # scale 2^126: the infinities store as +-448 (codes 0x7e / 0xfe) and dequantise to +-inf
    # in bf16 (448 * 2^126 is past bf16's largest finite value); finite elements store as 0
    hkv, d = 1, 4
    x = np.array([[[np.inf, 3.0, -np.inf, -2.0]]], np.float32)
    k = oracle.f32_to_bf16(x)
    kc = np.full((16, hkv, d), 0x55, np.uint8)
    ks = np.zeros(16 * hkv, np.float32)
    oracle.write_kv_cache_fp8(k, k, kc, kc.copy(), ks, ks.copy(), np.array([0], np.int32))
    assert ks[0] == 2.0 ** 126
    assert kc[0, 0].tolist() == [0x7E, 0x00, 0xFE, 0x80]
    assert 448.0 * float(ks[0]) > 3.3961e38  # beyond bf16's largest finite value
