"""Pins the CPU oracle (oracle/attn_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something it was not derived from:
  - known-answer vectors of the reference's own tests (write_kv_cache KAT,
    decode KAT inputs, the LCG of test_naive_attn.cu);
  - torch.nn.functional.scaled_dot_product_attention in float64 (an independent library
    routine) on K/V gathered with 4-D block indexing (a different formulation of the
    block-table address than the oracle's flat offset);
  - closed forms (uniform scores -> mean of V; bf16 rounding vs torch's converter);
  - identities between oracle functions (paged prefill == dense causal for prefix 0 and an
    identity table; prefill with one query token == decode).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

RTOL_LIB = 2e-5  # oracle (fp32 accumulation) vs float64 library routine


def rnd_bf16(rng, shape, scale=1.0):
    return oracle.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def f64(a):
    return torch.from_numpy(oracle.bf16_to_f32(a).astype(np.float64))


def gather_rows(cache, bt_row, ctx, block=16):
    """K/V rows of positions [0, ctx) via 4-D indexing [block, offset, head, dim]."""
    c4 = cache.reshape(-1, block, *cache.shape[1:])
    pos = np.arange(ctx)
    return c4[bt_row[pos // block], pos % block]


def sdpa_rows(q_rows, k_rows, v_rows, causal_offset=None):
    """float64 SDPA. q_rows [Tq, Hq, D], k/v [Tk, Hkv, D]; causal: query i sees keys
    <= causal_offset + i."""
    q = f64(q_rows).permute(1, 0, 2)
    k = f64(k_rows).permute(1, 0, 2)
    v = f64(v_rows).permute(1, 0, 2)
    mask = None
    if causal_offset is not None:
        tq, tk = q.shape[1], k.shape[1]
        mask = torch.ones(tq, tk, dtype=torch.bool).tril(diagonal=causal_offset)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True).permute(
        1, 0, 2).numpy()


# --------------------------------------------------------------------------- bf16

def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 200000),
        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.4028235e38, 1e-45, -1e-45, 1.00390625,
                  1.01171875, 0.2, 313.0, 613.0], np.float32),
        # exact ties between two bf16 values: round to even
        (np.arange(1, 4000, dtype=np.uint32) << 15 | 0x3f800000).view(np.float32),
    ]).astype(np.float32)
    got = oracle.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_roundtrip_all_patterns():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = oracle.bf16_to_f32(h)
    back = oracle.f32_to_bf16(f)
    finite_or_inf = ~np.isnan(f)
    assert np.array_equal(back[finite_or_inf], h[finite_or_inf])
    assert np.all(np.isnan(oracle.bf16_to_f32(back[~finite_or_inf])))


# --------------------------------------------------------------------------- addressing

def test_kv_base_offset_matches_4d_indexing():
    hkv, d, nb = 4, 32, 10
    cache = np.arange(nb * 16 * hkv * d, dtype=np.int64).reshape(nb * 16, hkv, d)
    row = np.array([7, 2, -1, 9, 0], np.int32)
    # Domain: ctx_pos >= 0 (every caller iterates positions from 0).
    for pos in range(0, 6 * 16 + 3):
        for h in range(hkv):
            off = oracle.kv_base_offset(pos, h, d, hkv, 16, row)
            lb = pos // 16
            if lb >= row.size or row[lb] < 0:
                assert off is None, (pos, h)
            else:
                want = cache.reshape(nb, 16, hkv, d)[row[lb], pos % 16, h, 0]
                assert off == want, (pos, h)


# --------------------------------------------------------------------------- write

def test_write_kv_cache_reference_kat():
    """tests/kernel/test_write_kv_cache.cu:15-98."""
    t, h, d = np.meshgrid(np.arange(4), np.arange(2), np.arange(4), indexing="ij")
    k = oracle.f32_to_bf16((t * 100 + h * 10 + d).astype(np.float32))
    v = oracle.f32_to_bf16((t * 200 + h * 10 + d).astype(np.float32))
    slots = np.array([5, 17, 0, 63], np.int32)
    kc = np.zeros((64, 2, 4), np.uint16)
    vc = np.zeros((64, 2, 4), np.uint16)
    oracle.write_kv_cache(k, v, kc, vc, slots)
    for i, s in enumerate(slots):
        assert np.array_equal(kc[s], k[i]) and np.array_equal(vc[s], v[i])
    assert np.all(kc[1] == 0) and np.all(vc[1] == 0)
    # small integers are exact in bf16; 313 and 613 round (to 312 and 612)
    assert oracle.bf16_to_f32(kc[63, 1, 3]) == 312.0
    assert oracle.bf16_to_f32(vc[63, 1, 3]) == 612.0


def test_write_kv_cache_skips_out_of_range_and_matches_scatter():
    rng = np.random.default_rng(2)
    k = rnd_bf16(rng, (7, 3, 8))
    v = rnd_bf16(rng, (7, 3, 8))
    slots = np.array([0, -1, 12, 40, 39, -100, 5], np.int32)
    kc = rnd_bf16(rng, (40, 3, 8))
    vc = rnd_bf16(rng, (40, 3, 8))
    want_k, want_v = kc.copy(), vc.copy()
    ok = (slots >= 0) & (slots < 40)
    want_k[slots[ok]] = k[ok]
    want_v[slots[ok]] = v[ok]
    oracle.write_kv_cache(k, v, kc, vc, slots)
    assert np.array_equal(kc, want_k) and np.array_equal(vc, want_v)


# --------------------------------------------------------------------------- decode

def decode_kat():
    b, hq, hkv, d = 2, 8, 2, 64
    qi = np.arange(b * hq * d)
    ki = np.arange(3 * 16 * hkv * d)
    q = oracle.f32_to_bf16((((qi * 17) % 23 - 11) * 0.03125).astype(np.float32)).reshape(b, hq, d)
    k = oracle.f32_to_bf16((((ki * 13) % 29 - 14) * 0.025).astype(np.float32)).reshape(48, hkv, d)
    v = oracle.f32_to_bf16((((ki * 7) % 31 - 15) * 0.02).astype(np.float32)).reshape(48, hkv, d)
    bt = np.array([[2, 0, 1], [1, 2, -1]], np.int32)
    ctx = np.array([31, 17], np.int32)
    return q, k, v, bt, ctx


def test_decode_kat_vs_float64_sdpa():
    """Inputs of RandomPagedGQAMatchesCpuReference (test_decode_attn.cu:229-311)."""
    q, k, v, bt, ctx = decode_kat()
    out = oracle.decode(q, k, v, bt, ctx)
    for b in range(2):
        want = sdpa_rows(q[b][None], gather_rows(k, bt[b], ctx[b]),
                         gather_rows(v, bt[b], ctx[b]))[0]
        np.testing.assert_allclose(out[b], want, atol=RTOL_LIB)


def test_decode_random_paged_vs_float64_sdpa():
    rng = np.random.default_rng(3)
    hq, hkv, d, pool = 16, 4, 128, 128
    ctx = np.array([1, 15, 16, 17, 200, 333], np.int32)
    bt = rng.permutation(pool)[:6 * 21].reshape(6, 21).astype(np.int32)
    q = rnd_bf16(rng, (6, hq, d))
    k = rnd_bf16(rng, (pool * 16, hkv, d))
    v = rnd_bf16(rng, (pool * 16, hkv, d))
    out = oracle.decode(q, k, v, bt, ctx)
    for b in range(6):
        want = sdpa_rows(q[b][None], gather_rows(k, bt[b], ctx[b]),
                         gather_rows(v, bt[b], ctx[b]))[0]
        np.testing.assert_allclose(out[b], want, atol=RTOL_LIB)


def test_decode_uniform_scores_give_mean_v():
    rng = np.random.default_rng(4)
    q = oracle.f32_to_bf16(np.full((1, 4, 64), 0.1, np.float32))
    k = oracle.f32_to_bf16(np.full((64, 2, 64), 0.1, np.float32))
    v = rnd_bf16(rng, (64, 2, 64))
    bt = np.array([[3, 1, 0, 2]], np.int32)
    out = oracle.decode(q, k, v, bt, np.array([50], np.int32))
    for hq in range(4):
        rows = gather_rows(v, bt[0], 50)[:, hq // 2]
        np.testing.assert_allclose(out[0, hq], oracle.bf16_to_f32(rows).mean(0), atol=1e-5)


def test_decode_edge_cases():
    """ctx <= 0 and more blocks than the row -> zeros; -1 blocks are skipped."""
    rng = np.random.default_rng(5)
    hq, hkv, d = 4, 2, 32
    q = rnd_bf16(rng, (4, hq, d))
    k = rnd_bf16(rng, (16 * 8, hkv, d))
    v = rnd_bf16(rng, (16 * 8, hkv, d))
    bt = np.array([[0, 1], [2, 3], [4, -1], [5, 6]], np.int32)
    ctx = np.array([0, 33, 32, -5], np.int32)
    out = oracle.decode(q, k, v, bt, ctx)
    assert np.all(out[0] == 0) and np.all(out[1] == 0) and np.all(out[3] == 0)
    want = sdpa_rows(q[2][None], gather_rows(k, np.array([4]), 16),
                     gather_rows(v, np.array([4]), 16))[0]
    np.testing.assert_allclose(out[2], want, atol=RTOL_LIB)


# --------------------------------------------------------------------------- prefill

def test_lcg_matches_known_rand_sequence():
    """The reference LCG (test_naive_attn.cu:67-74) is the C standard's example rand():
    seed 1 yields 16838, 5758, 10113, 17515, ... mapped to v/32768 - 1, times 0.5."""
    got = oracle.bf16_to_f32(oracle.lcg_fill(4, 1))
    want = [(r / 32768.0 - 1.0) * 0.5 for r in (16838, 5758, 10113, 17515)]
    want_bf = oracle.bf16_to_f32(oracle.f32_to_bf16(np.array(want, np.float32)))
    assert np.array_equal(got, want_bf)


def test_naive_vs_float64_sdpa():
    q = oracle.lcg_fill(4 * 4 * 8, 1).reshape(4, 4, 8)
    k = oracle.lcg_fill(4 * 2 * 8, 2).reshape(4, 2, 8)
    v = oracle.lcg_fill(4 * 2 * 8, 3).reshape(4, 2, 8)
    np.testing.assert_allclose(oracle.naive(q, k, v), sdpa_rows(q, k, v, causal_offset=0),
                               atol=RTOL_LIB)


def test_prefill_identity_table_equals_dense_causal():
    """The reference's own check (test_prefill_attn.cu:24-105): 32 tokens, 4/4 heads, D=64."""
    t, h, d = 32, 4, 64
    q = oracle.lcg_fill(t * h * d, 1).reshape(t, h, d)
    kc = oracle.lcg_fill(64 * h * d, 2).reshape(64, h, d)
    vc = oracle.lcg_fill(64 * h * d, 3).reshape(64, h, d)
    got = oracle.prefill(q, kc, vc, np.array([[0, 1]], np.int32), np.array([0, t], np.int32),
                         np.array([t], np.int32))
    np.testing.assert_allclose(got, oracle.naive(q, kc[:t], vc[:t]), atol=1e-6)


def test_prefill_prefix_causal_vs_float64_sdpa():
    rng = np.random.default_rng(6)
    hq, hkv, d, pool = 8, 2, 64, 40
    qlen = np.array([37, 1, 20], np.int32)
    pre = np.array([48, 90, 0], np.int32)
    ctx = qlen + pre
    qsl = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    bt = rng.permutation(pool)[:3 * 8].reshape(3, 8).astype(np.int32)
    q = rnd_bf16(rng, (int(qsl[-1]), hq, d))
    k = rnd_bf16(rng, (pool * 16, hkv, d))
    v = rnd_bf16(rng, (pool * 16, hkv, d))
    out = oracle.prefill(q, k, v, bt, qsl, ctx)
    for b in range(3):
        rows = slice(qsl[b], qsl[b + 1])
        want = sdpa_rows(q[rows], gather_rows(k, bt[b], ctx[b]), gather_rows(v, bt[b], ctx[b]),
                         causal_offset=int(pre[b]))
        np.testing.assert_allclose(out[rows], want, atol=RTOL_LIB)


def test_prefill_single_token_equals_decode():
    rng = np.random.default_rng(7)
    q = rnd_bf16(rng, (3, 8, 128))
    k = rnd_bf16(rng, (30 * 16, 4, 128))
    v = rnd_bf16(rng, (30 * 16, 4, 128))
    bt = rng.permutation(30)[:3 * 10].reshape(3, 10).astype(np.int32)
    ctx = np.array([5, 100, 160], np.int32)
    pre = oracle.prefill(q, k, v, bt, np.arange(4, dtype=np.int32), ctx)
    dec = oracle.decode(q, k, v, bt, ctx)
    np.testing.assert_allclose(pre, dec, rtol=1e-5, atol=1e-6)


def test_prefill_unwritten_rows_and_skips():
    """prefix < 0 rows untouched; -1 block skipped; positions past the row skipped."""
    rng = np.random.default_rng(8)
    hq, hkv, d = 4, 2, 32
    q = rnd_bf16(rng, (9, hq, d))
    k = rnd_bf16(rng, (8 * 16, hkv, d))
    v = rnd_bf16(rng, (8 * 16, hkv, d))
    qsl = np.array([0, 4, 9], np.int32)
    ctx = np.array([3, 40], np.int32)            # request 0: prefix -1 -> untouched
    bt = np.array([[0, 1], [2, -1]], np.int32)   # request 1 visible: block 2 only
    out = oracle.prefill(q, k, v, bt, qsl, ctx, out=np.full((9, hq, d), 5.0, np.float32))
    assert np.all(out[:4] == 5.0)
    for i in range(5):
        vis = 35 + i + 1
        keep = np.arange(vis) < 16   # positions 16..31 (block -1) and >= 32 (past row)
        kr = gather_rows(k, np.array([2, 0, 0]), vis)[keep]
        vr = gather_rows(v, np.array([2, 0, 0]), vis)[keep]
        want = sdpa_rows(q[4 + i][None], kr, vr)[0]
        np.testing.assert_allclose(out[4 + i], want, atol=RTOL_LIB)


def test_threads_do_not_change_results():
    rng = np.random.default_rng(9)
    q = rnd_bf16(rng, (5, 8, 64))
    k = rnd_bf16(rng, (20 * 16, 2, 64))
    v = rnd_bf16(rng, (20 * 16, 2, 64))
    bt = rng.permutation(20)[:15].reshape(5, 3).astype(np.int32)
    ctx = np.array([1, 20, 33, 48, 7], np.int32)
    a = oracle.decode(q, k, v, bt, ctx, nthreads=1)
    b = oracle.decode(q, k, v, bt, ctx, nthreads=7)
    assert np.array_equal(a, b)
    pairs = np.array([[1, 3], [4, 0]], np.int32)
    c = oracle.decode(q, k, v, bt, ctx, pairs=pairs)
    assert np.array_equal(c[1, 3], a[1, 3]) and np.array_equal(c[4, 0], a[4, 0])
    assert math.isfinite(float(np.abs(a).sum()))


@pytest.mark.parametrize("name", ["decode_kat", "write_kv_kat", "prefill_kat", "decode_small",
                                  "prefill_small", "mixed_small", "prologue_rope_kat",
                                  "prologue_small", "batch_meta_mixed", "fp8_write_small"])
def test_golden_fixtures_reproduce(name):
    """The committed fixtures (tests/golden/make_golden.py) match the current oracle."""
    from tests.golden import make_golden
    fx = np.load(make_golden.path(name))
    got = make_golden.compute(name, fx)
    for key, val in got.items():
        assert np.array_equal(val, fx[key]), (name, key)
