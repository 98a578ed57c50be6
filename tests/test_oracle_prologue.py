"""Pins the decode-side prologue functions of the CPU oracle (split QKV, RMSNorm, RoPE,
the fused prologue) before the HIP prologue is checked against them.

Checks, each independent of the oracle's own code:
  - the inputs and checks of the reference's kernel tests (tests/kernel/test_rms_norm.cu,
    tests/kernel/test_rope.cu), with their CPU loops and tolerances;
  - known answers that only the reference's reduction order produces (bf16 rounding of the
    per-thread partial sum after every addition);
  - closed forms: RoPE at angle 0 is the identity, at 90 degrees an exact swap with a sign;
    positions outside the table leave the row unchanged; numpy slicing for split_qkv;
  - float64 restatements within a stated number of bf16 ulps;
  - the fused prologue against the composition of the separately pinned functions.
"""
import numpy as np
import pytest

import oracle

bf = oracle.f32_to_bf16
fl = oracle.bf16_to_f32


def rnd_bf16(rng, shape, scale=1.0):
    return bf((rng.standard_normal(shape) * scale).astype(np.float32))


def ulp_bf16(x):
    """Spacing of bf16 numbers at |x| (x float array)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


# ---------------------------------------------------------------- split_qkv

@pytest.mark.parametrize("t,nq,nkv,hd", [(1, 1, 1, 8), (3, 8, 2, 64), (5, 16, 8, 128)])
def test_split_qkv_is_slicing(t, nq, nkv, hd):
    rng = np.random.default_rng(1)
    qkv = rnd_bf16(rng, (t, (nq + 2 * nkv) * hd))
    q, k, v = oracle.split_qkv(qkv, nq, nkv, hd)
    r = qkv.reshape(t, nq + 2 * nkv, hd)
    np.testing.assert_array_equal(q, r[:, :nq])
    np.testing.assert_array_equal(k, r[:, nq:nq + nkv])
    np.testing.assert_array_equal(v, r[:, nq + nkv:])


# ---------------------------------------------------------------- RMSNorm

def rms_norm_test_cpu(x, w, eps):
    """The CPU check of tests/kernel/test_rms_norm.cu:13-30 (float sums, one row at a time)."""
    xf, wf = fl(x).astype(np.float32), fl(w).astype(np.float32)
    out = np.empty(xf.shape, np.float32)
    for r in range(xf.shape[0]):
        s = np.float32(0)
        for v in xf[r]:
            s = np.float32(s + v * v)
        inv = np.float32(1) / np.sqrt(np.float32(s / np.float32(xf.shape[1]) + np.float32(eps)))
        out[r] = (xf[r] * inv) * wf
    return fl(bf(out))


def test_rms_norm_reference_single_row():
    x = bf(np.ones((1, 64), np.float32))
    w = bf(np.ones(64, np.float32))
    got = fl(oracle.rms_norm(x, w, 1e-5))
    np.testing.assert_allclose(got, rms_norm_test_cpu(x, w, 1e-5), atol=0.01)  # test_rms_norm.cu:69


def test_rms_norm_reference_multiple_rows():
    i = np.arange(4 * 128)
    x = bf((i % 7 - 3).astype(np.float32).reshape(4, 128))
    w = bf(((np.arange(128) % 5 + 1) / 3.0).astype(np.float32))
    got = fl(oracle.rms_norm(x, w, 1e-5))
    np.testing.assert_allclose(got, rms_norm_test_cpu(x, w, 1e-5), atol=0.02)  # :104


def test_rms_norm_rounds_partial_sums_to_bf16():
    # dim 2048: thread t of the 256-thread block sums pairs t, t+256, t+512, t+768. Pair t
    # holds (1, 0) and the other three (1/16, 0), so each partial is 1 + 3 * 2^-8; with bf16
    # rounding after every addition 1 + 2^-8 rounds (to even) back to 1, the total is 256
    # rather than 259, and 1 / sqrt(256/2048) = 2.8284 -> bf16 2.828125 (259 would give 2.8125).
    dim = 2048
    x = np.zeros((1, dim), np.float32)
    x[0, 0:512:2] = 1.0
    x[0, 512::2] = 1.0 / 16
    out = fl(oracle.rms_norm(bf(x), bf(np.ones(dim, np.float32)), 1e-30))
    assert out[0, 0] == 2.828125
    assert out[0, 1] == 0.0
    assert out[0, 512] == fl(bf(np.float32(2.828125 / 16)))


def test_rms_norm_odd_dim_scalar_path():
    # Odd dim: thread t sums elements t, t+256, ... one at a time. dim 257: thread 0 holds
    # x[0] = 1 and x[256] = 1/16, and 1 + 2^-8 rounds to 1; every other element is 0.
    dim = 257
    x = np.zeros((1, dim), np.float32)
    x[0, 0], x[0, 256] = 1.0, 1.0 / 16
    out = fl(oracle.rms_norm(bf(x), bf(np.ones(dim, np.float32)), 1e-6))
    inv = np.float32(1) / np.sqrt(np.float32(1) / np.float32(dim) + np.float32(1e-6))
    assert out[0, 0] == fl(bf(inv))[()]


@pytest.mark.parametrize("dim", [64, 128, 256, 1000])
def test_rms_norm_vs_float64(dim):
    rng = np.random.default_rng(dim)
    x = rnd_bf16(rng, (16, dim), 2.0)
    w = rnd_bf16(rng, (dim,))
    got = fl(oracle.rms_norm(x, w, 1e-6)).astype(np.float64)
    xd, wd = fl(x).astype(np.float64), fl(w).astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-6) * wd
    # bf16 partial sums perturb the total by a few 2^-8 relative: allow 3 % plus an ulp
    assert np.all(np.abs(got - ref) <= 0.03 * np.abs(ref) + ulp_bf16(ref))


# ---------------------------------------------------------------- RoPE

def rope_test_cpu(q, k, positions, cache, rotary_dim):
    """The CPU check of tests/kernel/test_rope.cu:30-54 (split-half pairs, float math)."""
    q, k = fl(q).copy(), fl(k).copy()
    half = rotary_dim // 2
    for x in (q, k):
        for t, pos in enumerate(positions):
            if pos < 0 or pos >= cache.shape[0]:
                continue
            for h in range(x.shape[1]):
                for p in range(half):
                    c, s = cache[pos, p]
                    x0, x1 = x[t, h, p], x[t, h, p + half]
                    x[t, h, p] = fl(bf(np.array([x0 * c - x1 * s], np.float32)))[0]
                    x[t, h, p + half] = fl(bf(np.array([x1 * c + x0 * s], np.float32)))[0]
    return q, k


def build_rope_cache_test(max_pos, rotary_dim, theta):
    """tests/kernel/test_rope.cu:15-27."""
    half = rotary_dim // 2
    c = np.empty((max_pos, half, 2), np.float32)
    for pos in range(max_pos):
        for pair in range(half):
            inv = np.float32(1) / np.power(np.float32(theta),
                                           np.float32(2 * pair) / np.float32(rotary_dim))
            ang = np.float32(pos) * inv
            c[pos, pair] = np.cos(ang), np.sin(ang)
    return c


def test_rope_reference_single_token_no_gqa():
    cache = build_rope_cache_test(16, 8, 10000.0)
    i = np.arange(2 * 8)
    q = bf((i % 5).astype(np.float32).reshape(1, 2, 8))
    k = bf(((i + 1) % 5).astype(np.float32).reshape(1, 2, 8))
    pos = np.array([3], np.int32)
    gq, gk = oracle.rope(q, k, pos, cache)
    eq, ek = rope_test_cpu(q, k, pos, cache, 8)
    np.testing.assert_allclose(fl(gq), eq, atol=0.02)  # test_rope.cu:111-112
    np.testing.assert_allclose(fl(gk), ek, atol=0.02)


def test_rope_reference_gqa():
    cache = build_rope_cache_test(32, 64, 10000.0)
    q = bf((np.arange(2 * 8 * 64) % 7 - 2).astype(np.float32).reshape(2, 8, 64))
    k = bf(((np.arange(2 * 2 * 64) + 3) % 9 - 3).astype(np.float32).reshape(2, 2, 64))
    pos = np.array([5, 17], np.int32)
    gq, gk = oracle.rope(q, k, pos, cache)
    eq, ek = rope_test_cpu(q, k, pos, cache, 64)
    np.testing.assert_allclose(fl(gq), eq, atol=0.02)  # test_rope.cu:154-156
    np.testing.assert_allclose(fl(gk), ek, atol=0.02)


def test_rope_cache_table_matches_reference_builder_and_float64():
    a = oracle.rope_cache_table(16, 32, 10000.0)
    assert a.shape == (16, 16, 2) and a.dtype == np.float32  # test_rope.cu:161-172
    np.testing.assert_allclose(a, build_rope_cache_test(16, 32, 10000.0), atol=2e-6)
    pos = np.arange(16)[:, None]
    ang = pos * 10000.0 ** (-(2.0 * np.arange(16)) / 32)
    np.testing.assert_allclose(a[..., 0], np.cos(ang), atol=1e-5)
    np.testing.assert_allclose(a[..., 1], np.sin(ang), atol=1e-5)


def test_rope_identity_quarter_turn_and_out_of_range():
    rng = np.random.default_rng(7)
    hd = 16
    q = rnd_bf16(rng, (4, 3, hd))
    k = rnd_bf16(rng, (4, 1, hd))
    cache = np.zeros((2, hd // 2, 2), np.float32)
    cache[0, :, 0] = 1.0                       # position 0: angle 0
    cache[1, :, 1] = 1.0                       # position 1: angle 90 degrees (cos 0, sin 1)
    pos = np.array([0, 1, -1, 2], np.int32)    # the last two are outside the table
    gq, gk = oracle.rope(q, k, pos, cache)
    h = hd // 2
    for x, g in ((q, gq), (k, gk)):
        np.testing.assert_array_equal(g[0], x[0])
        np.testing.assert_array_equal(fl(g[1, :, :h]), -fl(x[1, :, h:]))
        np.testing.assert_array_equal(g[1, :, h:], x[1, :, :h])
        np.testing.assert_array_equal(g[2:], x[2:])


def test_rope_vs_float64():
    rng = np.random.default_rng(3)
    hd, t = 128, 8
    q = rnd_bf16(rng, (t, 4, hd))
    k = rnd_bf16(rng, (t, 2, hd))
    cache = oracle.rope_cache_table(4096, hd, 1e6)
    pos = rng.integers(0, 4096, t).astype(np.int32)
    gq, _ = oracle.rope(q, k, pos, cache)
    x = fl(q).astype(np.float64)
    c = cache[pos][:, None, :, 0].astype(np.float64)
    s = cache[pos][:, None, :, 1].astype(np.float64)
    h = hd // 2
    ref = np.concatenate([x[..., :h] * c - x[..., h:] * s, x[..., h:] * c + x[..., :h] * s], -1)
    # float32 products round before the bf16 store: at most one bf16 ulp of the larger term
    bound = ulp_bf16(np.concatenate([np.abs(x[..., :h]) + np.abs(x[..., h:])] * 2, -1))
    assert np.all(np.abs(fl(gq) - ref) <= bound)


# ---------------------------------------------------------------- fused prologue

def _prologue_inputs(seed, t=6, nq=8, nkv=2, hd=64, slots=40, with_norm=True):
    rng = np.random.default_rng(seed)
    qkv = rnd_bf16(rng, (t, (nq + 2 * nkv) * hd), 1.5)
    qw = rnd_bf16(rng, (hd,)) if with_norm else None
    kw = rnd_bf16(rng, (hd,)) if with_norm else None
    pos = rng.integers(0, 100, t).astype(np.int32)
    pos[0] = -1                                            # rotation skipped
    sm = rng.permutation(slots)[:t].astype(np.int32)
    sm[1] = -1                                             # no K/V write
    sm[2] = slots + 3                                      # out of range: no K/V write
    cache = oracle.rope_cache_table(100, hd, 1e6)
    return qkv, qw, kw, pos, cache, sm


@pytest.mark.parametrize("with_norm", [True, False])
def test_qkv_prologue_is_the_reference_sequence(with_norm):
    nq, nkv, hd, slots, eps = 8, 2, 64, 40, 1e-6
    qkv, qw, kw, pos, cache, sm = _prologue_inputs(11, with_norm=with_norm)
    kc = oracle.lcg_fill(slots * nkv * hd, 5).reshape(slots, nkv, hd)
    vc = oracle.lcg_fill(slots * nkv * hd, 6).reshape(slots, nkv, hd)
    kc0, vc0 = kc.copy(), vc.copy()
    q_out = oracle.qkv_prologue(qkv, qw, kw, pos, cache, sm, kc, vc, nq, nkv, hd, eps)

    q, k, v = oracle.split_qkv(qkv, nq, nkv, hd)
    if with_norm:
        q, k = oracle.rms_norm(q, qw, eps), oracle.rms_norm(k, kw, eps)
    q, k = oracle.rope(q, k, pos, cache)
    np.testing.assert_array_equal(q_out, q)
    oracle.write_kv_cache(k, v, kc0, vc0, sm)
    np.testing.assert_array_equal(kc, kc0)
    np.testing.assert_array_equal(vc, vc0)
    # tokens 1 and 2 wrote nothing: exactly t - 2 slots changed
    changed = np.any(kc != oracle.lcg_fill(slots * nkv * hd, 5).reshape(slots, nkv, hd),
                     axis=(1, 2))
    assert changed.sum() == len(sm) - 2
