"""Fused decode prologue on the GPU (split QKV + q/k RMSNorm + RoPE + KV-cache write in one
launch) against the CPU oracle, which restates the reference's five kernels in sequence
(src/model/qwen3/qwen3_model.cpp:174-244).

Bar: q and K within one bf16 ulp of the oracle (a float32 result may sit on the other side
of a rounding boundary), widened by 2^-20 of the row's magnitude for RoPE cancellation;
V bit-exact (a copy); cache rows of skipped tokens and untouched slots bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import CcinferError, qkv_prologue
from tests._util import from_u16, say, u16

pytestmark = pytest.mark.gpu


def assert_within_one_ulp(got, want, what):
    """got/want uint16 bf16 patterns of [..., head_dim] rows: each value within one bf16 ulp
    of the oracle's, plus 2^-20 of the row's largest magnitude. The second term covers RoPE
    outputs that cancel (x0 c - x1 s with x0 c close to x1 s): there a float32 rounding of
    one product (fused multiply-add on the GPU, separate roundings in the oracle) moves the
    small result by up to 2^-23 of the products, which the output ulp does not bound."""
    g = oracle.bf16_to_f32(got).astype(np.float64)
    w = oracle.bf16_to_f32(want).astype(np.float64)
    row_max = np.abs(w).max(-1, keepdims=True)
    e = np.floor(np.log2(np.maximum(np.abs(w), 2.0 ** -126)))
    bound = 2.0 ** (e - 7) + 2.0 ** -20 * row_max
    bad = np.flatnonzero(np.abs(g - w) > bound)
    assert bad.size == 0, (f"{what}: {bad.size} values out of bound, first {bad[:5]}: "
                           f"got {g.ravel()[bad[:3]]} want {w.ravel()[bad[:3]]}")
    return float(np.mean(got != want))


def _run(gpu, seed, t, nq, nkv, hd, slots, with_norm=True, max_pos=4096, eps=1e-6,
         theta=1e6, scale=1.5):
    say(f"prologue seed={seed} T={t} nq={nq} nkv={nkv} hd={hd} norm={with_norm}")
    rng = np.random.default_rng(seed)
    qkv = oracle.f32_to_bf16((rng.standard_normal((t, (nq + 2 * nkv) * hd)) * scale)
                             .astype(np.float32))
    qw = oracle.f32_to_bf16(rng.standard_normal(hd).astype(np.float32)) if with_norm else None
    kw = oracle.f32_to_bf16(rng.standard_normal(hd).astype(np.float32)) if with_norm else None
    pos = rng.integers(0, max_pos, t).astype(np.int32)
    sm = rng.permutation(slots)[:t].astype(np.int32)
    if t >= 4:
        pos[0], pos[1] = -1, max_pos            # rotation skipped
        sm[2], sm[3] = -1, slots + 7            # no K/V write
    cache = oracle.rope_cache_table(max_pos, hd, theta)
    kc0 = oracle.lcg_fill(slots * nkv * hd, seed + 1).reshape(slots, nkv, hd)
    vc0 = oracle.lcg_fill(slots * nkv * hd, seed + 2).reshape(slots, nkv, hd)

    want_k, want_v = kc0.copy(), vc0.copy()
    want_q = oracle.qkv_prologue(qkv, qw, kw, pos, cache, sm, want_k, want_v, nq, nkv, hd, eps)

    kc, vc = from_u16(kc0, gpu), from_u16(vc0, gpu)
    dev = lambda a: None if a is None else from_u16(a, gpu)  # noqa: E731
    q = qkv_prologue(from_u16(qkv, gpu), dev(qw), dev(kw),
                     torch.from_numpy(pos).to(gpu), torch.from_numpy(cache).to(gpu),
                     torch.from_numpy(sm).to(gpu), kc, vc, nq, eps)
    torch.cuda.synchronize()
    diff_q = assert_within_one_ulp(u16(q), want_q, "q")
    diff_k = assert_within_one_ulp(u16(kc), want_k, "k_cache")
    assert np.array_equal(u16(vc), want_v), "v_cache"
    # slots no token wrote keep their contents exactly
    written = np.zeros(slots, bool)
    written[sm[(sm >= 0) & (sm < slots)]] = True
    assert np.array_equal(u16(kc)[~written], kc0[~written])
    return diff_q, diff_k


@pytest.mark.parametrize("t,nq,nkv", [(1, 32, 8), (7, 32, 8), (64, 32, 8), (256, 32, 8),
                                      (33, 64, 8), (5, 16, 2)])
def test_head_dim_128_fast_path(gpu, t, nq, nkv):
    dq, dk = _run(gpu, 100 + t, t, nq, nkv, 128, slots=max(2 * t, 16))
    # one-ulp differences are rare: they need a value within float32 noise of a tie
    assert dq < 0.01 and dk < 0.01


@pytest.mark.parametrize("t,nq,nkv", [(3000, 32, 8), (8000, 14, 2)])
def test_large_launch_eight_row_path(gpu, t, nq, nkv):
    # at least 131072 (token, head) rows selects eight rows per wavefront; 14 and 2 heads
    # leave partial groups in every section
    _run(gpu, 600 + nq, t, nq, nkv, 128, slots=2 * t)


@pytest.mark.parametrize("hd", [64, 96, 256, 2, 130])
def test_other_head_dims(gpu, hd):
    _run(gpu, 200 + hd, 9, 8, 2, hd, slots=32)


@pytest.mark.parametrize("hd", [128, 64])
def test_without_norm_weights(gpu, hd):
    _run(gpu, 300 + hd, 12, 16, 4, hd, slots=40, with_norm=False)


def test_large_activations(gpu):
    # large magnitudes: the sum of squares is far from 1 and the bf16 partial sums round a lot
    _run(gpu, 401, 16, 32, 8, 128, slots=64, scale=300.0)


def test_in_place_equivalent_to_reference_kat_shapes(gpu):
    # the reference RoPE test's GQA shape (tests/kernel/test_rope.cu:118-158) through the
    # fused path with no norm
    _run(gpu, 500, 2, 8, 2, 64, slots=8, with_norm=False, max_pos=32, theta=1e4)


def test_shape_errors_raise(gpu):
    say("prologue shape errors")
    qkv = torch.zeros((4, (8 + 4) * 128), dtype=torch.bfloat16, device=gpu)
    kc = torch.zeros((16, 2, 128), dtype=torch.bfloat16, device=gpu)
    pos = torch.zeros(4, dtype=torch.int32, device=gpu)
    cache = torch.zeros((8, 64, 2), dtype=torch.float32, device=gpu)
    with pytest.raises(CcinferError):
        qkv_prologue(qkv, None, None, pos[:3], cache, pos, kc, kc.clone(), 8)
    with pytest.raises(CcinferError):
        qkv_prologue(qkv, None, None, pos, cache, pos, kc, kc.clone(), 7)
    with pytest.raises(CcinferError):
        qkv_prologue(qkv, None, None, pos, cache, pos, kc, kc.clone(), 8, eps=0.0)
