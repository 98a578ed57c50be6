"""Device-built batch metadata against the oracle: bit-exact for every array and the
status word (src/worker/batch_translator.cpp:213-302, src/model/model_runner.h:102-171)."""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import ITEM_DECODE, ITEM_SAMPLE, build_batch_metadata
from tests._util import say

pytestmark = pytest.mark.gpu
BS = 16


def batch(rng, b, decode_frac, max_ctx, max_new, extra_blocks=2, ncb=1 << 16):
    kvw = rng.integers(0, max_ctx, b).astype(np.int32)
    is_dec = rng.random(b) < decode_frac
    new = np.where(is_dec, 1, rng.integers(1, max_new + 1, b)).astype(np.int32)
    flags = np.where(is_dec, ITEM_DECODE,
                     np.where(rng.random(b) < 0.5, ITEM_SAMPLE, 0)).astype(np.int32)
    need = -(-(kvw.astype(np.int64) + new) // BS)
    counts = need + rng.integers(0, extra_blocks + 1, b)
    perm = rng.permutation(ncb).astype(np.int32)
    start = np.zeros(b + 1, np.int32)
    start[1:] = np.cumsum(counts)
    blocks = perm[:start[-1]] if start[-1] <= ncb else rng.integers(0, ncb, start[-1]).astype(
        np.int32)
    return kvw, new, flags, start, blocks, int(counts.max())


def check(gpu, kvw, new, flags, start, blocks, T, mbpr, ncb, out=None):
    want_st, want = oracle.build_batch_metadata(kvw, new, flags, start, blocks, T, mbpr, BS, ncb)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(gpu)  # noqa: E731
    got = build_batch_metadata(dev(kvw), dev(new), dev(flags), dev(start), dev(blocks), T, mbpr,
                               ncb, block_size=BS, out=out)
    torch.cuda.synchronize()
    assert int(got["status"].item()) == want_st
    # token entries past the batch's tokens (T larger than the sum: a failing batch) are
    # written by neither side
    written = min(T, int(np.maximum(new, 0).sum()))
    for k, v in want.items():
        g = got[k].cpu().numpy()
        if k in ("positions", "slot_mapping"):
            g, v = g[:written], v[:written]
        np.testing.assert_array_equal(g, v, err_msg=k)
    return got


@pytest.mark.parametrize("seed,b,decode_frac,max_ctx,max_new", [
    (1, 64, 1.0, 4096, 1),        # configs[1]-shaped decode batch
    (2, 8, 0.0, 512, 1536),       # configs[2]-shaped prefill with prefixes
    (3, 132, 0.97, 4096, 512),    # configs[3]-shaped mixed batch
    (4, 3000, 0.8, 2000, 64),     # more items than one scan pass (1024)
    (5, 1, 0.0, 1, 20),
])
def test_valid_batches_bit_exact(gpu, seed, b, decode_frac, max_ctx, max_new):
    say(f"batch_meta seed={seed} B={b}")
    rng = np.random.default_rng(seed)
    kvw, new, flags, start, blocks, mbpr = batch(rng, b, decode_frac, max_ctx, max_new)
    got = check(gpu, kvw, new, flags, start, blocks, int(new.sum()), mbpr + 3, 1 << 16)
    assert int(got["status"].item()) == 0


def test_invalid_batches_status_and_sanitised_entries(gpu):
    rng = np.random.default_rng(9)
    kvw, new, flags, start, blocks, mbpr = batch(rng, 40, 0.5, 1000, 40, ncb=4096)
    T = int(new.sum())
    cases = []
    n2 = new.copy(); n2[3] = 0; cases.append(("zero length", kvw, n2, flags, start, blocks, T - new[3], mbpr))  # noqa: E702,E501
    f2 = flags.copy(); n3 = new.copy(); f2[5] = ITEM_DECODE; n3[5] = 2; cases.append(("decode 2", kvw, n3, f2, start, blocks, int(n3.sum()), mbpr))  # noqa: E702,E501
    k2 = kvw.copy(); k2[7] = -3; cases.append(("negative kv_written", k2, new, flags, start, blocks, T, mbpr))  # noqa: E702,E501
    b2 = blocks.copy(); b2[11] = 4096; cases.append(("block past cache", kvw, new, flags, start, b2, T, mbpr))  # noqa: E702,E501
    b3 = blocks.copy(); b3[0] = -5; cases.append(("negative block", kvw, new, flags, start, b3, T, mbpr))  # noqa: E702,E501
    s2 = start.copy(); s2[9] = s2[10] + 1; cases.append(("backward range", kvw, new, flags, s2, blocks, T, mbpr))  # noqa: E702,E501
    cases.append(("T too small", kvw, new, flags, start, blocks, T - 5, mbpr))
    cases.append(("T too large", kvw, new, flags, start, blocks, T + 5, mbpr))
    cases.append(("table too narrow", kvw, new, flags, start, blocks, T, mbpr - 1))
    for what, *args in cases:
        say(f"batch_meta invalid: {what}")
        st, _ = oracle.build_batch_metadata(*args[:5], args[5], args[6], BS, 4096)
        assert st == 6, what
        check(gpu, *args, 4096)


def test_status_is_rewritten_by_every_call(gpu):
    say("batch_meta status reuse")
    rng = np.random.default_rng(11)
    kvw, new, flags, start, blocks, mbpr = batch(rng, 16, 1.0, 300, 1)
    bad = blocks.copy()
    bad[0] = -1
    out = check(gpu, kvw, new, flags, start, bad, 16, mbpr, 1 << 16)
    assert int(out["status"].item()) == 6
    out = check(gpu, kvw, new, flags, start, blocks, 16, mbpr, 1 << 16, out=out)
    assert int(out["status"].item()) == 0


def test_feeds_the_attention_kernels(gpu):
    """The device-built table and slots drive write_kv_cache + decode exactly like
    host-built ones (the same arrays, so the same bits)."""
    from ccinfer_amd import decode_attention, write_kv_cache
    say("batch_meta -> write_kv + decode")
    rng = np.random.default_rng(12)
    b, hq, hkv, d, ncb = 24, 16, 8, 128, 2048
    kvw, new, flags, start, blocks, mbpr = batch(rng, b, 1.0, 900, 1, ncb=ncb)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(gpu)  # noqa: E731
    meta = build_batch_metadata(dev(kvw), dev(new), dev(flags), dev(start), dev(blocks), b, mbpr,
                                ncb)
    _, host = oracle.build_batch_metadata(kvw, new, flags, start, blocks, b, mbpr, BS, ncb)
    g = torch.Generator(device=gpu).manual_seed(3)
    kc = torch.randn((ncb * BS, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    vc = torch.randn((ncb * BS, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    kn = torch.randn((b, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    vn = torch.randn((b, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    q = torch.randn((b, hq, d), generator=g, device=gpu).to(torch.bfloat16)
    outs = []
    for bt, ctx, sm in ((meta["block_table"], meta["context_lens"], meta["slot_mapping"]),
                        (dev(host["block_table"]), dev(host["context_lens"]),
                         dev(host["slot_mapping"]))):
        k2, v2 = kc.clone(), vc.clone()
        write_kv_cache(kn, vn, k2, v2, sm)
        outs.append(decode_attention(q, k2, v2, bt, ctx))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
