"""Invariants of the seeded benchmark workloads (CPU): block tables follow the reference's
contract (src/worker/batch_translator.cpp:213-293) and the configurations match
BASELINE.json's descriptions."""
import numpy as np

from ccinfer_amd import workloads as W


def _valid_blocks(w):
    out = []
    for b in range(w.batch):
        n = -(-int(w.context_lens[b]) // 16)
        row = w.block_table[b]
        assert np.all(row[:n] >= 0) and np.all(row[n:] == -1)
        out.append(row[:n])
    return out


def test_decode_single_config1():
    w = W.decode_single(hq=2, hkv=1, d=16)
    assert w.context_lens.tolist() == [512] and w.block_table.shape == (1, 32)
    assert w.num_blocks == 256 and len(set(w.block_table[0].tolist())) == 32
    assert w.kv_bytes() == 512 * 1 * 16 * 4


def test_decode_batched_config2_pool_and_slots():
    w = W.decode_batched(hq=2, hkv=1, d=16)
    assert w.batch == 64
    assert w.context_lens.min() >= 128 and w.context_lens.max() <= 4096
    rows = _valid_blocks(w)
    used = np.concatenate(rows)
    assert len(set(used.tolist())) == used.size          # drawn without replacement
    assert w.num_blocks == int(np.ceil(1.1 * used.size))
    assert used.max() < w.num_blocks
    pos = w.context_lens - 1                              # the new token is the last position
    want = w.block_table[np.arange(64), pos // 16] * 16 + pos % 16
    assert np.array_equal(w.slot_mapping, want)


def test_prefill_config3_shared_prefix_and_flops():
    w = W.prefill_prefix(hq=16, hkv=8, d=128)
    assert w.batch == 8 and int(w.query_start_loc[-1]) == 8 * 1536
    assert np.all(w.context_lens == 2048)
    rows = _valid_blocks(w)
    assert np.array_equal(rows[0][:32], rows[1][:32])    # seqs 0 and 1 share the prefix
    others = np.concatenate([rows[0], rows[1][32:]] + rows[2:])
    assert len(set(others.tolist())) == others.size
    # slots of new tokens start after the 512 cached positions
    assert w.slot_mapping[0] == rows[0][32] * 16
    assert W.prefill_flops(w) == 4 * 128 * 16 * 8 * sum(512 + i + 1 for i in range(1536))


def test_mixed_config4_shapes():
    w = W.mixed_step(hq=2, hkv=1, d=16)
    qsl = w.query_start_loc
    ql = qsl[1:] - qsl[:-1]
    assert ql[:4].tolist() == [512] * 4 and np.all(ql[4:] == 1)
    pre = w.context_lens[:4] - 512
    assert np.all(pre % 16 == 0) and pre.min() >= 0 and pre.max() <= 2048
    assert w.context_lens[4:].min() >= 1024 and w.context_lens[4:].max() <= 32768
    _valid_blocks(w)


def test_decode_long_config5():
    w = W.decode_long(batch=2, ctx=4096, hq=4, hkv=1, d=16)
    rows = _valid_blocks(w)
    assert all(r.size == 256 for r in rows)
    used = np.concatenate(rows)
    assert len(set(used.tolist())) == used.size


def test_seeded_generation_is_deterministic():
    a = W.decode_batched(batch=4, hq=2, hkv=1, d=16)
    b = W.decode_batched(batch=4, hq=2, hkv=1, d=16)
    assert np.array_equal(a.block_table, b.block_table)
    assert (a.k_cache.view(-1)[:1000] == b.k_cache.view(-1)[:1000]).all()
