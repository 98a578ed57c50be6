"""Pins oracle.build_batch_metadata (the per-step arrays of BatchTranslator::translate,
src/worker/batch_translator.cpp:213-302, and the checks of src/model/model_runner.h:102-171)
before the device builder is checked against it.

Checks:
  - the shapes the reference's own translator tests assert (tests/unit/
    test_batch_translator.cpp: token counts, batch sizes, max_blocks_per_req, context after
    commit);
  - a vectorised numpy formulation (repeat / cumsum / table gather), independent of the
    oracle's per-item loops;
  - invariants: slot // bs is the table entry of pos // bs and slot % bs == pos % bs; slots
    of a batch with distinct blocks are distinct; query_start_loc is the prefix sum;
  - every validation rule, one at a time, and the sanitised entries it leaves.
"""
import numpy as np
import pytest

import oracle

BS = 16


def items_to_csr(tables):
    start = np.zeros(len(tables) + 1, np.int32)
    start[1:] = np.cumsum([len(t) for t in tables])
    blocks = np.concatenate([np.asarray(t, np.int32) for t in tables]) if start[-1] else \
        np.zeros(0, np.int32)
    return start, blocks


def run(kvw, new, flags, tables, mbpr=None, num_cache_blocks=64, T=None):
    start, blocks = items_to_csr(tables)
    T = int(np.sum(np.maximum(new, 0))) if T is None else T
    mbpr = max(1, max(len(t) for t in tables)) if mbpr is None else mbpr
    return oracle.build_batch_metadata(kvw, new, flags, start, blocks, T, mbpr, BS,
                                       num_cache_blocks)


def numpy_reference(kvw, new, flags, tables, mbpr):
    """Vectorised restatement: token arrays by repeat/arange, slots by table gather."""
    kvw, new = np.asarray(kvw, np.int64), np.asarray(new, np.int64)
    qsl = np.concatenate([[0], np.cumsum(new)])
    item_of_tok = np.repeat(np.arange(len(new)), new)
    t_in_item = np.arange(qsl[-1]) - qsl[item_of_tok]
    pos = kvw[item_of_tok] + t_in_item
    table = np.full((len(new), mbpr), -1, np.int64)
    for i, t in enumerate(tables):
        table[i, :len(t)] = t
    slot = table[item_of_tok, pos // BS] * BS + pos % BS
    sample = (np.asarray(flags) & (oracle.ITEM_DECODE | oracle.ITEM_SAMPLE)) != 0
    li = np.where(sample, qsl[1:] - 1, -1)
    return dict(positions=pos, slot_mapping=slot, block_table=table, query_start_loc=qsl,
                context_lens=kvw + new, logits_indices=li)


# ---- the reference translator tests (block ids are ours: the free-list order is the
# ---- KV manager's, the tests assert counts) ----

def test_reference_prefill_allocates_blocks():
    st, o = run([0], [16], [0], [[3]])
    assert st == 0 and len(o["positions"]) == 16 and o["block_table"].shape == (1, 1)
    assert o["context_lens"][0] == 16  # kv_written after commit (test :68)


def test_reference_decode_no_new_block():
    st, o = run([8], [1], [oracle.ITEM_DECODE], [[5]])
    assert st == 0 and len(o["positions"]) == 1 and o["positions"][0] == 8
    assert o["slot_mapping"][0] == 5 * 16 + 8 and o["context_lens"][0] == 9  # test :120


def test_reference_mixed_batch():
    st, o = run([8, 0], [1, 16], [oracle.ITEM_DECODE, 0], [[5], [9]])
    assert st == 0 and len(o["positions"]) == 17  # test :146
    assert list(o["query_start_loc"]) == [0, 1, 17]
    assert list(o["context_lens"]) == [9, 16]      # kv_written 9 and 16 after commit


def test_reference_prefill_spans_multiple_blocks():
    st, o = run([0], [20], [oracle.ITEM_SAMPLE], [[7, 2]])
    assert st == 0 and o["block_table"].shape == (1, 2) and len(o["positions"]) == 20
    assert o["slot_mapping"][16] == 2 * 16 and o["logits_indices"][0] == 19


def test_reference_partial_prefix_hit_runs_suffix():
    st, o = run([16], [4], [oracle.ITEM_SAMPLE], [[4, 11]])
    assert st == 0 and list(o["positions"]) == [16, 17, 18, 19]  # test :192-198
    assert list(o["slot_mapping"]) == [176, 177, 178, 179] and o["context_lens"][0] == 20


# ---- independent formulation and invariants ----

@pytest.mark.parametrize("seed", range(6))
def test_matches_vectorised_numpy(seed):
    rng = np.random.default_rng(seed)
    b = int(rng.integers(1, 40))
    kvw = rng.integers(0, 300, b)
    is_dec = rng.random(b) < 0.5
    new = np.where(is_dec, 1, rng.integers(1, 90, b))
    flags = np.where(is_dec, oracle.ITEM_DECODE, np.where(rng.random(b) < 0.5,
                                                          oracle.ITEM_SAMPLE, 0))
    perm = rng.permutation(4000)
    tables, cur = [], 0
    for i in range(b):
        need = -(-(kvw[i] + new[i]) // BS) + int(rng.integers(0, 3))
        tables.append(perm[cur:cur + need])
        cur += need
    mbpr = max(len(t) for t in tables) + 2
    st, o = run(kvw, new, flags, tables, mbpr=mbpr, num_cache_blocks=4000)
    assert st == 0
    want = numpy_reference(kvw, new, flags, tables, mbpr)
    for k, v in want.items():
        np.testing.assert_array_equal(o[k], v.astype(np.int32), err_msg=k)
    # invariants
    pos, slot = o["positions"], o["slot_mapping"]
    item = np.repeat(np.arange(b), new)
    assert np.all(o["block_table"][item, pos // BS] == slot // BS)
    assert np.all(slot % BS == pos % BS)
    assert len(np.unique(slot)) == len(slot)


# ---- validation (model_runner.h:102-171, batch_translator.cpp:196-211) ----

def test_each_check_fails_alone():
    ok = dict(kvw=[8, 0], new=[1, 16], flags=[oracle.ITEM_DECODE, 0], tables=[[5], [9]])
    assert run(**ok)[0] == 0
    cases = {
        "zero query length": dict(ok, new=[1, 0]),
        "decode item with two tokens": dict(ok, new=[2, 16]),
        "negative kv_written": dict(ok, kvw=[-1, 0]),
        "too few blocks for the context": dict(ok, kvw=[16, 0]),
        "block id past the cache": dict(ok, tables=[[5], [64]]),
        "negative block id": dict(ok, tables=[[-1], [9]]),
    }
    for what, kw in cases.items():
        assert run(**kw)[0] == 6, what
    assert run(**ok, T=18)[0] == 6                              # qsl[B] != T
    assert run(**ok, mbpr=65, num_cache_blocks=64)[0] == 6      # table wider than the cache
    assert run(kvw=[0], new=[40], flags=[0], tables=[[1, 2, 3]], mbpr=2)[0] == 6  # ctx > mbpr*bs


def test_failing_entries_are_sanitised():
    st, o = run([0, 0], [16, 16], [0, 0], [[5], [99]])
    assert st == 6
    assert np.all(o["slot_mapping"][:16] == 5 * 16 + np.arange(16))
    assert np.all(o["slot_mapping"][16:] == -1)
    assert list(o["block_table"][:, 0]) == [5, -1]


def test_bad_block_range_means_no_blocks():
    start = np.array([0, 5, 1], np.int32)  # item 1's range runs backwards
    st, o = oracle.build_batch_metadata([0, 0], [4, 4], [0, 0], start,
                                        np.arange(5, dtype=np.int32), 8, 5, BS, 64)
    assert st == 6 and np.all(o["slot_mapping"][4:] == -1) and np.all(o["block_table"][1] == -1)


def test_tokens_past_num_tokens_are_not_written():
    st, o = run([0, 0], [4, 4], [0, 0], [[1], [2]], T=6)
    assert st == 6 and len(o["positions"]) == 6
    assert list(o["positions"]) == [0, 1, 2, 3, 0, 1]
