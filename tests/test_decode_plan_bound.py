"""The flat decode plan's partial-slot bound (plan_decode in ccinfer_amd/csrc/decode_attn.hip)
against a replay of what decode_flat_index_kernel lays out, on extreme ragged batches.

The index kernel drops ranges and splits numbered at or past `slots` (and then flags the plan
so the merge writes NaN); this replays its counting in numpy and checks that the host bound
always leaves room: the number of ranges and the number of partial slots (splits) stay within
`slots`, for the even ranges, the snapped ranges and the whole-request layout.
Constants restate decode_attn.hip: kChunk 32, kMaxSplitTokens 2048, kEvenWaves 1024 (2048
for fp8 and for bf16 rows of up to 80 dims: the `fp8=True` cases), kFlatMinItems 4,
kSnapWaves 4096."""
import numpy as np
import pytest

K_CHUNK = 32
K_MAXT = 2048 // K_CHUNK
K_EVEN = {False: 1024, True: 2048}
K_SNAP_WAVES = 4096


def slots_bound(num_items, hkv, max_ctx, fp8=False):
    chunks = -(-max_ctx // K_CHUNK)
    w = max(max(1, K_EVEN[fp8] // hkv), num_items)
    capped = num_items * (-(-chunks // K_MAXT))
    return min(max(w, capped) + num_items, num_items * chunks), w


def replay(c, W, snap, rows):
    """(ranges, splits) of the index kernel for per-request chunk counts c."""
    C = int(c.sum())
    T = min(max(-(-C // W), 1), K_MAXT)
    if rows:
        ns = -(-c // K_MAXT)
        return int(ns.sum()), int(ns.sum())
    starts = np.arange(0, -(-C // T)) * T
    P = np.concatenate([[0], np.cumsum(c)])
    if snap:
        slack = min(T // 2, (K_MAXT - T) // 2)
        out = []
        for s in starts:
            r = int(np.searchsorted(P, s, side="right") - 1)
            dl, dr = s - P[r], P[r + 1] - s
            if dl <= slack and dl <= dr:
                s = P[r]
            elif dr <= slack:
                s = P[r + 1]
            out.append(s)
        starts = np.array(out)
    L = np.concatenate([starts, [C]])
    splits = 0
    for r in range(len(c)):
        if c[r] == 0:
            continue
        first = np.searchsorted(L, P[r], side="right") - 1
        last = np.searchsorted(L, P[r + 1] - 1, side="right") - 1
        splits += int(last - first + 1)
    return len(starts), splits


def batches(rng):
    yield "all max", np.full(300, 4096)
    yield "all one token", np.ones(5000, np.int64)
    yield "one huge + tiny", np.concatenate([[131072], np.ones(999, np.int64)])
    yield "alternating", np.tile([1, 32768], 64)
    yield "log-uniform", np.floor(np.exp(rng.uniform(np.log(1), np.log(65536), 2048))).astype(np.int64)
    yield "boundary multiples", np.full(4096, 2048)
    yield "just past chunk", np.full(777, 33)
    for n in (4, 5, 63, 257, 1023, 4097):
        yield f"uniform n={n}", rng.integers(1, 20000, n)


@pytest.mark.parametrize("hkv", [1, 2, 8, 32])
@pytest.mark.parametrize("fp8", [False, True])
def test_flat_index_fits_the_slot_bound(hkv, fp8):
    rng = np.random.default_rng(hkv * 7 + fp8)
    for name, ctx in batches(rng):
        ctx = np.asarray(ctx, np.int64)
        c = -(-ctx // K_CHUNK)
        max_ctx = int(ctx.max())
        slots, W = slots_bound(len(ctx), hkv, max_ctx, fp8)
        snap = W * hkv >= K_SNAP_WAVES
        for rows in (False, True):
            for s in ((snap,) if not rows else (True,)):
                ranges, splits = replay(c, W, s, rows)
                assert ranges <= slots, (name, hkv, fp8, rows, s, ranges, slots)
                assert splits <= slots, (name, hkv, fp8, rows, s, splits, slots)
