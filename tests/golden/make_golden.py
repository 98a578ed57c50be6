"""Writes the golden fixtures of tests/golden/*.npz (inputs + expected outputs).

    python -m tests.golden.make_golden

Inputs are the reference tests' own known-answer vectors (tests/kernel/test_decode_attn.cu
:229-311, test_write_kv_cache.cu:15-98, test_prefill_attn.cu:24-105 with the LCG of
test_naive_attn.cu:67-74, test_rope.cu:118-158, test_batch_translator.cu's mixed batch) and
tiny seeded instances of the benchmark configurations and of the fused prologue, the batch
metadata build and the fp8 cache write.
Expected outputs come from the CPU oracle (oracle/, pinned by tests/test_oracle.py).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

NAMES = ["decode_kat", "write_kv_kat", "prefill_kat", "decode_small", "prefill_small",
         "mixed_small", "prologue_rope_kat", "prologue_small", "batch_meta_mixed",
         "fp8_write_small"]


def path(name: str) -> Path:
    return HERE / f"{name}.npz"


def _bf(x):
    return oracle.f32_to_bf16(np.asarray(x, np.float32))


def inputs(name: str) -> dict:
    rng = np.random.default_rng(20261201)
    if name == "decode_kat":
        qi, ki = np.arange(2 * 8 * 64), np.arange(3 * 16 * 2 * 64)
        return dict(q=_bf(((qi * 17) % 23 - 11) * 0.03125).reshape(2, 8, 64),
                    k=_bf(((ki * 13) % 29 - 14) * 0.025).reshape(48, 2, 64),
                    v=_bf(((ki * 7) % 31 - 15) * 0.02).reshape(48, 2, 64),
                    bt=np.array([[2, 0, 1], [1, 2, -1]], np.int32),
                    ctx=np.array([31, 17], np.int32))
    if name == "write_kv_kat":
        t, h, d = np.meshgrid(np.arange(4), np.arange(2), np.arange(4), indexing="ij")
        return dict(k_new=_bf(t * 100 + h * 10 + d), v_new=_bf(t * 200 + h * 10 + d),
                    slots=np.array([5, 17, 0, 63], np.int32),
                    k_cache=np.zeros((64, 2, 4), np.uint16), v_cache=np.zeros((64, 2, 4), np.uint16))
    if name == "prefill_kat":
        return dict(q=oracle.lcg_fill(32 * 4 * 64, 1).reshape(32, 4, 64),
                    k=oracle.lcg_fill(64 * 4 * 64, 2).reshape(64, 4, 64),
                    v=oracle.lcg_fill(64 * 4 * 64, 3).reshape(64, 4, 64),
                    bt=np.array([[0, 1]], np.int32), qsl=np.array([0, 32], np.int32),
                    ctx=np.array([32], np.int32))
    if name == "decode_small":
        ctx = np.array([1, 16, 33, 64], np.int32)
        pool = 5
        bt = np.stack([rng.permutation(pool)[:4] for _ in range(4)]).astype(np.int32)
        return dict(q=_bf(rng.standard_normal((4, 16, 128))),
                    k=_bf(rng.standard_normal((pool * 16, 8, 128))),
                    v=_bf(rng.standard_normal((pool * 16, 8, 128))), bt=bt, ctx=ctx)
    if name == "prefill_small":
        # 2 sequences x (16 cached prefix + 24 new); both list the same prefix block.
        bt = np.array([[3, 0, 4], [3, 1, 2]], np.int32)
        return dict(q=_bf(rng.standard_normal((48, 16, 128))),
                    k=_bf(rng.standard_normal((5 * 16, 8, 128))),
                    v=_bf(rng.standard_normal((5 * 16, 8, 128))), bt=bt,
                    qsl=np.array([0, 24, 48], np.int32), ctx=np.array([40, 40], np.int32))
    if name == "mixed_small":
        # one 20-token chunk with 16 cached positions + two single-token decode items
        bt = np.array([[0, 2, 4], [1, 3, -1], [2, -1, -1]], np.int32)
        return dict(q=_bf(rng.standard_normal((22, 16, 128))),
                    k=_bf(rng.standard_normal((5 * 16, 8, 128))),
                    v=_bf(rng.standard_normal((5 * 16, 8, 128))), bt=bt,
                    qsl=np.array([0, 20, 21, 22], np.int32), ctx=np.array([36, 30, 9], np.int32))
    if name == "prologue_rope_kat":
        # the reference RoPE GQA test (tests/kernel/test_rope.cu:118-158): 2 tokens, 8 q / 2 kv
        # heads, d=64, positions 5 and 17, a 32-position table with theta 1e4; no norm
        q = ((np.arange(2 * 8 * 64) % 7) - 2).reshape(2, 8 * 64)
        k = (((np.arange(2 * 2 * 64) + 3) % 9) - 3).reshape(2, 2 * 64)
        v = ((np.arange(2 * 2 * 64) % 5) - 2).reshape(2, 2 * 64)
        return dict(qkv=_bf(np.concatenate([q, k, v], 1)), positions=np.array([5, 17], np.int32),
                    rope_cache=oracle.rope_cache_table(32, 64, 1e4),
                    slots=np.array([3, 12], np.int32),
                    k_cache=np.zeros((16, 2, 64), np.uint16),
                    v_cache=np.zeros((16, 2, 64), np.uint16), nq=8, nkv=2, hd=64)
    if name == "prologue_small":
        # 5 tokens, 16 q / 8 kv heads, d=128, norm weights; one position outside the table and
        # one skipped slot
        return dict(qkv=_bf(rng.standard_normal((5, 32 * 128)) * 2),
                    q_norm_w=_bf(rng.standard_normal(128)), k_norm_w=_bf(rng.standard_normal(128)),
                    positions=np.array([0, 7, 63, 64, 30], np.int32),
                    rope_cache=oracle.rope_cache_table(64, 128, 1e6),
                    slots=np.array([1, -1, 9, 4, 17], np.int32),
                    k_cache=oracle.lcg_fill(20 * 8 * 128, 9).reshape(20, 8, 128),
                    v_cache=oracle.lcg_fill(20 * 8 * 128, 10).reshape(20, 8, 128),
                    nq=16, nkv=8, hd=128)
    if name == "batch_meta_mixed":
        # the reference translator's mixed batch (a decode item with 8 cached tokens and a
        # 16-token prefill chunk), plus a sampled 20-token prefill over two blocks and a
        # decode item with a prefix-cache hit (16 cached tokens)
        return dict(kv_written=np.array([8, 0, 0, 16], np.int32),
                    new_tokens=np.array([1, 16, 20, 1], np.int32),
                    flags=np.array([1, 0, 2, 1], np.int32),
                    block_start=np.array([0, 1, 2, 4, 6], np.int32),
                    blocks=np.array([5, 9, 7, 2, 4, 11], np.int32),
                    num_tokens=38, mbpr=3, num_cache_blocks=32)
    if name == "fp8_write_small":
        k = rng.standard_normal((6, 2, 128)) * np.array([1.0, 300.0])[None, :, None]
        k[2, 1] = 0.0  # an all-zero row
        return dict(k_new=_bf(k), v_new=_bf(rng.standard_normal((6, 2, 128)) * 1e-3),
                    slots=np.array([0, 17, 5, -1, 31, 16], np.int32),
                    k_cache=np.zeros((32, 2, 128), np.uint8), v_cache=np.zeros((32, 2, 128), np.uint8),
                    k_scale=np.zeros(64, np.float32), v_scale=np.zeros(64, np.float32))
    raise KeyError(name)


def compute(name: str, fx) -> dict:
    """Expected outputs for the inputs held in fx."""
    if name == "write_kv_kat":
        kc, vc = np.array(fx["k_cache"]), np.array(fx["v_cache"])
        oracle.write_kv_cache(fx["k_new"], fx["v_new"], kc, vc, fx["slots"])
        return dict(k_out=kc, v_out=vc)
    if name in ("prologue_rope_kat", "prologue_small"):
        kc, vc = np.array(fx["k_cache"]), np.array(fx["v_cache"])
        qw = fx["q_norm_w"] if "q_norm_w" in fx else None
        kw = fx["k_norm_w"] if "k_norm_w" in fx else None
        q = oracle.qkv_prologue(fx["qkv"], qw, kw, fx["positions"], fx["rope_cache"], fx["slots"],
                                kc, vc, int(fx["nq"]), int(fx["nkv"]), int(fx["hd"]), 1e-6)
        return dict(q_out=q, k_out=kc, v_out=vc)
    if name == "batch_meta_mixed":
        st, o = oracle.build_batch_metadata(fx["kv_written"], fx["new_tokens"], fx["flags"],
                                            fx["block_start"], fx["blocks"], int(fx["num_tokens"]),
                                            int(fx["mbpr"]), 16, int(fx["num_cache_blocks"]))
        return dict(status=np.array(st, np.int32), **{f"out_{k}": v for k, v in o.items()})
    if name == "fp8_write_small":
        arr = {k: np.array(fx[k]) for k in ("k_cache", "v_cache", "k_scale", "v_scale")}
        oracle.write_kv_cache_fp8(fx["k_new"], fx["v_new"], arr["k_cache"], arr["v_cache"],
                                  arr["k_scale"], arr["v_scale"], fx["slots"])
        return {f"{k}_out": v for k, v in arr.items()}
    if name in ("decode_kat", "decode_small"):
        return dict(out=oracle.decode(fx["q"], fx["k"], fx["v"], fx["bt"], fx["ctx"], nthreads=1))
    out = oracle.prefill(fx["q"], fx["k"], fx["v"], fx["bt"], fx["qsl"], fx["ctx"], nthreads=1)
    res = dict(out=out)
    if name == "prefill_kat":
        res["out_dense"] = oracle.naive(fx["q"], fx["k"][:32], fx["v"][:32])
    return res


def main():
    for name in NAMES:
        fx = inputs(name)
        fx.update(compute(name, fx))
        np.savez_compressed(path(name), **fx)
        print(f"wrote {path(name)} ({path(name).stat().st_size} bytes)")


if __name__ == "__main__":
    main()
