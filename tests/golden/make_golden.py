"""Writes the golden fixtures of tests/golden/*.npz (inputs + expected outputs).

    python -m tests.golden.make_golden

Inputs are the reference tests' own known-answer vectors (tests/kernel/test_decode_attn.cu
:229-311, test_write_kv_cache.cu:15-98, test_prefill_attn.cu:24-105 with the LCG of
test_naive_attn.cu:67-74) and tiny seeded instances of the benchmark configurations.
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
         "mixed_small"]


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
    raise KeyError(name)


def compute(name: str, fx) -> dict:
    """Expected outputs for the inputs held in fx."""
    if name == "write_kv_kat":
        kc, vc = np.array(fx["k_cache"]), np.array(fx["v_cache"])
        oracle.write_kv_cache(fx["k_new"], fx["v_new"], kc, vc, fx["slots"])
        return dict(k_out=kc, v_out=vc)
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
