"""GPU results against the committed golden fixtures (tests/golden/*.npz): the reference
tests' known-answer inputs and tiny instances of the benchmark shapes, with the expected
outputs stored (no oracle call at run time)."""
import numpy as np
import pytest
import torch

from ccinfer_amd import decode_attention, prefill_attention, write_kv_cache
from tests._util import assert_attn_close, f32, from_u16, say, u16
from tests.golden import make_golden

pytestmark = pytest.mark.gpu


def _i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


def test_write_kv_kat(gpu):
    say("golden write_kv_kat")
    fx = np.load(make_golden.path("write_kv_kat"))
    kc, vc = from_u16(fx["k_cache"], gpu), from_u16(fx["v_cache"], gpu)
    write_kv_cache(from_u16(fx["k_new"], gpu), from_u16(fx["v_new"], gpu), kc, vc,
                   _i32(fx["slots"], gpu))
    torch.cuda.synchronize()
    assert np.array_equal(u16(kc), fx["k_out"]) and np.array_equal(u16(vc), fx["v_out"])


@pytest.mark.parametrize("name", ["decode_kat", "decode_small"])
def test_decode_fixture(gpu, name):
    say(f"golden {name}")
    fx = np.load(make_golden.path(name))
    out = decode_attention(from_u16(fx["q"], gpu), from_u16(fx["k"], gpu), from_u16(fx["v"], gpu),
                           _i32(fx["bt"], gpu), _i32(fx["ctx"], gpu))
    assert_attn_close(f32(out), fx["out"], name)


@pytest.mark.parametrize("name", ["prefill_kat", "prefill_small", "mixed_small"])
def test_prefill_fixture(gpu, name):
    say(f"golden {name}")
    fx = np.load(make_golden.path(name))
    out = prefill_attention(from_u16(fx["q"], gpu), from_u16(fx["k"], gpu),
                            from_u16(fx["v"], gpu), _i32(fx["bt"], gpu), _i32(fx["qsl"], gpu),
                            _i32(fx["ctx"], gpu))
    assert_attn_close(f32(out), fx["out"], name)
    if "out_dense" in fx:
        assert_attn_close(f32(out), fx["out_dense"], name + " vs dense")


@pytest.mark.parametrize("name", ["prologue_rope_kat", "prologue_small"])
def test_prologue_fixture(gpu, name):
    from ccinfer_amd import qkv_prologue
    say(f"golden {name}")
    fx = np.load(make_golden.path(name))
    kc, vc = from_u16(fx["k_cache"], gpu), from_u16(fx["v_cache"], gpu)
    qw = from_u16(fx["q_norm_w"], gpu) if "q_norm_w" in fx else None
    kw = from_u16(fx["k_norm_w"], gpu) if "k_norm_w" in fx else None
    q = qkv_prologue(from_u16(fx["qkv"], gpu), qw, kw, _i32(fx["positions"], gpu),
                     torch.from_numpy(fx["rope_cache"]).to(gpu), _i32(fx["slots"], gpu), kc, vc,
                     int(fx["nq"]), 1e-6)
    torch.cuda.synchronize()
    # q and K within one bf16 ulp (plus 2^-20 of the row maximum for RoPE cancellation);
    # V and untouched rows bit-exact
    for got, want in ((u16(q), fx["q_out"]), (u16(kc), fx["k_out"])):
        g = f32(from_u16(got)).astype(np.float64)
        w = f32(from_u16(want)).astype(np.float64)
        e = np.floor(np.log2(np.maximum(np.abs(w), 2.0 ** -126)))
        bound = 2.0 ** (e - 7) + 2.0 ** -20 * np.abs(w).max(-1, keepdims=True)
        assert np.all(np.abs(g - w) <= bound), name
    assert np.array_equal(u16(vc), fx["v_out"])


def test_batch_meta_fixture(gpu):
    from ccinfer_amd import build_batch_metadata
    say("golden batch_meta_mixed")
    fx = np.load(make_golden.path("batch_meta_mixed"))
    got = build_batch_metadata(_i32(fx["kv_written"], gpu), _i32(fx["new_tokens"], gpu),
                               _i32(fx["flags"], gpu), _i32(fx["block_start"], gpu),
                               _i32(fx["blocks"], gpu), int(fx["num_tokens"]), int(fx["mbpr"]),
                               int(fx["num_cache_blocks"]))
    torch.cuda.synchronize()
    assert int(got["status"].item()) == int(fx["status"])
    for k in ("positions", "slot_mapping", "block_table", "query_start_loc", "context_lens",
              "logits_indices"):
        assert np.array_equal(got[k].cpu().numpy(), fx[f"out_{k}"]), k


def test_fp8_write_fixture(gpu):
    from ccinfer_amd import write_kv_cache_fp8
    say("golden fp8_write_small")
    fx = np.load(make_golden.path("fp8_write_small"))
    dev = {k: torch.from_numpy(np.array(fx[k])).to(gpu)
           for k in ("k_cache", "v_cache", "k_scale", "v_scale")}
    write_kv_cache_fp8(from_u16(fx["k_new"], gpu), from_u16(fx["v_new"], gpu), dev["k_cache"],
                       dev["v_cache"], dev["k_scale"], dev["v_scale"], _i32(fx["slots"], gpu))
    torch.cuda.synchronize()
    for k, t in dev.items():
        got = t.cpu().numpy()
        want = fx[f"{k}_out"]
        if got.dtype == np.float32:
            got, want = got.view(np.uint32), want.view(np.uint32)
        assert np.array_equal(got, want), k
