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
