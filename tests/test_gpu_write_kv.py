"""KV-cache write on the GPU: bit-exact against the oracle and the reference KAT.

Reference: src/kernel/attention/write_kv_cache.cu:12-34; KAT from
tests/kernel/test_write_kv_cache.cu:15-98 (slots {5,17,0,63}, K=t*100+h*10+d,
V=t*200+h*10+d, bitwise compare, unwritten slot stays zero).
"""
import numpy as np
import pytest
import torch

import oracle
from ccinfer_amd import CcinferError, write_kv_cache
from ccinfer_amd import workloads as W
from tests._util import from_u16, say, u16

pytestmark = pytest.mark.gpu


def _kat_inputs(t=4, h=2, d=4):
    tt, hh, dd = np.meshgrid(np.arange(t), np.arange(h), np.arange(d), indexing="ij")
    k = oracle.f32_to_bf16((tt * 100 + hh * 10 + dd).astype(np.float32))
    v = oracle.f32_to_bf16((tt * 200 + hh * 10 + dd).astype(np.float32))
    return k, v


@pytest.mark.parametrize("head_dim", [4, 3])  # 16-byte rows (vector path) and 12-byte rows
def test_reference_kat(gpu, head_dim):
    say(f"write_kv KAT head_dim={head_dim}")
    k, v = _kat_inputs(d=head_dim)
    slots = np.array([5, 17, 0, 63], np.int32)
    kc = torch.zeros((64, 2, head_dim), dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    write_kv_cache(from_u16(k, gpu), from_u16(v, gpu), kc, vc,
                   torch.from_numpy(slots).to(gpu))
    torch.cuda.synchronize()
    kh, vh = u16(kc), u16(vc)
    for t, s in enumerate(slots):
        assert np.array_equal(kh[s], k[t]) and np.array_equal(vh[s], v[t])
    assert np.all(kh[1] == 0)  # unwritten slot stays zero
    want_k = np.zeros_like(kh)
    want_v = np.zeros_like(vh)
    oracle.write_kv_cache(k, v, want_k, want_v, slots)
    assert np.array_equal(kh, want_k) and np.array_equal(vh, want_v)


def test_out_of_range_slots_are_skipped(gpu):
    say("write_kv out-of-range slots")
    rng = np.random.default_rng(7)
    hkv, d, max_slots = 8, 128, 96
    k = oracle.f32_to_bf16(rng.standard_normal((6, hkv, d)).astype(np.float32))
    v = oracle.f32_to_bf16(rng.standard_normal((6, hkv, d)).astype(np.float32))
    slots = np.array([3, -1, max_slots, 95, 1 << 20, 0], np.int32)
    init_k = oracle.f32_to_bf16(rng.standard_normal((max_slots, hkv, d)).astype(np.float32))
    init_v = oracle.f32_to_bf16(rng.standard_normal((max_slots, hkv, d)).astype(np.float32))
    kc, vc = from_u16(init_k, gpu), from_u16(init_v, gpu)
    write_kv_cache(from_u16(k, gpu), from_u16(v, gpu), kc, vc, torch.from_numpy(slots).to(gpu))
    torch.cuda.synchronize()
    want_k, want_v = init_k.copy(), init_v.copy()
    oracle.write_kv_cache(k, v, want_k, want_v, slots)
    assert np.array_equal(u16(kc), want_k) and np.array_equal(u16(vc), want_v)


@pytest.mark.parametrize("cfg", ["decode_batched", "prefill_prefix", "mixed_step"])
def test_config_writes_bit_exact(gpu, cfg):
    say(f"write_kv {cfg}")
    w = getattr(W, cfg)(device=gpu)
    kc0, vc0 = u16(w.k_cache), u16(w.v_cache)
    sm = torch.from_numpy(w.slot_mapping).to(gpu)
    write_kv_cache(w.k_new, w.v_new, w.k_cache, w.v_cache, sm)
    torch.cuda.synchronize()
    oracle.write_kv_cache(u16(w.k_new), u16(w.v_new), kc0, vc0, w.slot_mapping)
    assert np.array_equal(u16(w.k_cache), kc0)
    assert np.array_equal(u16(w.v_cache), vc0)


def test_null_and_shape_errors(gpu):
    say("write_kv errors")
    kc = torch.zeros((8, 2, 4), dtype=torch.bfloat16, device=gpu)
    bad_new = torch.zeros((2, 3, 4), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(CcinferError) as e:
        write_kv_cache(bad_new, bad_new, kc, kc.clone(),
                       torch.zeros(2, dtype=torch.int32, device=gpu))
    assert e.value.code == 6
