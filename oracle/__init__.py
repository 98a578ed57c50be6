"""numpy front end of the CPU oracle (liboracle.so, built from attn_oracle.c by the Makefile).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py as the checker; the product path never imports it.
bf16 arrays are numpy uint16 bit patterns. Citations of the reference functions each
oracle routine restates are in attn_oracle.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None
_P = ctypes.c_void_p
_I = ctypes.c_int


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.orc_f32_to_bf16_array.argtypes = [_P, _P, ctypes.c_int64]
        lib.orc_kv_base_offset.argtypes = [_I, _I, _I, _I, _I, _I, _P, _P]
        lib.orc_kv_base_offset.restype = _I
        lib.orc_write_kv_cache.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I]
        lib.orc_decode_attention.argtypes = [_P, _P, _P, _P, _P, _P] + [_I] * 7
        lib.orc_decode_attention_pairs.argtypes = [_P, _P, _P, _P, _P, _P] + [_I] * 6 + [_P, _I, _I]
        lib.orc_prefill_attention.argtypes = [_P] * 7 + [_I] * 8
        lib.orc_prefill_attention_pairs.argtypes = [_P] * 7 + [_I] * 7 + [_P, _I, _I]
        lib.orc_naive_attention.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I]
        lib.orc_lcg_fill.argtypes = [_P, _I, ctypes.c_uint]
        lib.orc_split_qkv.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I]
        lib.orc_rms_norm.argtypes = [_P, _P, _P, _I, _I, ctypes.c_float]
        lib.orc_rope.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I]
        lib.orc_qkv_prologue.argtypes = [_P] * 11 + [_I] * 6 + [ctypes.c_float]
        lib.orc_build_batch_metadata.argtypes = [_P] * 5 + [_I] * 6 + [_P] * 6
        lib.orc_build_batch_metadata.restype = _I
        lib.orc_f32_to_e4m3.argtypes = [ctypes.c_float]
        lib.orc_f32_to_e4m3.restype = ctypes.c_uint8
        lib.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        lib.orc_e4m3_to_f32.restype = ctypes.c_float
        lib.orc_write_kv_cache_fp8.argtypes = [_P] * 7 + [_I] * 5
        lib.orc_decode_attention_fp8.argtypes = [_P] * 8 + [_I] * 7
        lib.orc_prefill_attention_fp8.argtypes = [_P] * 9 + [_I] * 8
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(_P)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    load().orc_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def kv_base_offset(ctx_pos, kv_head, head_dim, num_kv_heads, block_size, req_blocks):
    rb = _c(req_blocks, np.int32)
    out = np.zeros(1, np.int64)
    ok = load().orc_kv_base_offset(ctx_pos, kv_head, head_dim, num_kv_heads, block_size,
                                   rb.size, _p(rb), _p(out))
    return int(out[0]) if ok else None


def write_kv_cache(k_new, v_new, k_cache, v_cache, slot_mapping, max_slots=None) -> None:
    """In place on k_cache / v_cache (uint16 arrays [slots, Hkv, D])."""
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    kn, vn = _c(k_new, np.uint16), _c(v_new, np.uint16)
    sm = _c(slot_mapping, np.int32)
    slots, hkv, d = k_cache.shape
    load().orc_write_kv_cache(_p(kn), _p(vn), _p(k_cache), _p(v_cache), _p(sm), sm.size, hkv, d,
                              slots if max_slots is None else max_slots)


def decode(q, k_cache, v_cache, block_table, context_lens, block_size: int = 16,
           nthreads: Optional[int] = None, pairs=None) -> np.ndarray:
    """fp32 [B, Hq, D]; with `pairs` ([(b, hq)...]) only those rows are computed (rest 0)."""
    q, k, v = _c(q, np.uint16), _c(k_cache, np.uint16), _c(v_cache, np.uint16)
    bt, cl = _c(block_table, np.int32), _c(context_lens, np.int32)
    b, hq, d = q.shape
    hkv = k.shape[-2]
    out = np.zeros((b, hq, d), np.float32)
    nt = default_threads() if nthreads is None else nthreads
    if pairs is None:
        load().orc_decode_attention(_p(q), _p(k), _p(v), _p(bt), _p(cl), _p(out), b, bt.shape[1],
                                    hq, hkv, d, block_size, nt)
    else:
        pr = _c(pairs, np.int32).reshape(-1, 2)
        load().orc_decode_attention_pairs(_p(q), _p(k), _p(v), _p(bt), _p(cl), _p(out), b,
                                          bt.shape[1], hq, hkv, d, block_size, _p(pr),
                                          pr.shape[0], nt)
    return out


def prefill(q, k_cache, v_cache, block_table, query_start_loc, context_lens,
            block_size: int = 16, nthreads: Optional[int] = None, pairs=None,
            out: Optional[np.ndarray] = None) -> np.ndarray:
    """fp32 [T, Hq, D]; rows the reference leaves unwritten keep `out`'s values (0)."""
    q, k, v = _c(q, np.uint16), _c(k_cache, np.uint16), _c(v_cache, np.uint16)
    bt, qsl, cl = (_c(block_table, np.int32), _c(query_start_loc, np.int32),
                   _c(context_lens, np.int32))
    t, hq, d = q.shape
    hkv = k.shape[-2]
    if out is None:
        out = np.zeros((t, hq, d), np.float32)
    nt = default_threads() if nthreads is None else nthreads
    if pairs is None:
        load().orc_prefill_attention(_p(q), _p(k), _p(v), _p(bt), _p(qsl), _p(cl), _p(out),
                                     cl.size, t, bt.shape[1], hq, hkv, d, block_size, nt)
    else:
        pr = _c(pairs, np.int32).reshape(-1, 2)
        load().orc_prefill_attention_pairs(_p(q), _p(k), _p(v), _p(bt), _p(qsl), _p(cl), _p(out),
                                           cl.size, t, bt.shape[1], hq, hkv, d, block_size,
                                           _p(pr), pr.shape[0], nt)
    return out


def naive(q, k, v) -> np.ndarray:
    """Dense causal attention on contiguous q [T,Hq,D], k/v [T,Hkv,D]; fp32 out."""
    q, k, v = _c(q, np.uint16), _c(k, np.uint16), _c(v, np.uint16)
    t, hq, d = q.shape
    out = np.zeros((t, hq, d), np.float32)
    load().orc_naive_attention(_p(q), _p(k), _p(v), _p(out), t, hq, k.shape[1], d)
    return out


def lcg_fill(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.uint16)
    load().orc_lcg_fill(_p(out), n, seed)
    return out


# ---- decode-side prologue (split QKV, q/k RMSNorm, RoPE, KV write) ----

def split_qkv(qkv, nq: int, nkv: int, hd: int):
    """qkv uint16 [T, (nq + 2 nkv) * hd] -> (q [T, nq, hd], k [T, nkv, hd], v [T, nkv, hd])."""
    x = _c(qkv, np.uint16)
    t = x.shape[0]
    q = np.empty((t, nq, hd), np.uint16)
    k = np.empty((t, nkv, hd), np.uint16)
    v = np.empty((t, nkv, hd), np.uint16)
    load().orc_split_qkv(_p(x), _p(q), _p(k), _p(v), t, nq, nkv, hd)
    return q, k, v


def rms_norm(x, weight, eps: float):
    """Rows of x (uint16 [..., dim]) normalised as the reference kernel does; uint16 out."""
    x = _c(x, np.uint16)
    w = _c(weight, np.uint16)
    dim = x.shape[-1]
    out = np.empty_like(x)
    load().orc_rms_norm(_p(x), _p(w), _p(out), x.size // dim, dim, eps)
    return out


def rope(q, k, positions, rope_cache, rotary_dim=None):
    """Returns rotated copies of q [T, nq, hd] and k [T, nkv, hd] (uint16); rope_cache is
    float32 [max_pos, rotary_dim / 2, 2] of (cos, sin)."""
    q, k = _c(q, np.uint16).copy(), _c(k, np.uint16).copy()
    pos = _c(positions, np.int32)
    rc = _c(rope_cache, np.float32)
    t, nq, hd = q.shape
    rd = hd if rotary_dim is None else rotary_dim
    load().orc_rope(_p(q), _p(k), _p(pos), _p(rc), t, nq, k.shape[1], hd, rd, rc.shape[0])
    return q, k


def qkv_prologue(qkv, q_norm_w, k_norm_w, positions, rope_cache, slot_mapping, k_cache,
                 v_cache, nq: int, nkv: int, hd: int, eps: float, max_slots=None):
    """The fused prologue; returns q_out [T, nq, hd] and updates k_cache / v_cache in place."""
    x = _c(qkv, np.uint16)
    t = x.shape[0]
    qw = None if q_norm_w is None else _c(q_norm_w, np.uint16)
    kw = None if k_norm_w is None else _c(k_norm_w, np.uint16)
    pos = _c(positions, np.int32)
    rc = _c(rope_cache, np.float32)
    sm = _c(slot_mapping, np.int32)
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    q_out = np.empty((t, nq, hd), np.uint16)
    kt = np.empty((t, nkv, hd), np.uint16)
    vt = np.empty((t, nkv, hd), np.uint16)
    load().orc_qkv_prologue(_p(x), None if qw is None else _p(qw), None if kw is None else _p(kw),
                            _p(pos), _p(rc), _p(sm), _p(q_out), _p(kt), _p(vt), _p(k_cache),
                            _p(v_cache), t, nq, nkv, hd, rc.shape[0],
                            k_cache.shape[0] if max_slots is None else max_slots, eps)
    return q_out


def rope_cache_table(max_position: int, rotary_dim: int, theta: float) -> np.ndarray:
    """(cos, sin) table [max_position, rotary_dim / 2, 2] float32, computed in float32 as the
    reference builds it (src/model/rope/rope_cache.cpp:29-44)."""
    half = rotary_dim // 2
    pairs = np.arange(half, dtype=np.float32)
    inv = (np.float32(1.0) / np.power(np.float32(theta),
                                      pairs * np.float32(2) / np.float32(rotary_dim))).astype(np.float32)
    ang = (np.arange(max_position, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)


# ---- per-step batch metadata (block table, slot mapping, positions, ...) ----

ITEM_DECODE = 1
ITEM_SAMPLE = 2


def build_batch_metadata(kv_written, new_tokens, flags, block_start, blocks, num_tokens: int,
                         max_blocks_per_req: int, block_size: int, num_cache_blocks: int):
    """Returns (status, dict of int32 arrays) -- the arrays BatchTranslator builds on the host."""
    kvw = _c(kv_written, np.int32)
    nt = _c(new_tokens, np.int32)
    fl = _c(flags, np.int32)
    bst = _c(block_start, np.int32)
    blk = _c(blocks, np.int32) if len(blocks) else np.zeros(1, np.int32)
    b = kvw.shape[0]
    out = {
        "positions": np.full(max(num_tokens, 1), -7, np.int32),
        "slot_mapping": np.full(max(num_tokens, 1), -7, np.int32),
        "block_table": np.full((b, max_blocks_per_req), -7, np.int32),
        "query_start_loc": np.full(b + 1, -7, np.int32),
        "context_lens": np.full(b, -7, np.int32),
        "logits_indices": np.full(b, -7, np.int32),
    }
    st = load().orc_build_batch_metadata(
        _p(kvw), _p(nt), _p(fl), _p(bst), _p(blk), b, num_tokens, len(blocks), max_blocks_per_req,
        block_size, num_cache_blocks, _p(out["positions"]), _p(out["slot_mapping"]),
        _p(out["block_table"]), _p(out["query_start_loc"]), _p(out["context_lens"]),
        _p(out["logits_indices"]))
    out["positions"] = out["positions"][:num_tokens]
    out["slot_mapping"] = out["slot_mapping"][:num_tokens]
    return int(st), out


# ---- fp8 (OCP E4M3) KV cache with one fp32 scale per cache row ----

def fp8_scale_index(slot, kv_head, num_kv_heads: int, block_size: int = 16):
    slot = np.asarray(slot, np.int64)
    return ((slot // block_size) * num_kv_heads + kv_head) * block_size + slot % block_size


def f32_to_e4m3(x) -> np.ndarray:
    lib = load()
    x = np.asarray(x, np.float32)
    return np.array([lib.orc_f32_to_e4m3(float(v)) for v in x.ravel()], np.uint8).reshape(x.shape)


def e4m3_to_f32(b) -> np.ndarray:
    lib = load()
    b = np.asarray(b, np.uint8)
    return np.array([lib.orc_e4m3_to_f32(int(v)) for v in b.ravel()], np.float32).reshape(b.shape)


def write_kv_cache_fp8(k_new, v_new, k_cache, v_cache, k_scale, v_scale, slot_mapping,
                       max_slots=None, block_size: int = 16) -> None:
    """In place: k_cache/v_cache uint8 [slots, Hkv, D]; k_scale/v_scale float32 [slots*Hkv]."""
    k, v = _c(k_new, np.uint16), _c(v_new, np.uint16)
    sm = _c(slot_mapping, np.int32)
    for a in (k_cache, v_cache, k_scale, v_scale):
        assert a.flags.c_contiguous
    t, hkv, d = k.shape
    load().orc_write_kv_cache_fp8(_p(k), _p(v), _p(k_cache), _p(v_cache), _p(k_scale),
                                  _p(v_scale), _p(sm), t, hkv, d,
                                  k_cache.shape[0] if max_slots is None else max_slots,
                                  block_size)


def decode_fp8(q, k_cache, v_cache, k_scale, v_scale, block_table, context_lens,
               block_size: int = 16, nthreads=None) -> np.ndarray:
    """fp32 [B, Hq, D] over the fp8 cache."""
    q = _c(q, np.uint16)
    b, hq, d = q.shape
    bt = _c(block_table, np.int32)
    out = np.zeros((b, hq, d), np.float32)
    load().orc_decode_attention_fp8(
        _p(q), _p(_c(k_cache, np.uint8)), _p(_c(v_cache, np.uint8)), _p(_c(k_scale, np.float32)),
        _p(_c(v_scale, np.float32)), _p(bt), _p(_c(context_lens, np.int32)), _p(out), b,
        bt.shape[1], hq, k_cache.shape[1], d, block_size, nthreads or default_threads())
    return out


def prefill_fp8(q, k_cache, v_cache, k_scale, v_scale, block_table, query_start_loc,
                context_lens, block_size: int = 16, nthreads=None, out=None) -> np.ndarray:
    """fp32 [T, Hq, D] over the fp8 cache; rows the reference leaves unwritten keep `out`."""
    q = _c(q, np.uint16)
    t, hq, d = q.shape
    bt = _c(block_table, np.int32)
    qsl = _c(query_start_loc, np.int32)
    res = np.zeros((t, hq, d), np.float32) if out is None else _c(out, np.float32).copy()
    load().orc_prefill_attention_fp8(
        _p(q), _p(_c(k_cache, np.uint8)), _p(_c(v_cache, np.uint8)), _p(_c(k_scale, np.float32)),
        _p(_c(v_scale, np.float32)), _p(bt), _p(qsl), _p(_c(context_lens, np.int32)), _p(res),
        qsl.shape[0] - 1, t, bt.shape[1], hq, k_cache.shape[1], d, block_size,
        nthreads or default_threads())
    return res
