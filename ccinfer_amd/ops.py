"""Torch-facing operators over the C ABI, mirroring the reference's backend ops.

Reference interface: DeviceBackend::{write_kv_cache, decode_attention, prefill_attention}
(plus qkv_prologue, one launch for split_qkv + rms_norm + rope + write_kv_cache, and
build_batch_metadata, BatchTranslator's per-step arrays built on the device, and an fp8
KV cache: write_kv_cache_fp8 / decode_attention_fp8)
(src/backend/backend.h:172-223) with the parameter structs of src/backend/params.h:148-211.
Argument names, meaning and error behaviour follow it: invalid arguments raise
CcinferError with code ErrorCode::InvalidArgument (6), the same value the reference returns.

Tensors are device tensors (torch on ROCm: "cuda" is the HIP device). Layouts:
  q, output (decode)   [batch, num_q_heads, head_dim]            bf16
  q, output (prefill)  [total_query_tokens, num_q_heads, head_dim] bf16
  k_cache, v_cache     [num_slots, num_kv_heads, head_dim] bf16 (one layer), or
                       [num_blocks, block_size, num_kv_heads, head_dim]
  block_table          [batch, max_blocks_per_req] int32, -1 padded
  context_lens         [batch] int32; query_start_loc [batch + 1] int32
  slot_mapping         [total_tokens] int32
Work is enqueued on torch's current stream; workspaces come from torch's caching
allocator unless passed in (scratch: no initialisation needed).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

INVALID_ARGUMENT = 6


class CcinferError(RuntimeError):
    """A non-zero status from the C ABI (value of the reference's ErrorCode)."""

    def __init__(self, code: int, op: str):
        msg = _lib.load().ccinfer_error_message(code).decode()
        super().__init__(f"{op}: {msg} (code {code})")
        self.code = code


def _check(code: int, op: str) -> None:
    if code != 0:
        raise CcinferError(code, op)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require(cond: bool, op: str) -> None:
    if not cond:
        raise CcinferError(INVALID_ARGUMENT, op)


def _dev_tensor(t: Optional[torch.Tensor], dtype: torch.dtype, op: str) -> None:
    _require(t is not None and t.is_cuda and t.dtype == dtype and t.is_contiguous(), op)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class SideStream:
    """A side stream with its fork/join events, for prefill_attention(..., overlap=...): a
    mixed batch's decode items then run there beside the prompt tiles. Owned by the caller
    (the library keeps no streams); one per concurrent caller."""

    def __init__(self, device=None):
        self.stream = torch.cuda.Stream(device=device)
        self.fork = torch.cuda.Event()
        self.join = torch.cuda.Event()
        # torch creates an event on its first record
        self.fork.record(self.stream)
        self.join.record(self.stream)

    def handles(self):
        return self.stream.cuda_stream, self.fork.cuda_event, self.join.cuda_event


def _kv_shape(k_cache: torch.Tensor):
    """(num_slots, num_kv_heads, head_dim) of a 3-D or 4-D cache tensor."""
    if k_cache.dim() == 4:
        nb, bs, h, d = k_cache.shape
        return nb * bs, h, d
    s, h, d = k_cache.shape
    return s, h, d


def write_kv_cache(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                   v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                   max_slots: Optional[int] = None) -> None:
    """cache[slot_mapping[t]] = new[t] for K and V (write_kv_cache.cu:12-34)."""
    op = "write_kv_cache"
    for t in (k_new, v_new, k_cache, v_cache):
        _dev_tensor(t, torch.bfloat16, op)
    _dev_tensor(slot_mapping, torch.int32, op)
    slots, hkv, d = _kv_shape(k_cache)
    _require(k_new.shape[-2:] == (hkv, d) and v_new.shape == k_new.shape, op)
    _require(v_cache.numel() == k_cache.numel(), op)
    total = k_new.numel() // (hkv * d)
    _require(slot_mapping.numel() == total, op)
    lib = _lib.load()
    _check(lib.ccinfer_write_kv_cache(_ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache),
                                      _ptr(slot_mapping), total, hkv, d,
                                      slots if max_slots is None else max_slots, _stream()), op)


def qkv_prologue(qkv: torch.Tensor, q_norm_weight: Optional[torch.Tensor],
                 k_norm_weight: Optional[torch.Tensor], positions: torch.Tensor,
                 rope_cache: torch.Tensor, slot_mapping: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, num_q_heads: int, eps: float = 1e-6,
                 q_out: Optional[torch.Tensor] = None,
                 max_slots: Optional[int] = None) -> torch.Tensor:
    """One launch for the per-layer attention prologue of src/model/qwen3/qwen3_model.cpp:
    174-244: split_qkv, rms_norm of q and k (skipped for a None weight), rope with
    rotary_dim = head_dim, write_kv_cache. Returns q [num_tokens, num_q_heads, head_dim].

    qkv [num_tokens, (num_q_heads + 2 num_kv_heads) * head_dim] bf16; rope_cache
    [max_position, head_dim / 2, 2] float32 (cos, sin); num_kv_heads and head_dim come from
    k_cache."""
    op = "qkv_prologue"
    for t in (qkv, k_cache, v_cache):
        _dev_tensor(t, torch.bfloat16, op)
    for t in (q_norm_weight, k_norm_weight):
        if t is not None:
            _dev_tensor(t, torch.bfloat16, op)
    _dev_tensor(positions, torch.int32, op)
    _dev_tensor(slot_mapping, torch.int32, op)
    _dev_tensor(rope_cache, torch.float32, op)
    slots, hkv, d = _kv_shape(k_cache)
    _require(v_cache.numel() == k_cache.numel() and num_q_heads > 0, op)
    width = (num_q_heads + 2 * hkv) * d
    _require(qkv.numel() % width == 0 and qkv.shape[-1] == width, op)
    tokens = qkv.numel() // width
    _require(positions.numel() == tokens and slot_mapping.numel() == tokens, op)
    for w in (q_norm_weight, k_norm_weight):
        _require(w is None or w.numel() == d, op)
    _require(rope_cache.dim() >= 2 and rope_cache.numel() % d == 0, op)
    max_pos = rope_cache.numel() // d
    if q_out is None:
        q_out = torch.empty(tokens, num_q_heads, d, dtype=torch.bfloat16, device=qkv.device)
    else:
        _dev_tensor(q_out, torch.bfloat16, op)
        _require(q_out.numel() == tokens * num_q_heads * d, op)
    lib = _lib.load()
    _check(lib.ccinfer_qkv_prologue(_ptr(qkv), _ptr(q_norm_weight), _ptr(k_norm_weight),
                                    _ptr(positions), _ptr(rope_cache), _ptr(slot_mapping),
                                    _ptr(q_out), _ptr(k_cache), _ptr(v_cache), tokens,
                                    num_q_heads, hkv, d, max_pos,
                                    slots if max_slots is None else max_slots, float(eps),
                                    _stream()), op)
    return q_out


ITEM_DECODE = 1  # decode item: one new token, always sampled
ITEM_SAMPLE = 2  # prefill chunk whose last token needs logits


def build_batch_metadata(item_kv_written: torch.Tensor, item_new_tokens: torch.Tensor,
                         item_flags: torch.Tensor, item_block_start: torch.Tensor,
                         blocks: torch.Tensor, num_tokens: int, max_blocks_per_req: int,
                         num_cache_blocks: int, block_size: int = 16,
                         out: Optional[dict] = None) -> dict:
    """One step's attention metadata built on the device (the arrays of
    src/worker/batch_translator.cpp:213-302 and the checks of src/model/model_runner.h:
    102-171). Returns int32 device tensors positions, slot_mapping, block_table,
    query_start_loc, context_lens, logits_indices and status ([1]: 0 or 6). Nothing is
    synchronised: read `status` when the result is needed. `out` reuses tensors of an
    earlier call with the same shapes."""
    op = "build_batch_metadata"
    for t in (item_kv_written, item_new_tokens, item_flags, item_block_start, blocks):
        _dev_tensor(t, torch.int32, op)
    b = item_kv_written.numel()
    _require(b > 0 and item_new_tokens.numel() == b and item_flags.numel() == b, op)
    _require(item_block_start.numel() == b + 1, op)
    dev = item_kv_written.device
    shapes = {"positions": (num_tokens,), "slot_mapping": (num_tokens,),
              "block_table": (b, max_blocks_per_req), "query_start_loc": (b + 1,),
              "context_lens": (b,), "logits_indices": (b,), "status": (1,)}
    if out is None:
        out = {k: torch.empty(v, dtype=torch.int32, device=dev) for k, v in shapes.items()}
    for k, v in shapes.items():
        _dev_tensor(out[k], torch.int32, op)
        _require(tuple(out[k].shape) == v, op)
    lib = _lib.load()
    _check(lib.ccinfer_build_batch_metadata(
        _ptr(item_kv_written), _ptr(item_new_tokens), _ptr(item_flags), _ptr(item_block_start),
        _ptr(blocks) if blocks.numel() else None, b, num_tokens, blocks.numel(),
        max_blocks_per_req, block_size, num_cache_blocks, _ptr(out["positions"]),
        _ptr(out["slot_mapping"]), _ptr(out["block_table"]), _ptr(out["query_start_loc"]),
        _ptr(out["context_lens"]), _ptr(out["logits_indices"]), _ptr(out["status"]),
        _stream()), op)
    return out


def decode_workspace_size(batch_size: int, max_blocks_per_req: int, num_q_heads: int,
                          num_kv_heads: int, head_dim: int, cache_block_size: int = 16) -> int:
    return int(_lib.load().ccinfer_decode_workspace_size(
        batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim, cache_block_size))


def prefill_workspace_size(batch_size: int, total_query_tokens: int, max_blocks_per_req: int,
                           num_q_heads: int, num_kv_heads: int, head_dim: int,
                           cache_block_size: int = 16) -> int:
    return int(_lib.load().ccinfer_prefill_workspace_size(
        batch_size, total_query_tokens, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim,
        cache_block_size))


def _workspace(nbytes: int, device, workspace: Optional[torch.Tensor]):
    if nbytes == 0:
        return None, 0
    if workspace is not None:
        _require(workspace.is_cuda and workspace.numel() * workspace.element_size() >= nbytes,
                 "workspace")
        return workspace, workspace.numel() * workspace.element_size()
    return torch.zeros(nbytes, dtype=torch.uint8, device=device), nbytes


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     block_table: torch.Tensor, context_lens: torch.Tensor,
                     output: Optional[torch.Tensor] = None, cache_block_size: int = 16,
                     workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Paged decode attention (decode_attn.cu:364-473 semantics); returns output."""
    op = "decode_attention"
    for t in (q, k_cache, v_cache):
        _dev_tensor(t, torch.bfloat16, op)
    _dev_tensor(block_table, torch.int32, op)
    _dev_tensor(context_lens, torch.int32, op)
    _require(q.dim() == 3 and block_table.dim() == 2, op)
    b, hq, d = q.shape
    _, hkv, dk = _kv_shape(k_cache)
    _require(dk == d and block_table.shape[0] == b and context_lens.numel() == b, op)
    if output is None:
        output = torch.empty_like(q)
    _dev_tensor(output, torch.bfloat16, op)
    _require(output.shape == q.shape, op)
    mbpr = block_table.shape[1]
    need = decode_workspace_size(b, mbpr, hq, hkv, d, cache_block_size)
    ws, ws_bytes = _workspace(need, q.device, workspace)
    _check(_lib.load().ccinfer_decode_attention(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_table), _ptr(context_lens),
        _ptr(output), b, mbpr, hq, hkv, d, cache_block_size, _ptr(ws), ws_bytes, _stream()), op)
    return output


def decode_shared_workspace_size(batch_size: int, max_blocks_per_req: int, num_q_heads: int,
                                 num_kv_heads: int, head_dim: int,
                                 cache_block_size: int = 16) -> int:
    return int(_lib.load().ccinfer_decode_shared_workspace_size(
        batch_size, max_blocks_per_req, num_q_heads, num_kv_heads, head_dim, cache_block_size))


def decode_attention_shared_prefix(q: torch.Tensor, k_cache: torch.Tensor,
                                   v_cache: torch.Tensor, block_table: torch.Tensor,
                                   context_lens: torch.Tensor,
                                   output: Optional[torch.Tensor] = None,
                                   cache_block_size: int = 16,
                                   workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """decode_attention for a batch whose requests may share cached prompt prefixes (equal
    leading block ids): each group's common prefix is read once per MFMA tile of requests.
    Same semantics as decode_attention; returns output."""
    op = "decode_attention_shared_prefix"
    for t in (q, k_cache, v_cache):
        _dev_tensor(t, torch.bfloat16, op)
    _dev_tensor(block_table, torch.int32, op)
    _dev_tensor(context_lens, torch.int32, op)
    _require(q.dim() == 3 and block_table.dim() == 2, op)
    b, hq, d = q.shape
    _, hkv, dk = _kv_shape(k_cache)
    _require(dk == d and block_table.shape[0] == b and context_lens.numel() == b, op)
    if output is None:
        output = torch.empty_like(q)
    _dev_tensor(output, torch.bfloat16, op)
    _require(output.shape == q.shape, op)
    mbpr = block_table.shape[1]
    need = decode_shared_workspace_size(b, mbpr, hq, hkv, d, cache_block_size)
    ws, ws_bytes = _workspace(need, q.device, workspace)
    _check(_lib.load().ccinfer_decode_attention_shared_prefix(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_table), _ptr(context_lens),
        _ptr(output), b, mbpr, hq, hkv, d, cache_block_size, _ptr(ws), ws_bytes, _stream()), op)
    return output


def decode_attention_write_kv(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                              k_cache: torch.Tensor, v_cache: torch.Tensor,
                              block_table: torch.Tensor, context_lens: torch.Tensor,
                              output: Optional[torch.Tensor] = None, cache_block_size: int = 16,
                              workspace: Optional[torch.Tensor] = None,
                              max_slots: Optional[int] = None) -> torch.Tensor:
    """One decode step: write_kv_cache of each request's new token k_new[b] / v_new[b]
    ([B, Hkv, D]) into the slot of its last position (context_lens[b] - 1, through its table
    row), then decode_attention (write_kv_cache.cu:12-34 + decode_attn.cu:364-473
    semantics, in one launch on the MFMA path). Returns output."""
    op = "decode_attention_write_kv"
    for t in (q, k_new, v_new, k_cache, v_cache):
        _dev_tensor(t, torch.bfloat16, op)
    _dev_tensor(block_table, torch.int32, op)
    _dev_tensor(context_lens, torch.int32, op)
    _require(q.dim() == 3 and block_table.dim() == 2, op)
    b, hq, d = q.shape
    slots, hkv, dk = _kv_shape(k_cache)
    _require(dk == d and block_table.shape[0] == b and context_lens.numel() == b, op)
    _require(k_new.shape == (b, hkv, d) and v_new.shape == k_new.shape, op)
    if output is None:
        output = torch.empty_like(q)
    _dev_tensor(output, torch.bfloat16, op)
    _require(output.shape == q.shape, op)
    mbpr = block_table.shape[1]
    need = decode_workspace_size(b, mbpr, hq, hkv, d, cache_block_size)
    ws, ws_bytes = _workspace(need, q.device, workspace)
    _check(_lib.load().ccinfer_decode_attention_write_kv(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), _ptr(block_table),
        _ptr(context_lens), _ptr(output), b, mbpr, hq, hkv, d, cache_block_size,
        slots if max_slots is None else max_slots, _ptr(ws), ws_bytes, _stream()), op)
    return output


def fp8_scale_numel(max_slots: int, num_kv_heads: int, block_size: int = 16) -> int:
    """Floats in each scale array of an fp8 cache of `max_slots` slots."""
    return -(-max_slots // block_size) * block_size * num_kv_heads


def write_kv_cache_fp8(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, k_scale: torch.Tensor, v_scale: torch.Tensor,
                       slot_mapping: torch.Tensor, max_slots: Optional[int] = None) -> None:
    """write_kv_cache into an fp8 (OCP E4M3) cache with one fp32 scale per cache row (the
    smallest power of two P with max|row| <= 448 P; the row is stored as e4m3(row / P)).
    k_cache / v_cache: uint8 [slots, Hkv, D] (or [blocks, 16, Hkv, D]); scales: float32 of
    fp8_scale_numel(slots, Hkv) elements."""
    op = "write_kv_cache_fp8"
    for t in (k_new, v_new):
        _dev_tensor(t, torch.bfloat16, op)
    for t in (k_cache, v_cache):
        _dev_tensor(t, torch.uint8, op)
    for t in (k_scale, v_scale):
        _dev_tensor(t, torch.float32, op)
    _dev_tensor(slot_mapping, torch.int32, op)
    slots, hkv, d = _kv_shape(k_cache)
    _require(k_new.shape[-2:] == (hkv, d) and v_new.shape == k_new.shape, op)
    _require(v_cache.numel() == k_cache.numel(), op)
    _require(min(k_scale.numel(), v_scale.numel()) >= fp8_scale_numel(slots, hkv), op)
    total = k_new.numel() // (hkv * d)
    _require(slot_mapping.numel() == total, op)
    _check(_lib.load().ccinfer_write_kv_cache_fp8(
        _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
        _ptr(slot_mapping), total, hkv, d, slots if max_slots is None else max_slots,
        _stream()), op)


def decode_attention_fp8(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                         k_scale: torch.Tensor, v_scale: torch.Tensor,
                         block_table: torch.Tensor, context_lens: torch.Tensor,
                         output: Optional[torch.Tensor] = None, cache_block_size: int = 16,
                         workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """decode_attention over an fp8 cache written by write_kv_cache_fp8."""
    op = "decode_attention_fp8"
    _dev_tensor(q, torch.bfloat16, op)
    for t in (k_cache, v_cache):
        _dev_tensor(t, torch.uint8, op)
    for t in (k_scale, v_scale):
        _dev_tensor(t, torch.float32, op)
    _dev_tensor(block_table, torch.int32, op)
    _dev_tensor(context_lens, torch.int32, op)
    _require(q.dim() == 3 and block_table.dim() == 2, op)
    b, hq, d = q.shape
    slots, hkv, dk = _kv_shape(k_cache)
    _require(dk == d and block_table.shape[0] == b and context_lens.numel() == b, op)
    _require(min(k_scale.numel(), v_scale.numel()) >= fp8_scale_numel(slots, hkv), op)
    if output is None:
        output = torch.empty_like(q)
    _dev_tensor(output, torch.bfloat16, op)
    _require(output.shape == q.shape, op)
    mbpr = block_table.shape[1]
    need = decode_workspace_size(b, mbpr, hq, hkv, d, cache_block_size)
    ws, ws_bytes = _workspace(need, q.device, workspace)
    _check(_lib.load().ccinfer_decode_attention_fp8(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_table),
        _ptr(context_lens), _ptr(output), b, mbpr, hq, hkv, d, cache_block_size, _ptr(ws),
        ws_bytes, _stream()), op)
    return output


def prefill_attention_fp8(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                          k_scale: torch.Tensor, v_scale: torch.Tensor,
                          block_table: torch.Tensor, query_start_loc: torch.Tensor,
                          context_lens: torch.Tensor, output: Optional[torch.Tensor] = None,
                          cache_block_size: int = 16,
                          workspace: Optional[torch.Tensor] = None,
                          overlap: Optional[SideStream] = None) -> torch.Tensor:
    """prefill_attention over an fp8 cache written by write_kv_cache_fp8."""
    op = "prefill_attention_fp8"
    _dev_tensor(q, torch.bfloat16, op)
    for t in (k_cache, v_cache):
        _dev_tensor(t, torch.uint8, op)
    for t in (k_scale, v_scale):
        _dev_tensor(t, torch.float32, op)
    for t in (block_table, query_start_loc, context_lens):
        _dev_tensor(t, torch.int32, op)
    _require(q.dim() == 3 and block_table.dim() == 2, op)
    total, hq, d = q.shape
    slots, hkv, dk = _kv_shape(k_cache)
    b = block_table.shape[0]
    _require(dk == d and query_start_loc.numel() == b + 1 and context_lens.numel() == b, op)
    _require(min(k_scale.numel(), v_scale.numel()) >= fp8_scale_numel(slots, hkv), op)
    if output is None:
        output = torch.empty_like(q)
    _dev_tensor(output, torch.bfloat16, op)
    _require(output.shape == q.shape, op)
    mbpr = block_table.shape[1]
    need = prefill_workspace_size(b, total, mbpr, hq, hkv, d, cache_block_size)
    ws, ws_bytes = _workspace(need, q.device, workspace)
    args = (_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
            _ptr(block_table), _ptr(query_start_loc), _ptr(context_lens), _ptr(output), b, total,
            mbpr, hq, hkv, d, cache_block_size, _ptr(ws), ws_bytes, _stream())
    if overlap is None:
        _check(_lib.load().ccinfer_prefill_attention_fp8(*args), op)
    else:
        _check(_lib.load().ccinfer_prefill_attention_fp8_overlap(*args, *overlap.handles()), op)
    return output


def prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      block_table: torch.Tensor, query_start_loc: torch.Tensor,
                      context_lens: torch.Tensor, output: Optional[torch.Tensor] = None,
                      cache_block_size: int = 16,
                      workspace: Optional[torch.Tensor] = None,
                      overlap: Optional[SideStream] = None) -> torch.Tensor:
    """Paged causal prefill attention (prefill_attn.cu:43-242 semantics); returns output.

    Rows the reference leaves unwritten (requests with context_len < query_len) keep the
    contents of `output` (uninitialised when `output` is None). With `overlap`, a mixed
    batch's decode items run on its side stream beside the prompt tiles.
    """
    op = "prefill_attention"
    for t in (q, k_cache, v_cache):
        _dev_tensor(t, torch.bfloat16, op)
    for t in (block_table, query_start_loc, context_lens):
        _dev_tensor(t, torch.int32, op)
    _require(q.dim() == 3 and block_table.dim() == 2, op)
    total, hq, d = q.shape
    _, hkv, dk = _kv_shape(k_cache)
    b = context_lens.numel()
    _require(dk == d and block_table.shape[0] == b and query_start_loc.numel() == b + 1, op)
    if output is None:
        output = torch.empty_like(q)
    _dev_tensor(output, torch.bfloat16, op)
    _require(output.shape == q.shape, op)
    mbpr = block_table.shape[1]
    need = prefill_workspace_size(b, total, mbpr, hq, hkv, d, cache_block_size)
    ws, ws_bytes = _workspace(need, q.device, workspace)
    args = (_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_table), _ptr(query_start_loc),
            _ptr(context_lens), _ptr(output), b, total, mbpr, hq, hkv, d, cache_block_size,
            _ptr(ws), ws_bytes, _stream())
    if overlap is None:
        _check(_lib.load().ccinfer_prefill_attention(*args), op)
    else:
        _check(_lib.load().ccinfer_prefill_attention_overlap(*args, *overlap.handles()), op)
    return output
