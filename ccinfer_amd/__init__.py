"""MI355X (gfx950) paged-attention hot path of ccInfer: HIP kernels behind a C ABI.

The product is libccinfer_attn.so (built in-tree by ccinfer_amd.build). This package is the
Python host side: a ctypes binding of the C ABI (`_lib`), torch-facing operators that mirror
the reference's backend ops (`ops`), and seeded synthetic workloads (`workloads`).
"""
from .ops import (  # noqa: F401
    ITEM_DECODE,
    ITEM_SAMPLE,
    CcinferError,
    SideStream,
    build_batch_metadata,
    decode_attention,
    decode_attention_fp8,
    decode_attention_shared_prefix,
    decode_attention_write_kv,
    decode_shared_workspace_size,
    decode_workspace_size,
    prefill_attention,
    prefill_attention_fp8,
    prefill_workspace_size,
    qkv_prologue,
    write_kv_cache,
    write_kv_cache_fp8,
    fp8_scale_numel,
)

__all__ = [
    "ITEM_DECODE",
    "ITEM_SAMPLE",
    "CcinferError",
    "SideStream",
    "build_batch_metadata",
    "decode_attention",
    "decode_attention_fp8",
    "decode_attention_shared_prefix",
    "decode_attention_write_kv",
    "decode_shared_workspace_size",
    "decode_workspace_size",
    "prefill_attention",
    "prefill_attention_fp8",
    "prefill_workspace_size",
    "qkv_prologue",
    "write_kv_cache",
    "write_kv_cache_fp8",
    "fp8_scale_numel",
]
