"""Decode-path modules: int8 linear, paged KV pool, paged-attention decode, HF hook and cache adapters."""

from .int8_linear import Int8Linear, int8_linear, pack_weight, quantize_model_, quantize_weight
from .paged_attention_hip import (
    PagedDecodeBatchMetadata,
    PagedDecodeContext,
    get_paged_decode_batch_metadata,
    get_paged_decode_context,
    hip_kernel_available,
    paged_attention_decode,
    paged_attention_decode_batched,
    reference_sdpa_attention,
    reset_paged_decode_batch_metadata,
    set_paged_decode_batch_metadata,
    set_paged_decode_context,
    warmup_paged_attention_kernel,
)
from .paged_kv_kernel import GpuKVBlockPool, PoolShape

__all__ = [
    "GpuKVBlockPool",
    "Int8Linear",
    "PagedDecodeBatchMetadata",
    "PagedDecodeContext",
    "PoolShape",
    "get_paged_decode_batch_metadata",
    "get_paged_decode_context",
    "hip_kernel_available",
    "int8_linear",
    "pack_weight",
    "paged_attention_decode",
    "paged_attention_decode_batched",
    "quantize_model_",
    "quantize_weight",
    "reference_sdpa_attention",
    "reset_paged_decode_batch_metadata",
    "set_paged_decode_batch_metadata",
    "set_paged_decode_context",
    "warmup_paged_attention_kernel",
]
