"""Transformers attention hook: HIP paged decode when q_len == 1.

Same contract as the reference hook (``runtime/phase2/block_paged_attention.py:24-60``):
registered as ``ALL_ATTENTION_FUNCTIONS["block_paged"]`` with
``config._attn_implementation = "block_paged"`` (``runtime/phase2/worker_server.py:274-281``).
When decode metadata is set, ``q_len == 1`` and the query is on a device, the
fused HIP kernel runs and ``[B, 1, Hq, D]`` is returned (``:37-48``); otherwise
eager attention on the gathered K/V (prefill, ``:50-60``).

Difference kept on purpose: transformers 5.x hands a custom attention
implementation that has no registered mask function ``attention_mask=None``
(``masking_utils._preprocess_mask_arguments`` returns early for it), so the
reference's eager branch, which only adds a mask when one is given, attends
bidirectionally during prefill. Here a missing mask with ``q_len > 1`` is
replaced by the causal mask (query ``i`` sees keys ``0 .. kv_len - q_len + i``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .paged_attention_hip import get_paged_decode_batch_metadata, paged_attention_decode_batched


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    if n_rep == 1:
        return hidden_states
    batch, num_key_value_heads, slen, head_dim = hidden_states.shape
    hidden_states = hidden_states[:, :, None, :, :].expand(batch, num_key_value_heads, n_rep, slen, head_dim)
    return hidden_states.reshape(batch, num_key_value_heads * n_rep, slen, head_dim)


def _causal_block(q_len: int, kv_len: int, device: torch.device) -> torch.Tensor:
    """``True`` where query ``i`` (the last ``q_len`` of ``kv_len`` positions) must not see key ``j``."""
    qpos = torch.arange(kv_len - q_len, kv_len, device=device).view(-1, 1)
    return torch.arange(kv_len, device=device).view(1, -1) > qpos


def block_paged_attention_forward(module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                  attention_mask: torch.Tensor | None, scaling: float, dropout: float = 0.0, **kwargs):
    num_kv_groups = getattr(module, "num_key_value_groups", 1)
    meta = get_paged_decode_batch_metadata()
    if meta is not None and query.shape[-2] == 1 and query.is_cuda:
        attn_output = paged_attention_decode_batched(query=query, metadata=meta, num_kv_groups=num_kv_groups,
                                                     scaling=scaling)
        return attn_output.transpose(1, 2).contiguous(), None

    key_states = repeat_kv(key, num_kv_groups)
    value_states = repeat_kv(value, num_kv_groups)
    attn_weights = torch.matmul(query, key_states.transpose(2, 3).contiguous()) * scaling
    if attention_mask is not None:
        attn_weights = attn_weights + attention_mask
    elif query.shape[-2] > 1:
        attn_weights = attn_weights.masked_fill(_causal_block(query.shape[-2], key.shape[-2], query.device),
                                                float("-inf"))
    attn_weights = F.softmax(attn_weights, dim=-1, dtype=torch.float32).to(query.dtype)
    if dropout > 0.0 and module.training:
        attn_weights = F.dropout(attn_weights, p=dropout)
    attn_output = torch.matmul(attn_weights, value_states)
    return attn_output.transpose(1, 2).contiguous(), attn_weights


def register_block_paged_attention() -> None:
    """``ALL_ATTENTION_FUNCTIONS.register("block_paged", ...)`` as ``worker_server.py:274-281`` does."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    ALL_ATTENTION_FUNCTIONS.register("block_paged", block_paged_attention_forward)
