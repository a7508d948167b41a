"""Greedy paged decode of an HF decoder through the block-paged cache and the HIP kernels.

The slice of ``TransformersBackend`` that drives the hot path
(``runtime/phase2/worker_server.py``):

* :func:`enable_block_paged_attention` — register the attention hook and switch
  the model to it (``:274-281``);
* :func:`prefill_request` — one request's prompt through a batch-1
  :class:`BlockPagedCache` (``:643-731``; mixed prompt lengths prefill one row at
  a time, as there, ``:685-692``), first token from the prefill logits;
* :func:`paged_decode_step` — one ragged batched decode forward over a
  :class:`BlockPagedBatchCache` and greedy argmax (``:733-794``);
* :func:`greedy_decode` — prefill every row, bind the rows into one batch
  cache (``BlockPagedBatchCache.from_caches``, ``:605-611``), then ``steps``
  decode steps.

One deliberate difference: the decode forward passes each row's own position
(``position_ids = seq_lens``) to the model. The reference passes none, so HF
derives one position for the whole batch from ``get_seq_length()``, the
*longest* row (``paged_kv_cache.py:406-407``), and rows shorter than the
longest get rotary phases of the wrong position. With equal lengths both agree.

Greedy tokens stay on the device until the caller reads them; a step makes the
host syncs HF's mask construction makes (``get_mask_sizes``) and no others.
"""

from __future__ import annotations

import torch

from .block_paged_attention import register_block_paged_attention
from .paged_attention_hip import set_paged_decode_batch_metadata
from .paged_kv_cache import BlockPagedBatchCache, BlockPagedCache
from .paged_kv_kernel import GpuKVBlockPool


def enable_block_paged_attention(model) -> None:
    """``ALL_ATTENTION_FUNCTIONS.register("block_paged", ...)`` + ``config._attn_implementation``."""
    register_block_paged_attention()
    model.config._attn_implementation = "block_paged"


@torch.no_grad()
def prefill_request(model, pool: GpuKVBlockPool, block_ids: list[int], input_ids: torch.Tensor
                    ) -> tuple[BlockPagedCache, torch.Tensor]:
    """Prefill one prompt ``input_ids [1, P]``; returns the filled cache and the last logits ``[1, V]``."""
    if input_ids.dim() != 2 or input_ids.shape[0] != 1:
        raise ValueError("prefill_request takes input_ids of shape [1, P]")
    cache = BlockPagedCache(model.config, pool)
    cache.set_block_ids(block_ids)
    try:
        out = model(input_ids=input_ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
    finally:
        set_paged_decode_batch_metadata(None)
    return cache, out.logits[:, -1, :]


@torch.no_grad()
def paged_decode_step(model, cache: BlockPagedBatchCache, input_ids: torch.Tensor) -> torch.Tensor:
    """One decode forward of ``input_ids [B, 1]`` at each row's own position; returns logits ``[B, V]``."""
    if input_ids.dim() != 2 or input_ids.shape[1] != 1 or input_ids.shape[0] != cache.block_tables.shape[0]:
        raise ValueError("paged_decode_step takes input_ids of shape [B, 1] matching the cache rows")
    positions = cache.seq_lens.to(torch.long).unsqueeze(1)
    try:
        out = model(input_ids=input_ids, position_ids=positions, past_key_values=cache, use_cache=True,
                    logits_to_keep=1)
    finally:
        set_paged_decode_batch_metadata(None)
    return out.logits[:, -1, :]


@torch.no_grad()
def greedy_decode(model, pool: GpuKVBlockPool, prompts: list[torch.Tensor], block_ids_rows: list[list[int]],
                  steps: int, keep_logits: bool = False):
    """Prefill each prompt, then ``steps`` batched greedy decode steps.

    Returns ``tokens [B, steps + 1]`` (the prefill token first) on the device,
    and, with ``keep_logits``, the fp32 logits ``[B, steps + 1, V]`` each token
    was chosen from.
    """
    if len(prompts) != len(block_ids_rows) or not prompts:
        raise ValueError("one block-id row per prompt is required")
    device = pool.device
    caches: list[BlockPagedCache] = []
    first_logits: list[torch.Tensor] = []
    for ids, blocks in zip(prompts, block_ids_rows):
        need = (int(ids.numel()) + steps + pool.block_size_tokens - 1) // pool.block_size_tokens
        if len(blocks) < need:
            raise ValueError(f"a row of {ids.numel()} prompt tokens and {steps} steps needs {need} blocks, "
                             f"got {len(blocks)}")
        cache, logits = prefill_request(model, pool, blocks, ids.view(1, -1).to(device))
        caches.append(cache)
        first_logits.append(logits)
    batch = BlockPagedBatchCache.from_caches(caches, pool)
    logits = torch.cat(first_logits, dim=0)
    tokens = [logits.argmax(dim=-1)]
    kept = [logits.float()] if keep_logits else []
    for _ in range(steps):
        logits = paged_decode_step(model, batch, tokens[-1].view(-1, 1))
        tokens.append(logits.argmax(dim=-1))
        if keep_logits:
            kept.append(logits.float())
    out_tokens = torch.stack(tokens, dim=1)
    if keep_logits:
        return out_tokens, torch.stack(kept, dim=1)
    return out_tokens
