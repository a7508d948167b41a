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
  decode steps;
* :class:`PagedDecoder` — the worker's persistent-slot sequence around the same
  forward (``_bind_states_to_persistent`` -> ``dense_active_cache`` -> model ->
  ``write_back_dense`` -> ``extract_cache``, ``:366-389,619-641,733-794``), with an
  optional HIP-graph replay of the step (``hip_graph_decode``).

One deliberate difference: the decode forward passes each row's own position
(``position_ids = seq_lens``) to the model. The reference passes none, so HF
derives one position for the whole batch from ``get_seq_length()``, the
*longest* row (``paged_kv_cache.py:406-407``), and rows shorter than the
longest get rotary phases of the wrong position. With equal lengths both agree.

Greedy tokens stay on the device until the caller reads them, and a decode
step makes no host sync: the custom attention implementation has no mask
function, so transformers builds no mask and never asks the cache for its
lengths, the positions are passed in, and the KV writes report table overruns
through the pool's device error word, which :func:`greedy_decode` checks once
after the prefill and once at the end (``GpuKVBlockPool.check_write_errors``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

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
    pool.check_write_errors()
    batch = BlockPagedBatchCache.from_caches(caches, pool)
    logits = torch.cat(first_logits, dim=0)
    tokens = [logits.argmax(dim=-1)]
    kept = [logits.float()] if keep_logits else []
    for _ in range(steps):
        logits = paged_decode_step(model, batch, tokens[-1].view(-1, 1))
        tokens.append(logits.argmax(dim=-1))
        if keep_logits:
            kept.append(logits.float())
    pool.check_write_errors()
    out_tokens = torch.stack(tokens, dim=1)
    if keep_logits:
        return out_tokens, torch.stack(kept, dim=1)
    return out_tokens


# ---------------------------------------------------------------------------------------------
# The worker's persistent-slot decode sequence (TransformersBackend, worker_server.py).
# ---------------------------------------------------------------------------------------------


@dataclass
class DecodeRequest:
    request_id: str


@dataclass
class DecodeState:
    """The fields of the worker's ``ActiveState`` (``worker_server.py:59-90``) that the paged
    decode step reads and writes."""

    req: DecodeRequest
    past_key_values: object
    last_token_id: int
    generated_token_ids: list[int] = field(default_factory=list)


class PagedDecoder:
    """Persistent decode slots and the ragged batched decode step of ``TransformersBackend``.

    * :meth:`ensure_persistent` — ``_ensure_paged_persistent`` (``worker_server.py:366-389``):
      one :class:`BlockPagedBatchCache` of at least ``max_active`` slots, grown (rows re-bound)
      when a batch needs more;
    * :meth:`bind_states_to_persistent` — ``:619-641``: a new request is bound to a free slot
      from its batch-1 cache; a bound one has its blocks and length re-synced;
    * :meth:`decode_step` — ``_paged_decode_step`` (``:733-794``): a captured graph when
      ``graph_mgr`` replays one; else one row decodes through its own
      :class:`BlockPagedCache` (the batch-1 ``BlockPagedLayer`` path) and several rows through
      ``dense_active_cache`` -> model -> ``write_back_dense`` -> ``extract_cache``; then greedy
      argmax (``:786-792``);
    * :meth:`release` — ``release_paged_request`` (``:361-364``).

    One difference, as in :func:`paged_decode_step`: the dense forward passes each row's own
    position (``position_ids = seq_lens``); the reference lets HF take one position for the
    whole batch from the longest row (``paged_kv_cache.py:406-407``).
    """

    def __init__(self, model, pool: GpuKVBlockPool, max_active: int = 8, graph_mgr=None) -> None:
        self.model = model
        self.kv_pool = pool
        self.max_active = int(max_active)
        self.graph_mgr = graph_mgr
        self._paged_persistent: BlockPagedBatchCache | None = None
        self._paged_persistent_capacity = 0
        self.last_logits: torch.Tensor | None = None  # [B, vocab] of the last step

    def ensure_persistent(self, min_batch: int, max_blocks: int) -> BlockPagedBatchCache:
        capacity = max(min_batch, self.max_active, 1)
        persistent = self._paged_persistent
        if persistent is None or self._paged_persistent_capacity < capacity:
            old = persistent
            persistent = BlockPagedBatchCache.empty(self.model.config, self.kv_pool, max_batch_size=capacity,
                                                    max_blocks=max(max_blocks, 1))
            if old is not None:
                for rid, old_slot in list(old._request_to_slot.items()):
                    new_slot = persistent.allocate_slot(rid)
                    persistent.sync_block_ids_row(new_slot, list(old.block_ids_rows[old_slot]))
                    persistent.seq_lens[new_slot] = old.seq_lens[old_slot]
            self._paged_persistent = persistent
            self._paged_persistent_capacity = capacity
        else:
            persistent.ensure_max_blocks(max_blocks)
        return persistent

    def bind_states_to_persistent(self, states: list[DecodeState]) -> BlockPagedBatchCache:
        max_blocks = 1
        for state in states:
            if isinstance(state.past_key_values, BlockPagedCache):
                max_blocks = max(max_blocks, len(state.past_key_values.block_table_ids) or 1)
        persistent = self.ensure_persistent(len(states), max_blocks)
        for state in states:
            rid = state.req.request_id
            cache = state.past_key_values
            if persistent.slot_of(rid) is None:
                if not isinstance(cache, BlockPagedCache):
                    raise TypeError("binding persistent slot requires BlockPagedCache")
                persistent.bind_cache(rid, cache)
            elif isinstance(cache, BlockPagedCache):
                slot = persistent.slot_of(rid)
                persistent.sync_block_ids_row(slot, list(cache.block_table_ids))
                persistent.seq_lens[slot] = int(cache.get_seq_length())
        return persistent

    def release(self, request_id: str) -> None:
        if self._paged_persistent is not None:
            self._paged_persistent.release_slot(request_id)

    @torch.no_grad()
    def decode_step(self, states: list[DecodeState]) -> list[int]:
        """One decode step of ``states``; appends and returns each row's greedy token."""
        device = self.kv_pool.device
        input_ids = torch.tensor([[s.last_token_id] for s in states], device=device)
        persistent = self.bind_states_to_persistent(states)
        logits_row = None
        if self.graph_mgr is not None:
            logits_row = self.graph_mgr.try_decode(persistent=persistent, decode_states=states, input_ids=input_ids)
        if logits_row is None:
            try:
                if len(states) == 1:
                    state = states[0]
                    out = self.model(input_ids=input_ids, past_key_values=state.past_key_values, use_cache=True)
                    if isinstance(out.past_key_values, BlockPagedCache):
                        state.past_key_values = out.past_key_values
                        self.bind_states_to_persistent([state])
                    logits_row = out.logits[:, -1, :]
                else:
                    dense, slots = persistent.dense_active_cache([s.req.request_id for s in states])
                    lens = [s.past_key_values.get_seq_length() for s in states]
                    out = self.model(input_ids=input_ids, position_ids=dense.seq_lens.to(torch.long).unsqueeze(1),
                                     past_key_values=dense, use_cache=True)
                    if isinstance(out.past_key_values, BlockPagedBatchCache):
                        dense = out.past_key_values
                    persistent.write_back_dense(dense, slots)
                    for idx, state in enumerate(states):
                        state.past_key_values = persistent.extract_cache(slots[idx], seq_len=lens[idx] + 1)
                    logits_row = out.logits[:, -1, :]
            finally:
                set_paged_decode_batch_metadata(None)
        self.last_logits = logits_row
        next_ids = logits_row.argmax(dim=-1).tolist()
        self.kv_pool.check_write_errors()
        for idx, state in enumerate(states):
            state.last_token_id = int(next_ids[idx])
            state.generated_token_ids.append(int(next_ids[idx]))
        return [int(t) for t in next_ids]
