"""Transformers ``Cache`` adapters over :class:`GpuKVBlockPool` for the HIP decode path.

Same classes, constructor arguments and methods as the reference's
``runtime/phase2/paged_kv_cache.py`` (``BlockPagedLayer`` ``:22-98``,
``BlockPagedBatchLayer`` ``:101-193``, ``BlockPagedCache`` ``:196-230``,
``BlockPagedBatchCache`` ``:233-431``), so the worker's prefill / bind / dense
decode / write-back sequence (``runtime/phase2/worker_server.py:605-794``) runs
unchanged on top of ``paged_attention_hip``.

Behaviour a decode layer relies on (``paged_kv_cache.py:44-82,121-170``):

* ``update`` writes the new K/V into the pool *before* attention, advances the
  row lengths, and for ``kv_len == 1`` publishes
  ``PagedDecodeBatchMetadata(pool, layer_idx, block_tables, seq_lens)`` with
  ``seq_lens`` counting the token just written; the attention hook then reads
  K/V from the pool and ignores the returned tensors;
* for ``kv_len > 1`` (prefill) it clears the metadata and returns the gathered
  ``[B, Hkv, S, D]`` K/V for eager attention;
* block tables are zero-padded past a row's blocks; the decode kernel bounds
  every row by ``ceil(seq_len / block_size)``.

Differences that keep the decode step free of host round trips:

* ``BlockPagedLayer`` keeps its block table and a one-element length tensor
  on the device and updates the length in place, so a decode step makes no
  host-to-device copies (the reference builds two ``torch.tensor`` per layer
  per step, ``:58-62,71-77``);
* the batched layer advances lengths in place whenever the parent is marked
  ``_graph_safe`` (as the reference's graph path does, ``:130-145``) and
  otherwise rebinds fresh tensors, as the reference's eager path does
  (``:146-157``).

transformers 5.15 makes ``get_max_length`` abstract; it returns the same value
as ``get_max_cache_shape`` (the capacity of the row's blocks).
"""

from __future__ import annotations

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from .paged_attention_hip import PagedDecodeBatchMetadata, set_paged_decode_batch_metadata
from .paged_kv_kernel import GpuKVBlockPool


def _decoder_layer_count(config) -> int:
    n_layers = int(config.num_hidden_layers)
    if hasattr(config, "num_kv_shared_layers"):
        n_layers -= int(config.num_kv_shared_layers)
    return n_layers


def _text_config(config):
    return config.get_text_config(decoder=True) if hasattr(config, "get_text_config") else config


def _table_row(block_ids: list[int], width: int, device: torch.device) -> torch.Tensor:
    row = torch.zeros(width, dtype=torch.int32)
    if block_ids:
        row[: len(block_ids)] = torch.tensor(block_ids, dtype=torch.int32)
    return row.to(device)


class BlockPagedLayer(CacheLayerMixin):
    """One layer of a batch-1 request cache over the shared pool (``paged_kv_cache.py:22-98``)."""

    is_compileable = False
    is_sliding = False

    def __init__(self, pool: GpuKVBlockPool, layer_idx: int) -> None:
        super().__init__()
        self.pool = pool
        self.layer_idx = layer_idx
        self._block_ids: list[int] = []
        self._block_table: torch.Tensor | None = None
        self._seq_len = 0
        self._seq_len_dev: torch.Tensor | None = None

    def set_block_ids(self, block_ids: list[int], block_table: torch.Tensor | None = None) -> None:
        self._block_ids = list(block_ids)
        self._block_table = block_table

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.dtype, self.device = key_states.dtype, key_states.device
        self.is_initialized = True

    def _table(self) -> torch.Tensor:
        if self._block_table is None:
            self._block_table = torch.tensor(self._block_ids, dtype=torch.int32).to(self.pool.device)
        return self._block_table

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if not self._block_ids:
            raise RuntimeError("BlockPagedLayer.update called before block_ids were assigned")
        if key_states.dim() == 3:
            key_states = key_states.unsqueeze(0)
            value_states = value_states.unsqueeze(0)
        kv_len = int(key_states.shape[-2])
        start = self._seq_len
        if start + kv_len > len(self._block_ids) * self.pool.block_size_tokens:
            raise IndexError(f"block table underrun: {start + kv_len} tokens in {len(self._block_ids)} blocks")
        table = self._table().view(1, -1)
        if self._seq_len_dev is None:
            self._seq_len_dev = torch.tensor([start], dtype=torch.int32).to(self.pool.device)
        self.pool.write_tokens_batch(self.layer_idx, table, self._seq_len_dev, key_states, value_states)
        self._seq_len += kv_len
        self._seq_len_dev.add_(kv_len)

        if kv_len == 1:
            set_paged_decode_batch_metadata(PagedDecodeBatchMetadata(
                pool=self.pool, layer_idx=self.layer_idx, block_tables=table, seq_lens=self._seq_len_dev))
            return key_states, value_states

        set_paged_decode_batch_metadata(None)
        return self.pool.gather_layer(self.layer_idx, self._block_ids, self._seq_len)

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self._seq_len + query_length, 0

    def get_seq_length(self) -> int:
        return self._seq_len

    def get_max_cache_shape(self) -> int:
        return len(self._block_ids) * self.pool.block_size_tokens

    def get_max_length(self) -> int:
        return self.get_max_cache_shape()

    def set_seq_length(self, seq_len: int) -> None:
        """Mark the row as filled through ``seq_len`` tokens (prefix hydration, ``worker_server.py:339-350``)."""
        self._seq_len = int(seq_len)
        self._seq_len_dev = None

    def reset(self) -> None:
        self._seq_len = 0
        self._seq_len_dev = None
        self._block_ids = []
        self._block_table = None
        self.is_initialized = False
        self.keys = None
        self.values = None


class BlockPagedBatchLayer(CacheLayerMixin):
    """One layer of a batched decode cache (``paged_kv_cache.py:101-193``).

    ``_row_seq_lens`` holds this layer's per-row lengths (int32, on the pool's
    device); every layer writes at its own lengths, and layer 0 publishes the
    advanced lengths to ``parent.seq_lens``, which the attention metadata of
    every layer of the step points at.
    """

    is_compileable = False
    is_sliding = False

    def __init__(self, pool: GpuKVBlockPool, layer_idx: int, parent: "BlockPagedBatchCache") -> None:
        super().__init__()
        self.pool = pool
        self.layer_idx = layer_idx
        self._parent = parent
        self._row_seq_lens = parent.seq_lens.clone()

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.dtype, self.device = key_states.dtype, key_states.device
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        parent = self._parent
        kv_len = int(key_states.shape[-2])
        parent.pool.write_tokens_batch(self.layer_idx, parent.block_tables, self._row_seq_lens, key_states,
                                       value_states)
        if getattr(parent, "_graph_safe", False):
            self._row_seq_lens.add_(kv_len)
            if self.layer_idx == 0:
                parent.seq_lens.copy_(self._row_seq_lens)
        else:
            self._row_seq_lens = self._row_seq_lens + kv_len
            if self.layer_idx == 0:
                parent.seq_lens = self._row_seq_lens.clone()

        if kv_len == 1:
            set_paged_decode_batch_metadata(PagedDecodeBatchMetadata(
                pool=self.pool, layer_idx=self.layer_idx, block_tables=parent.block_tables,
                seq_lens=parent.seq_lens))
            return key_states, value_states

        set_paged_decode_batch_metadata(None)
        return parent.pool.gather_layer_batch(self.layer_idx, parent.block_tables, parent.seq_lens)

    def _cached_length(self) -> int | None:
        if getattr(self._parent, "_graph_safe", False):
            cached = getattr(self._parent, "_cached_seq_len_py", None)
            return int(cached) if cached is not None else self.get_max_cache_shape()
        return None

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        cached = self._cached_length()
        if cached is not None:
            return cached + query_length, 0
        return int(self._row_seq_lens.max().item()) + query_length, 0

    def get_seq_length(self) -> int:
        cached = self._cached_length()
        if cached is not None:
            return cached
        return int(self._row_seq_lens.max().item())

    def get_max_cache_shape(self) -> int:
        return int(self._parent.block_tables.shape[1]) * self.pool.block_size_tokens

    def get_max_length(self) -> int:
        return self.get_max_cache_shape()

    def reset(self) -> None:
        self.is_initialized = False
        self._row_seq_lens = self._parent.seq_lens.clone()


class BlockPagedCache(Cache):
    """Per-request (batch 1) cache over the shared pool (``paged_kv_cache.py:196-230``)."""

    def __init__(self, config, pool: GpuKVBlockPool) -> None:
        config = _text_config(config)
        layers = [BlockPagedLayer(pool=pool, layer_idx=i) for i in range(_decoder_layer_count(config))]
        super().__init__(layers=layers)
        self.pool = pool
        self._config = config
        self._block_table: torch.Tensor | None = None
        self.block_table_ids: list[int] = []

    def set_block_ids(self, block_ids: list[int]) -> None:
        if self._block_table is not None and self.block_table_ids == list(block_ids):
            return
        table = torch.tensor(list(block_ids), dtype=torch.int32).to(self.pool.device)
        for layer in self.layers:
            layer.set_block_ids(block_ids, table)
        self._block_table = table
        self.block_table_ids = list(block_ids)

    def sync_block_ids(self, block_ids: list[int]) -> None:
        self.set_block_ids(block_ids)

    def block_table(self) -> torch.Tensor | None:
        return self._block_table

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.layers[layer_idx].get_seq_length()


class BlockPagedBatchCache(Cache):
    """Batched decode cache with persistent slots (``paged_kv_cache.py:233-431``).

    ``block_tables [B, max_blocks]`` and ``seq_lens [B]`` are int32 on the pool's
    device; ``block_ids_rows`` mirrors the tables on the host. ``empty``
    creates a fixed-capacity batch whose slots are handed out by
    ``allocate_slot``/``bind_cache`` and returned by ``release_slot``;
    ``dense_active_cache`` / ``write_back_dense`` run one decode over a subset
    of slots and copy lengths and tables back.
    """

    def __init__(self, config, pool: GpuKVBlockPool, *, block_tables: torch.Tensor, seq_lens: torch.Tensor,
                 block_ids_rows: list[list[int]]) -> None:
        config = _text_config(config)
        self.pool = pool
        self._config = config
        self.block_tables = block_tables.to(device=pool.device, dtype=torch.int32)
        self.seq_lens = seq_lens.to(device=pool.device, dtype=torch.int32)
        self.block_ids_rows = [list(row) for row in block_ids_rows]
        self._batch_size = int(self.block_tables.shape[0])
        self._slot_occupied: list[bool] = [True] * self._batch_size
        self._free_slots: list[int] = []
        self._request_to_slot: dict[str, int] = {}
        layers = [BlockPagedBatchLayer(pool=pool, layer_idx=i, parent=self)
                  for i in range(_decoder_layer_count(config))]
        super().__init__(layers=layers)

    @classmethod
    def empty(cls, config, pool: GpuKVBlockPool, *, max_batch_size: int, max_blocks: int) -> "BlockPagedBatchCache":
        if max_batch_size <= 0 or max_blocks <= 0:
            raise ValueError("max_batch_size and max_blocks must be positive")
        cache = cls(config, pool,
                    block_tables=torch.zeros(max_batch_size, max_blocks, dtype=torch.int32),
                    seq_lens=torch.zeros(max_batch_size, dtype=torch.int32),
                    block_ids_rows=[[] for _ in range(max_batch_size)])
        cache._slot_occupied = [False] * max_batch_size
        # Slots are popped from the end, so slot 0 is handed out first.
        cache._free_slots = list(range(max_batch_size - 1, -1, -1))
        return cache

    @classmethod
    def from_caches(cls, caches: list[BlockPagedCache], pool: GpuKVBlockPool) -> "BlockPagedBatchCache":
        if not caches:
            raise ValueError("from_caches requires at least one cache")
        rows = [list(c.layers[0]._block_ids) for c in caches]
        lens = [c.layers[0].get_seq_length() for c in caches]
        width = max(len(r) for r in rows)
        tables = torch.stack([_table_row(r, width, torch.device("cpu")) for r in rows])
        return cls(caches[0]._config, pool, block_tables=tables,
                   seq_lens=torch.tensor(lens, dtype=torch.int32), block_ids_rows=rows)

    # Slot management --------------------------------------------------------------------

    def allocate_slot(self, request_id: str) -> int:
        slot = self._request_to_slot.get(request_id)
        if slot is not None:
            return slot
        if not self._free_slots:
            raise RuntimeError("persistent paged batch has no free slots")
        slot = self._free_slots.pop()
        self._slot_occupied[slot] = True
        self._request_to_slot[request_id] = slot
        return slot

    def release_slot(self, request_id: str) -> None:
        slot = self._request_to_slot.pop(request_id, None)
        if slot is None:
            return
        self._slot_occupied[slot] = False
        self.block_ids_rows[slot] = []
        self.seq_lens[slot] = 0
        self.block_tables[slot].zero_()
        self._free_slots.append(slot)

    def _set_row_length(self, slot: int, seq_len: int) -> None:
        self.seq_lens[slot] = int(seq_len)
        for layer in self.layers:
            layer._row_seq_lens[slot] = int(seq_len)

    def bind_cache(self, request_id: str, cache: BlockPagedCache) -> int:
        slot = self.allocate_slot(request_id)
        layer0 = cache.layers[0]
        self.sync_block_ids_row(slot, list(layer0._block_ids))
        self._set_row_length(slot, layer0.get_seq_length())
        return slot

    def slot_of(self, request_id: str) -> int | None:
        return self._request_to_slot.get(request_id)

    def dense_active_cache(self, request_ids: list[str]) -> tuple["BlockPagedBatchCache", list[int]]:
        """A dense ``len(request_ids)``-row cache over the selected slots (tables copied on the device)."""
        slots: list[int] = []
        for rid in request_ids:
            slot = self._request_to_slot.get(rid)
            if slot is None:
                raise KeyError(f"request {rid} is not bound to a persistent slot")
            slots.append(slot)
        if not slots:
            raise ValueError("dense_active_cache requires at least one request")
        index = torch.tensor(slots, dtype=torch.long).to(self.block_tables.device)
        dense = BlockPagedBatchCache(self._config, self.pool,
                                     block_tables=self.block_tables.index_select(0, index),
                                     seq_lens=self.seq_lens.index_select(0, index),
                                     block_ids_rows=[self.block_ids_rows[s] for s in slots])
        return dense, slots

    def write_back_dense(self, dense: "BlockPagedBatchCache", slots: list[int]) -> None:
        """Copy lengths and tables of a dense decode back into the persistent slots.

        The lengths move device to device (one ``index_copy_`` per length tensor, no host
        read; the reference reads each row's length back per layer, ``:389-396``), and a
        table row is re-uploaded only when its block ids changed.
        """
        index = torch.tensor(slots, dtype=torch.long).to(self.seq_lens.device)
        lens = dense.seq_lens.to(self.seq_lens.dtype)
        self.seq_lens.index_copy_(0, index, lens)
        for layer in self.layers:
            layer._row_seq_lens.index_copy_(0, index, lens)
        for i, slot in enumerate(slots):
            if self.block_ids_rows[slot] != dense.block_ids_rows[i]:
                self.sync_block_ids_row(slot, list(dense.block_ids_rows[i]))

    def extract_cache(self, index: int, seq_len: int | None = None) -> BlockPagedCache:
        """A batch-1 cache over slot ``index``. ``seq_len``, when the caller knows it (a decode
        step adds one token per row), saves reading the length back from the device."""
        cache = BlockPagedCache(self._config, self.pool)
        cache.set_block_ids(self.block_ids_rows[index])
        if seq_len is None:
            seq_len = int(self.seq_lens[index].item())
        for layer in cache.layers:
            layer.set_seq_length(seq_len)
        return cache

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return int(self.seq_lens.max().item())

    def ensure_max_blocks(self, max_blocks: int) -> None:
        width = int(self.block_tables.shape[1])
        if max_blocks <= width:
            return
        grown = torch.zeros(self._batch_size, max_blocks, dtype=torch.int32, device=self.block_tables.device)
        grown[:, :width] = self.block_tables
        self.block_tables = grown

    def sync_block_ids_row(self, index: int, block_ids: list[int]) -> None:
        self.block_ids_rows[index] = list(block_ids)
        if len(block_ids) > int(self.block_tables.shape[1]):
            self.ensure_max_blocks(len(block_ids))
        self.block_tables[index] = _table_row(block_ids, int(self.block_tables.shape[1]), self.block_tables.device)
