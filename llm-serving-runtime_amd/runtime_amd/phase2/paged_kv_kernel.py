"""Block-paged KV storage read by the HIP paged-attention decode kernel.

Keeps the reference's ``GpuKVBlockPool`` API (``runtime/phase2/paged_kv_kernel.py:24-315``):
``k_layer_view(l)`` / ``v_layer_view(l)`` are ``[num_blocks, Hkv, bs, D]`` per
layer with every (block, kv-head) one contiguous ``bs*D`` run (4 KiB at bs=16,
D=128, fp16), and token ``pos`` of a row is stored in block
``table[pos // bs]`` at offset ``pos % bs`` (``:163-174``, ``:217-227``).

MI355X-first differences:

* Layer-major storage, K beside V. The reference stores K and V in two
  ``[num_blocks, num_layers, Hkv, bs, D]`` tensors (``:101-107``), so one
  layer's blocks are spread over the whole pool, one ``Hkv*bs*D`` run every
  ``num_layers`` runs. Here one tensor ``[num_layers, num_blocks, Hkv, 2, bs,
  D]`` holds both: a layer is one contiguous region (``num_blocks * 64 KiB``
  for Llama-3-8B's 8 KV heads), so the decode kernel's random block reads for a
  layer stay inside a region the GPU's address-translation caches cover instead
  of landing on a different 2 MiB page almost every time across a 17 GB pool,
  and the K and V runs of a (block, kv-head) are one run. The views keep the
  reference's shape and per-block contents; only the strides of the first two
  dimensions differ, and every consumer takes strides from the view
  (``kv_layout="split"`` keeps K and V in two layer-major tensors).
* The reference grows its slabs lazily 8 blocks at a time and copies the
  whole slab on every growth (``:86-115``). Here the first use allocates all
  ``num_blocks`` at once (288 GB of HBM per GPU makes that the cheap choice),
  so tensor addresses never change after ``_ensure_pools`` and a captured HIP
  graph stays valid.
* ``write_tokens_batch`` on a device pool makes no host round trip. The
  reference checks the table bounds with ``.item()`` and records the written
  blocks with ``unique().tolist()`` on every call (``:221,229-231``), four
  syncs per layer per step. Here the one ``mx_kv_append`` launch skips a slot
  outside the table or the pool and sets the pool's device error word, and
  marks the blocks it writes in a device byte map. The ``IndexError`` the
  reference raises is raised by :meth:`check_write_errors` (one sync, called
  once per decode step by the decode loop), and ``allocated_block_count`` /
  ``peak_allocated_block_count`` read the byte map when asked. A caller that
  relies on the reference's raise at the write itself sets
  ``sync_write_checks`` (or ``PHASE2_KV_SYNC_CHECKS=1`` before the pool is
  built): every batched write then checks the word right away (one host sync
  per call, skipped while a HIP graph is being captured).
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass

import torch


KV_LAYOUTS = ("split", "interleaved")


@dataclass(frozen=True)
class PoolShape:
    num_blocks: int
    block_size_tokens: int
    num_layers: int
    num_kv_heads: int
    head_dim: int


class GpuKVBlockPool:
    """Shared block pool; same constructor and methods as the reference's."""

    def __init__(self, *, num_blocks: int, block_size_tokens: int, num_layers: int, num_kv_heads: int, head_dim: int,
                 dtype: torch.dtype, device: str | torch.device, kv_layout: str = "interleaved") -> None:
        if num_blocks <= 0 or block_size_tokens <= 0:
            raise ValueError("num_blocks and block_size_tokens must be positive")
        if kv_layout not in KV_LAYOUTS:
            raise ValueError(f"kv_layout must be one of {KV_LAYOUTS}, got {kv_layout!r}")
        # "interleaved" (default): one tensor [L, nb, Hkv, 2, bs, D] whose K and V runs of a
        # (block, kv-head) are adjacent, one 2*bs*D run that the decode kernel reads as a unit; the
        # layer views keep the shape [nb, Hkv, bs, D] with strides (Hkv*2*bs*D, 2*bs*D, D, 1).
        # Measured on MI355X at the Llama-3-8B batch-32 step: attention 56.7-57.0 -> 54.6-55.4 us
        # per call, 7,773-7,817 -> 7,921-7,929 tokens/s. "split": K and V in two [L, nb, Hkv, bs, D]
        # tensors, each (block, kv-head) run bs*D elements.
        self.kv_layout = kv_layout
        self.shape = PoolShape(num_blocks=num_blocks, block_size_tokens=block_size_tokens, num_layers=num_layers,
                               num_kv_heads=num_kv_heads, head_dim=head_dim)
        self.dtype = dtype
        self.device = torch.device(device)
        self._k_pool: torch.Tensor | None = None
        self._v_pool: torch.Tensor | None = None
        self._used_blocks: set[int] = set()
        self._peak_allocated_blocks = 0
        self._used_map: torch.Tensor | None = None    # uint8 [num_blocks]: blocks written on the device
        self._write_err: torch.Tensor | None = None   # int32 [1]: kv append error bits since the last check
        # True: write_tokens_batch raises IndexError at the call, as the reference does (:221-222),
        # at one host sync per call; False: at the next check_write_errors().
        self.sync_write_checks = os.getenv("PHASE2_KV_SYNC_CHECKS", "0").strip() == "1"

    @property
    def block_size_tokens(self) -> int:
        return self.shape.block_size_tokens

    def _sync_used_map(self) -> None:
        """Fold the device byte map of written blocks into the host set (one host sync)."""
        if self._used_map is None:
            return
        ids = torch.nonzero(self._used_map).flatten().tolist()
        if ids:
            self._used_blocks.update(int(i) for i in ids)
            self._peak_allocated_blocks = max(self._peak_allocated_blocks, len(self._used_blocks))

    def allocated_block_count(self) -> int:
        self._sync_used_map()
        return len(self._used_blocks)

    def peak_allocated_block_count(self) -> int:
        self._sync_used_map()
        return self._peak_allocated_blocks

    def check_write_errors(self) -> None:
        """Raise ``IndexError`` if a device KV write met a slot outside its block table or the
        pool since the last check (the reference's ``:221-222`` check, deferred to one host
        sync); the error word is cleared."""
        if self._write_err is None:
            return
        bits = int(self._write_err.item())
        if bits:
            self._write_err.zero_()
            raise IndexError("block table underrun or physical block id out of range during batched write")

    def bytes_per_block(self) -> int:
        s = self.shape
        elems = s.num_layers * s.num_kv_heads * s.block_size_tokens * s.head_dim * 2
        return elems * torch.empty((), dtype=self.dtype).element_size()

    def bytes_for_blocks(self, block_count: int) -> int:
        return block_count * self.bytes_per_block()

    def peak_allocated_bytes(self) -> int:
        return self.bytes_for_blocks(self.peak_allocated_block_count())

    def _ensure_pools(self) -> None:
        if self._k_pool is not None:
            return
        s = self.shape
        if self.kv_layout == "interleaved":
            kv = torch.zeros(s.num_layers, s.num_blocks, s.num_kv_heads, 2, s.block_size_tokens, s.head_dim,
                             dtype=self.dtype, device=self.device)
            self._k_pool, self._v_pool = kv[:, :, :, 0], kv[:, :, :, 1]
        else:
            shape = (s.num_layers, s.num_blocks, s.num_kv_heads, s.block_size_tokens, s.head_dim)
            self._k_pool = torch.zeros(shape, dtype=self.dtype, device=self.device)
            self._v_pool = torch.zeros(shape, dtype=self.dtype, device=self.device)
        if self.device.type == "cuda":
            self._used_map = torch.zeros(s.num_blocks, dtype=torch.uint8, device=self.device)
            self._write_err = torch.zeros(1, dtype=torch.int32, device=self.device)

    def _touch_block(self, physical: int) -> None:
        if physical < 0 or physical >= self.shape.num_blocks:
            raise IndexError(f"physical block id out of range: {physical}")
        self._used_blocks.add(physical)
        self._peak_allocated_blocks = max(self._peak_allocated_blocks, len(self._used_blocks))

    def _touch_blocks(self, physical_ids: torch.Tensor) -> None:
        for physical in physical_ids.unique().tolist():
            self._touch_block(int(physical))

    def k_layer_view(self, layer_idx: int) -> torch.Tensor:
        """Per-layer K blocks: ``[num_blocks, num_kv_heads, block_size, head_dim]``."""
        self._ensure_pools()
        assert self._k_pool is not None
        return self._k_pool[layer_idx]

    def v_layer_view(self, layer_idx: int) -> torch.Tensor:
        """Per-layer V blocks: ``[num_blocks, num_kv_heads, block_size, head_dim]``."""
        self._ensure_pools()
        assert self._v_pool is not None
        return self._v_pool[layer_idx]

    def write_tokens(self, layer_idx: int, block_ids: list[int], start_pos: int, key_states: torch.Tensor,
                     value_states: torch.Tensor) -> None:
        """Write K/V for positions ``[start_pos, start_pos + kv_len)`` of one row (``:136-174``)."""
        if key_states.dim() == 3:
            key_states = key_states.unsqueeze(0)
            value_states = value_states.unsqueeze(0)
        if key_states.shape[0] != 1:
            raise ValueError("write_tokens takes a single row; use write_tokens_batch")
        kv_len = int(key_states.shape[-2])
        block_size = self.block_size_tokens
        n_logical = math.ceil((start_pos + kv_len) / block_size)
        if n_logical > len(block_ids):
            raise IndexError(f"block table underrun at pos={start_pos + kv_len - 1}: need block {n_logical - 1}, "
                             f"have {len(block_ids)}")
        table = torch.tensor([list(block_ids)], device=self.device, dtype=torch.int32)
        starts = torch.tensor([start_pos], device=self.device, dtype=torch.int64)
        self.write_tokens_batch(layer_idx, table, starts, key_states, value_states)

    def write_tokens_batch(self, layer_idx: int, block_tables: torch.Tensor, start_positions: torch.Tensor,
                           key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """KV write: tables ``[B, max_blocks]``, starts ``[B]``, states ``[B, Hkv, kv_len, D]``.

        Same semantics as the reference (``:176-227``). On a device pool it is
        one ``mx_kv_append`` launch (no per-token loop) and no host sync: a slot
        outside the table or the pool is skipped and recorded in the pool's
        error word, which :meth:`check_write_errors` turns into the reference's
        ``IndexError`` (``:221-222``); written blocks are marked in a device map
        for the usage accounting. A pool on the CPU (host-side tests of the
        cache bookkeeping) checks on the host and takes an indexed torch store.
        """
        if key_states.shape != value_states.shape:
            raise ValueError("key_states and value_states must match shape")
        batch_size = int(key_states.shape[0])
        kv_len = int(key_states.shape[-2])
        if block_tables.shape[0] != batch_size or start_positions.shape[0] != batch_size:
            raise ValueError("batch dimension mismatch in write_tokens_batch")
        if kv_len == 0 or batch_size == 0:
            return
        self._ensure_pools()
        assert self._k_pool is not None and self._v_pool is not None
        device = self.device
        bs = self.block_size_tokens
        k_layer = self._k_pool[layer_idx]
        v_layer = self._v_pool[layer_idx]
        if device.type == "cuda":
            from .decode_glue import kv_append

            kv_append(k_layer, v_layer, block_tables, start_positions, key_states.to(self.dtype),
                      value_states.to(self.dtype), err=self._write_err, used_blocks=self._used_map)
            if self.sync_write_checks and not torch.cuda.is_current_stream_capturing():
                self.check_write_errors()
            return
        tables = block_tables.to(device=device, dtype=torch.int64)
        pos = start_positions.to(device=device, dtype=torch.int64).view(-1, 1) + torch.arange(
            kv_len, device=device, dtype=torch.int64).view(1, -1)  # [B, T]
        logical = torch.div(pos, bs, rounding_mode="floor")
        if int(logical.max().item()) >= tables.shape[1] or int(pos.min().item()) < 0:
            raise IndexError("block table underrun during batched write")
        physical = torch.gather(tables, 1, logical)  # [B, T]
        if int(physical.min().item()) < 0 or int(physical.max().item()) >= self.shape.num_blocks:
            raise IndexError("physical block id out of range during batched write")
        self._touch_blocks(physical)
        offset = (pos % bs).reshape(-1)
        phys = physical.reshape(-1)
        # pool[physical, layer, :, offset, :] = states[b, :, t, :]
        k_layer[phys, :, offset, :] = key_states.to(self.dtype).permute(0, 2, 1, 3).reshape(
            -1, key_states.shape[1], key_states.shape[3])
        v_layer[phys, :, offset, :] = value_states.to(self.dtype).permute(0, 2, 1, 3).reshape(
            -1, value_states.shape[1], value_states.shape[3])

    def copy_blocks(self, src_block_ids: list[int], dst_block_ids: list[int]) -> None:
        """Copy full physical blocks (all layers) from src ids to dst ids (``:233-250``)."""
        if len(src_block_ids) != len(dst_block_ids):
            raise ValueError(f"copy_blocks length mismatch: src={len(src_block_ids)} dst={len(dst_block_ids)}")
        if not src_block_ids:
            return
        self._ensure_pools()
        assert self._k_pool is not None and self._v_pool is not None
        pairs = [(int(s), int(d)) for s, d in zip(src_block_ids, dst_block_ids) if int(s) != int(d)]
        for s, d in pairs:
            self._touch_block(s)
            self._touch_block(d)
        if not pairs:
            return
        src = torch.tensor([s for s, _ in pairs], device=self.device, dtype=torch.long)
        dst = torch.tensor([d for _, d in pairs], device=self.device, dtype=torch.long)
        self._k_pool[:, dst] = self._k_pool[:, src]
        self._v_pool[:, dst] = self._v_pool[:, src]

    def gather_layer(self, layer_idx: int, block_ids: list[int], seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Gather one row as ``[1, Hkv, seq_len, D]`` (prefill / parity, ``:252-283``)."""
        if seq_len <= 0:
            raise ValueError("seq_len must be positive")
        bs = self.block_size_tokens
        n_logical = math.ceil(seq_len / bs)
        if n_logical > len(block_ids):
            raise IndexError("block table underrun during gather")
        self._ensure_pools()
        assert self._k_pool is not None and self._v_pool is not None
        ids_list = [int(b) for b in list(block_ids)[:n_logical]]
        for b in ids_list:
            self._touch_block(b)
        ids = torch.tensor(ids_list, device=self.device, dtype=torch.long)
        s = self.shape
        k = self._k_pool[layer_idx, ids].permute(1, 0, 2, 3).reshape(s.num_kv_heads, n_logical * bs, s.head_dim)
        v = self._v_pool[layer_idx, ids].permute(1, 0, 2, 3).reshape(s.num_kv_heads, n_logical * bs, s.head_dim)
        return k[:, :seq_len].unsqueeze(0), v[:, :seq_len].unsqueeze(0)

    def gather_layer_batch(self, layer_idx: int, block_tables: torch.Tensor, seq_lens: torch.Tensor
                           ) -> tuple[torch.Tensor, torch.Tensor]:
        """Gather rows as zero-padded ``[B, Hkv, max_seq, D]`` (batched prefill, ``:285-309``)."""
        batch_size = int(block_tables.shape[0])
        lens = [int(x) for x in seq_lens.tolist()]
        max_seq = max(lens) if lens else 0
        if max_seq <= 0:
            raise ValueError("seq_len must be positive")
        s = self.shape
        keys = torch.zeros(batch_size, s.num_kv_heads, max_seq, s.head_dim, device=self.device, dtype=self.dtype)
        values = torch.zeros_like(keys)
        for b in range(batch_size):
            n_logical = math.ceil(lens[b] / self.block_size_tokens)
            row_ids = [int(x) for x in block_tables[b, :n_logical].tolist()]
            k, v = self.gather_layer(layer_idx, row_ids, lens[b])
            keys[b, :, : lens[b]] = k[0]
            values[b, :, : lens[b]] = v[0]
        return keys, values

    def reset(self) -> None:
        self._k_pool = None
        self._v_pool = None
        self._used_map = None
        self._write_err = None
        self._used_blocks.clear()
        self._peak_allocated_blocks = 0
