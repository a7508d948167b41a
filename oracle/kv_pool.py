"""Oracle: paged KV pool layout, token write and gather. TEST INFRASTRUCTURE ONLY.

Restates ``runtime/phase2/paged_kv_kernel.py`` of the reference on plain CPU
tensors:

* storage ``[num_blocks, num_layers, num_kv_heads, block_size, head_dim]`` for
  K and for V (``paged_kv_kernel.py:101-107``); the per-layer view is
  ``pool[:, layer]`` -> ``[num_blocks, Hkv, bs, D]`` (``:124-134``);
* token ``pos`` of a row lives in physical block ``table[pos // bs]`` at
  offset ``pos % bs`` (``:163-174``, ``:217-227``), an index past the table is
  an underrun error (``:167-170``, ``:221-222``);
* gather concatenates the first ``ceil(S / bs)`` logical blocks and keeps
  ``S`` tokens (``:252-283``).

Parity pinning: the reference's own known-answer round trip
(``tests/test_paged_kv_kernel.py:11-28``: K = 1s, V = 2s, bs = 2, Hkv = 2, D = 4)
and a write -> gather identity over random tables (tests/test_oracle_kv_pool.py).
"""

from __future__ import annotations

import math

import torch


def empty_pool(num_blocks: int, num_layers: int, num_kv_heads: int, block_size: int, head_dim: int,
               dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    shape = (num_blocks, num_layers, num_kv_heads, block_size, head_dim)
    return torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)


def write_tokens(k_pool: torch.Tensor, v_pool: torch.Tensor, layer: int, block_ids: list[int], start_pos: int,
                 key_states: torch.Tensor, value_states: torch.Tensor) -> None:
    """Write ``key/value_states [Hkv, T, D]`` (or ``[1, Hkv, T, D]``) at positions ``start_pos..``."""
    if key_states.dim() == 4:
        key_states = key_states[0]
        value_states = value_states[0]
    block_size = k_pool.shape[3]
    for t in range(int(key_states.shape[-2])):
        pos = start_pos + t
        logical = pos // block_size
        if logical >= len(block_ids):
            raise IndexError(f"block table underrun at pos={pos}")
        phys = int(block_ids[logical])
        k_pool[phys, layer, :, pos % block_size, :] = key_states[:, t, :]
        v_pool[phys, layer, :, pos % block_size, :] = value_states[:, t, :]


def gather_layer(k_pool: torch.Tensor, v_pool: torch.Tensor, layer: int, block_ids: list[int],
                 seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``[1, Hkv, seq_len, D]`` keys and values of one row."""
    if seq_len <= 0:
        raise ValueError("seq_len must be positive")
    block_size = k_pool.shape[3]
    n_logical = math.ceil(seq_len / block_size)
    if n_logical > len(block_ids):
        raise IndexError("block table underrun during gather")
    ids = [int(b) for b in block_ids[:n_logical]]
    k = torch.cat([k_pool[i, layer] for i in ids], dim=1)[:, :seq_len]
    v = torch.cat([v_pool[i, layer] for i in ids], dim=1)[:, :seq_len]
    return k.unsqueeze(0), v.unsqueeze(0)


def gather_layer_view(k_layer: torch.Tensor, v_layer: torch.Tensor, block_ids, seq_len: int
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather from per-layer views ``[num_blocks, Hkv, bs, D]`` -> ``[1, Hkv, seq_len, D]``."""
    block_size = k_layer.shape[2]
    n_logical = math.ceil(seq_len / block_size)
    ids = torch.as_tensor([int(b) for b in list(block_ids)[:n_logical]], dtype=torch.long)
    if int(ids.numel()) < n_logical:
        raise IndexError("block table underrun during gather")
    k = k_layer.index_select(0, ids).permute(1, 0, 2, 3).reshape(k_layer.shape[1], -1, k_layer.shape[3])
    v = v_layer.index_select(0, ids).permute(1, 0, 2, 3).reshape(v_layer.shape[1], -1, v_layer.shape[3])
    return k[:, :seq_len].unsqueeze(0), v[:, :seq_len].unsqueeze(0)
