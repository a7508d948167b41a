"""Shared-prefix block tables and a join/finish schedule for batched decode.

The reference serves requests that share a prompt prefix through its prefix cache
(``runtime/phase2/prefix_cache.py:146-262``) and block allocator
(``runtime/phase2/kv_allocator.py:46-133``). On a paged prefix hit the worker *copies*
the cached prefix blocks into the new request's own blocks
(``runtime/phase2/worker_server.py:1372-1375,1442-1449`` via ``GpuKVBlockPool.copy_blocks``,
``runtime/phase2/paged_kv_kernel.py:233-250``). Here the rows of a group alias the
group's prefix block ids instead. The decode kernels only read a row's blocks below its
length and append past it, so a block-aligned prefix is shared without copies: a
1024-token prefix read by 8 rows is stored once.

This module is the host side of that workload (block bookkeeping, not a serving
scheduler):

* :class:`BlockAllocator` — a free list of physical block ids with reference counts
  (a prefix block is freed when the last row using it finishes);
* :class:`PrefixBatch` — ``batch`` row slots in ``groups`` groups. Each row holds
  ``ctx ~ U[lo, hi]`` tokens; a row longer than the prefix starts with its group's
  prefix blocks. ``rotate(rows)`` finishes those rows and admits new requests of the
  same group into their slots (join/finish). ``tables`` / ``lens`` are the int32 block
  tables and KV lengths the decode step reads, kept on the host and copied to
  fixed device tensors by :meth:`upload` (addresses stay valid for a captured graph);
* :meth:`PrefixBatch.unique_tokens` / :meth:`PrefixBatch.logical_tokens` — K/V tokens
  stored once vs. read per step, the byte counts the measurement is quoted on.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


class BlockAllocator:
    """Physical block ids ``[0, num_blocks)`` with reference counts; allocation order is seeded."""

    def __init__(self, num_blocks: int, seed: int = 0) -> None:
        if num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        g = torch.Generator().manual_seed(seed)
        self._free = torch.randperm(num_blocks, generator=g).tolist()
        self._refs = [0] * num_blocks

    @property
    def free_blocks(self) -> int:
        return len(self._free)

    def alloc(self, n: int) -> list[int]:
        if n > len(self._free):
            raise RuntimeError(f"out of KV blocks: need {n}, {len(self._free)} free")
        ids = [self._free.pop() for _ in range(n)]
        for i in ids:
            self._refs[i] = 1
        return ids

    def incref(self, ids: list[int]) -> None:
        for i in ids:
            if self._refs[i] <= 0:
                raise RuntimeError(f"block {i} is not allocated")
            self._refs[i] += 1

    def decref(self, ids: list[int]) -> None:
        for i in ids:
            if self._refs[i] <= 0:
                raise RuntimeError(f"block {i} freed twice")
            self._refs[i] -= 1
            if self._refs[i] == 0:
                self._free.append(i)

    def refcount(self, i: int) -> int:
        return self._refs[i]


@dataclass
class Row:
    group: int
    length: int          # tokens in the KV cache (the next token's position)
    shared: int          # leading blocks that are the group's prefix (0 when not shared)
    blocks: list[int]    # physical ids, prefix first


class PrefixBatch:
    """Row slots with group-shared prefix blocks and a join/finish schedule.

    Row ``b`` belongs to group ``b // (batch // groups)``. Every row gets blocks for its
    context plus ``headroom`` decode tokens. Context lengths are drawn from ``U[lo, hi]``
    (seeded) unless ``lengths`` gives them.
    """

    def __init__(self, *, batch: int, groups: int, prefix_tokens: int, lo: int, hi: int, block_size: int,
                 num_blocks: int, headroom: int, seed: int = 0, lengths: list[int] | None = None) -> None:
        if batch % groups:
            raise ValueError("batch must be a multiple of groups")
        if prefix_tokens % block_size:
            raise ValueError("the shared prefix must be a whole number of blocks")
        if not 1 <= lo <= hi:
            raise ValueError("need 1 <= lo <= hi")
        self.batch, self.groups, self.block_size = batch, groups, block_size
        self.prefix_tokens, self.lo, self.hi, self.headroom = prefix_tokens, lo, hi, headroom
        self.max_blocks = math.ceil((hi + headroom) / block_size)
        self.alloc = BlockAllocator(num_blocks, seed)
        self._gen = torch.Generator().manual_seed(seed + 1)
        nprefix = prefix_tokens // block_size
        # Each group holds one reference to its prefix blocks for its whole life, so the
        # prefix survives while no row of the group is live.
        self.prefix_blocks = [self.alloc.alloc(nprefix) for _ in range(groups)]
        if lengths is not None and len(lengths) != batch:
            raise ValueError("lengths needs one entry per row")
        self.rows: list[Row] = [self._admit(b // (batch // groups), None if lengths is None else lengths[b])
                                for b in range(batch)]

    # -- requests ---------------------------------------------------------------
    def _admit(self, group: int, length: int | None = None) -> Row:
        if length is None:
            length = int(torch.randint(self.lo, self.hi + 1, (1,), generator=self._gen))
        need = math.ceil((length + self.headroom) / self.block_size)
        nprefix = self.prefix_tokens // self.block_size
        if length > self.prefix_tokens and nprefix > 0:
            pre = self.prefix_blocks[group]
            self.alloc.incref(pre)
            return Row(group, length, nprefix, pre + self.alloc.alloc(need - nprefix))
        return Row(group, length, 0, self.alloc.alloc(need))

    def rotate(self, rows: list[int], lengths: list[int] | None = None) -> None:
        """Finish the requests in ``rows`` and admit new ones of the same group in their slots."""
        for j, b in enumerate(rows):
            old = self.rows[b]
            self.alloc.decref(old.blocks)
            self.rows[b] = self._admit(old.group, None if lengths is None else lengths[j])

    def advance(self, steps: int = 1) -> None:
        """Host mirror of the decode step's length advance."""
        for r in self.rows:
            r.length += steps
            if r.length > len(r.blocks) * self.block_size:
                raise RuntimeError("row ran past its blocks; raise headroom")

    # -- device views ------------------------------------------------------------
    @property
    def tables(self) -> torch.Tensor:
        t = torch.zeros(self.batch, self.max_blocks, dtype=torch.int32)
        for b, r in enumerate(self.rows):
            t[b, :len(r.blocks)] = torch.tensor(r.blocks, dtype=torch.int32)
        return t

    @property
    def lens(self) -> torch.Tensor:
        return torch.tensor([r.length for r in self.rows], dtype=torch.int32)

    def upload(self, tables_d: torch.Tensor, lens_d: torch.Tensor) -> None:
        """Copy tables and lengths into fixed device tensors (graph-safe: addresses unchanged)."""
        tables_d.copy_(self.tables)
        lens_d.copy_(self.lens)

    def upload_rows(self, rows: list[int], tables_d: torch.Tensor, lens_d: torch.Tensor) -> None:
        """:meth:`upload` for the table rows in ``rows`` only (the slots :meth:`rotate` just
        refilled); every other table row is unchanged since the last upload. All lengths are
        copied, as the decode step advances them on the device."""
        if rows:
            part = torch.zeros(len(rows), self.max_blocks, dtype=torch.int32)
            for j, b in enumerate(rows):
                blocks = self.rows[b].blocks
                part[j, :len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
            idx = torch.tensor(rows, dtype=torch.int64, device=tables_d.device)
            tables_d.index_copy_(0, idx, part.to(tables_d.device))
        lens_d.copy_(self.lens)

    # -- byte accounting ---------------------------------------------------------
    def logical_tokens(self, extra: int = 0) -> int:
        """K/V tokens the rows attend over (each row counts its prefix), with ``extra`` more per row."""
        return sum(r.length + extra for r in self.rows)

    def unique_tokens(self, extra: int = 0) -> int:
        """Distinct stored K/V tokens behind :meth:`logical_tokens`: a shared prefix counts once."""
        seen: set[int] = set()
        total = 0
        for r in self.rows:
            n = r.length + extra
            for j, blk in enumerate(r.blocks):
                used = min(self.block_size, n - j * self.block_size)
                if used <= 0:
                    break
                if j < r.shared:
                    if blk in seen:
                        continue
                    seen.add(blk)
                total += used
        return total
