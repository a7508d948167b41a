"""Replay the HF paged decode forward from HIP graphs.

The reference's worker builds ``CudaGraphDecodeManager(model=, device=, warmup_steps=)``
(``runtime/phase2/worker_server.py:242-249``) and, on every batched decode step, asks it for
the step's logits with ``try_decode(persistent=, decode_states=, input_ids=)``; ``None`` sends
the worker down its eager path (``:747-753``). That constructor and that call are the whole
interface kept here. Everything behind them is this module's own design.

How a step is replayed:

* One :class:`StepGraph` per ``(rows, table width)``. The width is the persistent cache's own
  ``block_tables`` width, the width the eager path's ``dense_active_cache`` hands to attention,
  so a replay and an eager step launch the same kernels on the same table shape. A persistent
  cache that grows its tables gets a new graph; at most ``max_graphs`` are kept (least recently
  used dropped first).
* A graph owns a staging :class:`BlockPagedBatchCache` of ``rows`` rows in graph-safe mode
  (lengths advance in place on the device), the static ``input_ids`` and ``position_ids``
  (each row's own length) and, once captured, the graph and its logits.
* ``load`` gathers the active slots' table rows and lengths from the persistent cache with one
  device ``index_select`` each; ``run`` replays (or, while warming, runs eagerly); ``store``
  scatters the advanced lengths back with ``index_copy_`` and brings each request's batch-1
  cache to its new length in place. Block tables do not change inside a decode forward, so only
  lengths travel back. Nothing here reads a device value on the host.
* The first ``warmup_steps`` calls of a graph run the forward eagerly on the staging cache
  (they size every kernel workspace), the next one captures and replays it, and later ones
  replay. Capture only records, so the staging lengths are exactly as ``load`` left them.
* A capture that raises marks that key as eager-only and the call returns ``None``; the other
  keys keep their graphs. Only when the device reports a sticky error afterwards is the whole
  manager switched off.

Opt-in: ``enabled=True``, or ``PHASE2_CUDA_GRAPH=1`` in the environment (the switch the
reference's worker reads before it builds the manager). The reference also requires
``PHASE2_CUDA_GRAPH_TRY_HF=1`` because its HF capture breaks on host syncs; this path's
forward has none (the ``block_paged`` hook has no mask function, positions are passed in, KV
overruns go to the pool's device error word), so that second switch is accepted and ignored.

One observable difference from the reference: the forward gets each row's own position
(``position_ids``); the reference passes a ``[B]`` ``cache_position``, which HF reads as one
position sequence for the whole batch.
"""

from __future__ import annotations

import os
from collections import OrderedDict
from typing import Any

import torch

from .paged_attention_hip import set_paged_decode_batch_metadata
from .paged_kv_cache import BlockPagedBatchCache, BlockPagedCache


def _opted_in() -> bool:
    return os.getenv("PHASE2_CUDA_GRAPH", "0").strip() == "1"


class StepGraph:
    """The HF decode forward of ``rows`` rows over tables ``width`` blocks wide, as a HIP graph."""

    def __init__(self, model: Any, template: BlockPagedBatchCache, rows: int, width: int,
                 device: torch.device) -> None:
        self.model = model
        self.rows, self.width = rows, width
        stage = BlockPagedBatchCache.empty(template._config, template.pool, max_batch_size=rows, max_blocks=width)
        # Every slot is live and the lengths advance in place on the device: the same tensors are
        # read and written by each replay.
        stage._graph_safe = True
        stage._cached_seq_len_py = None
        stage._slot_occupied = [True] * rows
        stage._free_slots = []
        for layer in stage.layers:
            layer._row_seq_lens = stage.seq_lens.clone()
            layer.is_initialized = True
        self.stage = stage
        self.ids = torch.zeros(rows, 1, dtype=torch.long, device=device)
        self.pos = torch.zeros(rows, 1, dtype=torch.long, device=device)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.logits: torch.Tensor | None = None
        self.eager_steps = 0
        self.replays = 0
        self.refused = ""

    def load(self, persistent: BlockPagedBatchCache, index: torch.Tensor, input_ids: torch.Tensor) -> None:
        stage = self.stage
        stage.block_tables.copy_(persistent.block_tables.index_select(0, index))
        stage.seq_lens.copy_(persistent.seq_lens.index_select(0, index))
        for layer in stage.layers:
            layer._row_seq_lens.copy_(stage.seq_lens)
        self.ids.copy_(input_ids.view(self.rows, 1))
        self.pos.copy_(stage.seq_lens.unsqueeze(1))

    def _forward(self) -> torch.Tensor:
        try:
            out = self.model(input_ids=self.ids, position_ids=self.pos, past_key_values=self.stage, use_cache=True,
                             logits_to_keep=1)
        finally:
            set_paged_decode_batch_metadata(None)
        return out.logits[:, -1, :]

    @torch.no_grad()
    def run(self, warmup_steps: int) -> torch.Tensor:
        if self.graph is not None:
            self.graph.replay()
            self.replays += 1
            return self.logits
        if self.eager_steps < warmup_steps:
            self.eager_steps += 1
            return self._forward()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = self._forward()
        self.graph, self.logits = graph, logits
        graph.replay()
        self.replays += 1
        return logits

    def store(self, persistent: BlockPagedBatchCache, index: torch.Tensor, slots: list[int],
              states: list[Any], new_lens: list[int]) -> None:
        lens = self.stage.seq_lens
        persistent.seq_lens.index_copy_(0, index, lens)
        for layer in persistent.layers:
            layer._row_seq_lens.index_copy_(0, index, lens)
        for state, slot, n in zip(states, slots, new_lens):
            cache = state.past_key_values
            if isinstance(cache, BlockPagedCache) and cache.block_table_ids == persistent.block_ids_rows[slot]:
                for layer in cache.layers:
                    layer.set_seq_length(n)
            else:
                state.past_key_values = persistent.extract_cache(slot, seq_len=n)

    def describe(self) -> dict[str, Any]:
        state = "refused" if self.refused else ("captured" if self.graph is not None else "warming")
        return {"rows": self.rows, "width": self.width, "state": state, "eager_steps": self.eager_steps,
                "replays": self.replays, "error": self.refused}


class CudaGraphDecodeManager:
    """HIP-graph decode for the worker's batched paged step (``worker_server.py:242-249,747-753``)."""

    def __init__(self, model: Any, device: torch.device | str, warmup_steps: int = 3, enabled: bool = False,
                 max_graphs: int = 8) -> None:
        self.model = model
        self.device = torch.device(device)
        self.warmup_steps = int(warmup_steps)
        self.enabled = bool(enabled)
        self.max_graphs = max(1, int(max_graphs))
        self.graphs: OrderedDict[tuple[int, int], StepGraph] = OrderedDict()
        self.off_reason = ""

    def _graph_for(self, persistent: BlockPagedBatchCache, rows: int) -> StepGraph:
        key = (rows, int(persistent.block_tables.shape[1]))
        graph = self.graphs.get(key)
        if graph is None:
            graph = StepGraph(self.model, persistent, rows, key[1], self.device)
            self.graphs[key] = graph
            while len(self.graphs) > self.max_graphs:
                self.graphs.popitem(last=False)
        self.graphs.move_to_end(key)
        return graph

    def try_decode(self, *, persistent: BlockPagedBatchCache, decode_states: list[Any],
                   input_ids: torch.Tensor) -> torch.Tensor | None:
        """This step's logits ``[rows, vocab]`` from a graph, or ``None`` to decode eagerly."""
        if self.off_reason or not (self.enabled or _opted_in()) or not torch.cuda.is_available():
            return None
        rows = len(decode_states)
        if rows == 0 or int(input_ids.numel()) != rows:
            return None
        slot_of = persistent._request_to_slot
        slots = [slot_of.get(s.req.request_id) for s in decode_states]
        if any(slot is None for slot in slots):
            return None
        graph = self._graph_for(persistent, rows)
        if graph.refused:
            return None
        new_lens = [s.past_key_values.get_seq_length() + 1 for s in decode_states]
        index = torch.tensor(slots, dtype=torch.long).to(self.device)
        graph.load(persistent, index, input_ids)
        try:
            logits = graph.run(self.warmup_steps)
        except Exception as exc:  # noqa: BLE001 - the worker decodes this key eagerly from now on
            graph.graph, graph.refused = None, f"{type(exc).__name__}: {exc}"
            try:
                torch.cuda.synchronize()
            except Exception as sticky:  # noqa: BLE001 - the device is unusable for graphs
                self.off_reason = f"device error after a failed capture: {sticky}"
            return None
        graph.store(persistent, index, slots, decode_states, new_lens)
        return logits

    def stats(self) -> dict[str, Any]:
        return {"enabled": self.enabled or _opted_in(), "off_reason": self.off_reason,
                "graphs": [g.describe() for g in self.graphs.values()]}


HipGraphDecodeManager = CudaGraphDecodeManager
