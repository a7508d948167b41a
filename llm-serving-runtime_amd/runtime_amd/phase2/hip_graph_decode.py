"""HIP-graph capture and replay of the HF paged decode step.

Drop-in for ``runtime/phase2/cuda_graph_decode.py``: the same names
(``cuda_graph_enabled``, ``cuda_graph_try_hf``, ``CudaGraphBucket``,
``CudaGraphDecodeManager``), the same ``try_decode(persistent=, decode_states=,
input_ids=)`` contract (logits ``[B, vocab]`` or ``None`` for the eager path)
and the same buckets keyed by ``(batch_size, max_blocks rounded up to a power
of two)`` (``:54-59``), each with its own dense :class:`BlockPagedBatchCache`
marked ``_graph_safe`` (``:61-95``). ``torch.cuda.CUDAGraph`` is a HIP graph on
ROCm.

Why the capture holds here while the reference keeps it opt-in and expects it to
fail (``:16-19,147-150``: host syncs inside the forward invalidate the capture):
on this path the decode forward makes no host round trip. The ``block_paged``
implementation has no mask function, so transformers builds no mask and never
asks the cache for lengths; the positions are passed in; the KV writes report
table overruns through the pool's device error word
(``GpuKVBlockPool.check_write_errors``); the attention and linear workspaces are
sized by the eager warm-up steps before capture. ``enabled=True`` turns the
manager on without the environment variables.

Differences from the reference (documented, observable):

* the forward gets ``position_ids`` (each row's length) in a static buffer; the
  reference passes a ``[B]`` ``cache_position`` (``:104-107,204-210``), which HF
  reads as one position sequence for the whole batch;
* rows are copied into the bucket and back with device-side ``index_copy_``; the
  reference writes each slot with a host-read length per layer (``:116-132``);
* after capture, the graph's recording step has not advanced the KV lengths
  (they are restored before capture, ``:185-198``) and this call's logits come
  from one replay, so every call returns the logits of a replayed graph.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Any

import torch

from .paged_attention_hip import set_paged_decode_batch_metadata
from .paged_kv_cache import BlockPagedBatchCache, BlockPagedBatchLayer


def cuda_graph_enabled() -> bool:
    return os.getenv("PHASE2_CUDA_GRAPH", "0").strip() == "1"


def cuda_graph_try_hf() -> bool:
    return os.getenv("PHASE2_CUDA_GRAPH_TRY_HF", "0").strip() == "1"


@dataclass
class CudaGraphBucket:
    batch_size: int
    max_blocks: int
    static_input_ids: torch.Tensor
    dense_cache: BlockPagedBatchCache
    static_position_ids: torch.Tensor
    graph: torch.cuda.CUDAGraph | None = None
    static_logits: torch.Tensor | None = None
    warmups_done: int = 0
    capture_failed: bool = False
    capture_error: str = ""
    replays: int = 0


@dataclass
class CudaGraphDecodeManager:
    """Bucketed HIP-graph decode keyed by ``(batch_size, max_blocks)`` (``cuda_graph_decode.py:41-245``)."""

    model: Any
    device: torch.device
    warmup_steps: int = 3
    enabled: bool = False  # True: capture without PHASE2_CUDA_GRAPH / PHASE2_CUDA_GRAPH_TRY_HF
    buckets: dict[tuple[int, int], CudaGraphBucket] = field(default_factory=dict)
    disabled: bool = False
    disable_reason: str = ""

    def _bucket_key(self, batch_size: int, max_blocks: int) -> tuple[int, int]:
        quantized = 1
        while quantized < max_blocks:
            quantized *= 2
        return batch_size, quantized

    def _ensure_bucket(self, batch_size: int, max_blocks: int, template: BlockPagedBatchCache) -> CudaGraphBucket:
        key = self._bucket_key(batch_size, max_blocks)
        bucket = self.buckets.get(key)
        if bucket is not None:
            return bucket
        dense = BlockPagedBatchCache.empty(template._config, template.pool, max_batch_size=batch_size,
                                           max_blocks=key[1])
        dense._graph_safe = True
        dense._cached_seq_len_py = None  # lengths are never read on the host: capacity stands in
        for i in range(batch_size):
            dense._slot_occupied[i] = True
        dense._free_slots = []
        for layer in dense.layers:
            layer._row_seq_lens = dense.seq_lens.clone()
        bucket = CudaGraphBucket(
            batch_size=batch_size, max_blocks=key[1],
            static_input_ids=torch.zeros(batch_size, 1, device=self.device, dtype=torch.long),
            dense_cache=dense,
            static_position_ids=torch.zeros(batch_size, 1, device=self.device, dtype=torch.long))
        self.buckets[key] = bucket
        return bucket

    def _copy_rows_into_bucket(self, bucket: CudaGraphBucket, source: BlockPagedBatchCache, slots: list[int],
                               input_ids: torch.Tensor) -> None:
        dense = bucket.dense_cache
        index = torch.tensor(slots, dtype=torch.long).to(self.device)
        width = min(int(source.block_tables.shape[1]), bucket.max_blocks)
        dense.block_tables.zero_()
        dense.block_tables[:, :width].copy_(source.block_tables.index_select(0, index)[:, :width])
        dense.seq_lens.copy_(source.seq_lens.index_select(0, index))
        for i, slot in enumerate(slots):
            dense.block_ids_rows[i] = list(source.block_ids_rows[slot])
        for layer in dense.layers:
            layer._row_seq_lens.copy_(dense.seq_lens)
            layer.is_initialized = True
        bucket.static_input_ids.copy_(input_ids)
        bucket.static_position_ids.copy_(dense.seq_lens.to(torch.long).unsqueeze(1))

    def _write_back(self, persistent: BlockPagedBatchCache, bucket: CudaGraphBucket, slots: list[int],
                    decode_states: list[Any]) -> None:
        dense = bucket.dense_cache
        persistent.write_back_dense(dense, slots)
        for idx, state in enumerate(decode_states):
            seq_len = state.past_key_values.get_seq_length() + 1
            state.past_key_values = persistent.extract_cache(slots[idx], seq_len=seq_len)

    def try_decode(self, *, persistent: BlockPagedBatchCache, decode_states: list[Any],
                   input_ids: torch.Tensor) -> torch.Tensor | None:
        """Replay (capturing first if needed) the bucket's graph; logits ``[B, vocab]`` or None."""
        if self.disabled or not torch.cuda.is_available():
            return None
        if not self.enabled and not (cuda_graph_enabled() and cuda_graph_try_hf()):
            return None
        batch_size = len(decode_states)
        if batch_size <= 0:
            return None
        try:
            slots = [persistent._request_to_slot[s.req.request_id] for s in decode_states]
        except KeyError:
            return None
        max_blocks = max(max(len(persistent.block_ids_rows[s]), 1) for s in slots)
        bucket = self._ensure_bucket(batch_size, max_blocks, persistent)
        if bucket.capture_failed:
            return None
        self._copy_rows_into_bucket(bucket, persistent, slots, input_ids)
        if bucket.graph is None:
            logits = self._capture(bucket)
            if logits is None:
                return None
        else:
            bucket.graph.replay()
            bucket.replays += 1
            logits = bucket.static_logits
        self._write_back(persistent, bucket, slots, decode_states)
        return logits

    def _forward(self, bucket: CudaGraphBucket) -> Any:
        try:
            return self.model(input_ids=bucket.static_input_ids, position_ids=bucket.static_position_ids,
                              past_key_values=bucket.dense_cache, use_cache=True)
        finally:
            set_paged_decode_batch_metadata(None)

    def _capture(self, bucket: CudaGraphBucket) -> torch.Tensor | None:
        """Warm up (eager steps, which also size every workspace), then capture and replay once."""
        try:
            if bucket.warmups_done < self.warmup_steps:
                with torch.no_grad():
                    out = self._forward(bucket)
                bucket.warmups_done += 1
                return out.logits[:, -1, :]
            dense = bucket.dense_cache
            seq_before = dense.seq_lens.clone()
            rows_before = [layer._row_seq_lens.clone() for layer in dense.layers]
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.no_grad(), torch.cuda.graph(graph):
                out = self._forward(bucket)
            # Recording runs nothing; restore the lengths the capture's Python side touched.
            dense.seq_lens.copy_(seq_before)
            for layer, snap in zip(dense.layers, rows_before):
                layer._row_seq_lens.copy_(snap)
            bucket.graph = graph
            bucket.static_logits = out.logits[:, -1, :]
            graph.replay()
            bucket.replays += 1
            return bucket.static_logits
        except Exception as exc:  # noqa: BLE001 - the worker falls back to eager decode
            bucket.capture_failed = True
            bucket.capture_error = f"capture failed: {exc}"
            bucket.graph = None
            self.disabled = True
            self.disable_reason = bucket.capture_error
            try:
                torch.cuda.synchronize()
            except Exception:  # noqa: BLE001
                pass
            return None

    def stats(self) -> dict[str, Any]:
        return {
            "enabled": self.enabled or cuda_graph_enabled(),
            "try_hf": self.enabled or cuda_graph_try_hf(),
            "disabled": self.disabled,
            "disable_reason": self.disable_reason,
            "buckets": [{"batch_size": b.batch_size, "max_blocks": b.max_blocks, "captured": b.graph is not None,
                         "capture_failed": b.capture_failed, "capture_error": b.capture_error,
                         "warmups_done": b.warmups_done, "replays": b.replays} for b in self.buckets.values()],
        }


HipGraphDecodeManager = CudaGraphDecodeManager
HipGraphBucket = CudaGraphBucket
