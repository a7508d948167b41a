"""Paged-attention decode on the HIP kernel of libmxdecode (gfx950).

Drop-in for ``runtime/phase2/paged_attention_triton.py``: the same public names
and argument meanings, dispatching to ``mx_paged_attn_decode`` instead of the
four Triton kernels (``:148-457``). One launch covers any batch and any mix of
context lengths; there is no per-row loop (``:537-552``), no host sync
(``seq_lens.max().item()``, ``:495``) and no fp32 scratch-then-cast
(``:500,533-535``); the kernel writes the query dtype directly.

Differences from the reference that a caller can observe:

* device tensors only: a CPU query raises ``ValueError`` instead of running a
  torch fallback (``:761-775``);
* fp16 or bf16 queries and pools (one dtype), ``head_dim`` in {64, 128}, ``block_size``
  in {4, 8, 16, 32} (``ValueError`` otherwise); any GQA group (above 8 the kernel splits a
  kv-head's query heads into groups of at most 8 and reads its K/V once per group);
* ``seq_len == 0`` rows produce zeros (the reference divides by zero,
  ``:238``); ``paged_attention_decode`` still rejects ``seq_len <= 0`` (``:789-790``);
* the returned tensor is freshly allocated, never an alias of a cached buffer
  (the reference's fp32 path aliases its scratch, ``:108-115,600``);
* ``PagedDecodeBatchMetadata.shared_blocks`` (default ``False``) says that rows may
  alias block ids (a shared prefix); the kernel then reads K/V with the default cache
  policy instead of streaming loads. The result is the same either way.
"""

from __future__ import annotations

import contextvars
import math
import os
import threading
from dataclasses import dataclass
from typing import TYPE_CHECKING

import torch
import torch.nn.functional as F

from . import _hip

if TYPE_CHECKING:
    from .paged_kv_kernel import GpuKVBlockPool

_CHUNK_TOKENS = int(os.getenv("MX_PAGED_ATTN_CHUNK_TOKENS", "0"))
MX_PA_SHARED_BLOCKS = 1
MX_PA_BF16 = 2
MX_PA_PLAN_WRITE = 4  # also record each wave's tiles in the workspace (block size >= 16)
MX_PA_PLAN_READ = 8   # start from the tiles a PLAN_WRITE call recorded (same lengths and tables)
_DTYPE_FLAGS = {torch.float16: 0, torch.bfloat16: MX_PA_BF16}

_decode_batch_metadata: contextvars.ContextVar["PagedDecodeBatchMetadata | None"] = contextvars.ContextVar(
    "paged_decode_batch_metadata", default=None
)


@dataclass(frozen=True)
class PagedDecodeBatchMetadata:
    """Batched decode metadata (``paged_attention_triton.py:43-50``)."""

    pool: "GpuKVBlockPool"
    layer_idx: int
    block_tables: torch.Tensor  # [B, max_blocks] int32
    seq_lens: torch.Tensor  # [B] int32, KV length to attend over (includes current token)
    shared_blocks: bool = False  # rows may alias block ids (MX_PA_SHARED_BLOCKS)


PagedDecodeContext = PagedDecodeBatchMetadata


def set_paged_decode_batch_metadata(meta: PagedDecodeBatchMetadata | None) -> contextvars.Token:
    return _decode_batch_metadata.set(meta)


def reset_paged_decode_batch_metadata(token: contextvars.Token) -> None:
    _decode_batch_metadata.reset(token)


def get_paged_decode_batch_metadata() -> PagedDecodeBatchMetadata | None:
    return _decode_batch_metadata.get()


def set_paged_decode_context(ctx: PagedDecodeBatchMetadata | None) -> None:
    _decode_batch_metadata.set(ctx)


def get_paged_decode_context() -> PagedDecodeBatchMetadata | None:
    return get_paged_decode_batch_metadata()


def hip_kernel_available() -> bool:
    """Counterpart of ``triton_available()`` (``:78-79``): the HIP library loads and a device is present."""
    return _hip.available()


# --------------------------------------------------------------------------
# Workspace: fp32 split partials and the error word, keyed by shape like the
# reference's scratch caches (:90-115). Zeroed once at allocation.
# --------------------------------------------------------------------------
_workspaces: dict[tuple, torch.Tensor] = {}
_ws_lock = threading.Lock()


def _workspace(device: torch.device, key: tuple) -> tuple[torch.Tensor, int]:
    nbytes = int(_hip.load().mx_paged_attn_workspace_bytes(*key))
    full_key = (device, *key)
    ws = _workspaces.get(full_key)
    if ws is None:
        with _ws_lock:
            ws = _workspaces.get(full_key)
            if ws is None:
                if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
                    raise RuntimeError(
                        "paged attention workspace must be created before graph capture; "
                        "call warmup_paged_attention_kernel or run one eager step first"
                    )
                ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
                _workspaces[full_key] = ws
    return ws, nbytes


def workspace_error_flag(device: torch.device | None = None) -> int:
    """OR of the error words of all cached workspaces (one host sync). Nonzero: an
    out-of-range block id was met and skipped since the workspace was created."""
    flag = 0
    with _ws_lock:
        cached = list(_workspaces.items())
    for key, ws in cached:
        if device is not None and key[0] != device:
            continue
        off = int(_hip.load().mx_paged_attn_error_offset(*key[1:]))
        flag |= int(ws[off:off + 4].view(torch.int32).item())
    return flag


def _decode(query: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor, block_tables: torch.Tensor,
            seq_lens: torch.Tensor, scaling: float, num_kv_groups: int, out: torch.Tensor | None = None,
            shared_blocks: bool = False, plan: int = 0) -> torch.Tensor:
    """One ``mx_paged_attn_decode`` call. ``plan`` is 0, ``MX_PA_PLAN_WRITE`` or ``MX_PA_PLAN_READ``:
    a decode step records the tile plan at its first layer and the later layers, whose lengths and
    tables are the same, start from it (block size >= 16, not with ``shared_blocks``)."""
    bsz, hq, q_len, d = query.shape
    if q_len != 1:
        raise ValueError("paged decode expects q_len=1")
    if query.dtype not in _DTYPE_FLAGS or k_layer.dtype != query.dtype or v_layer.dtype != query.dtype:
        raise ValueError(f"HIP paged decode supports fp16 or bf16 query and pool of one dtype, got "
                         f"{query.dtype}/{k_layer.dtype}/{v_layer.dtype}")
    nb, hkv, bs, dk = k_layer.shape
    if tuple(v_layer.shape) != tuple(k_layer.shape) or v_layer.stride() != k_layer.stride():
        raise ValueError("K and V layer views must have the same shape and strides")
    if dk != d:
        raise ValueError(f"head_dim mismatch: query {d} vs pool {dk}")
    if hkv * num_kv_groups != hq:
        raise ValueError(f"num_heads {hq} != num_kv_heads {hkv} * num_kv_groups {num_kv_groups}")
    if k_layer.stride(3) != 1 or k_layer.stride(2) != d:
        raise ValueError("pool layer views must be contiguous within a (block, kv-head) run")
    if query.stride(3) != 1:
        query = query.contiguous()
    if block_tables.dim() != 2 or block_tables.shape[0] != bsz:
        raise ValueError("block_tables must be [B, max_blocks]")
    if block_tables.dtype != torch.int32 or block_tables.stride(1) != 1 or block_tables.device != query.device:
        block_tables = block_tables.to(device=query.device, dtype=torch.int32).contiguous()
    if seq_lens.dtype != torch.int32 or seq_lens.device != query.device or not seq_lens.is_contiguous():
        seq_lens = seq_lens.to(device=query.device, dtype=torch.int32).contiguous()
    max_blocks = int(block_tables.shape[1])
    if out is None:
        out = torch.empty((bsz, hq, 1, d), dtype=query.dtype, device=query.device)
    elif (tuple(out.shape) != (bsz, hq, 1, d) or out.dtype != query.dtype or out.stride(3) != 1
          or out.device != query.device):
        raise ValueError("out must be a [B, heads, 1, dim] tensor of the query dtype with unit inner stride")
    if bsz == 0:
        return out
    key = (bsz, hq, hkv, d, max_blocks, bs, _CHUNK_TOKENS)
    ws, nbytes = _workspace(query.device, key)
    lib = _hip.load()
    _hip.check(
        lib.mx_paged_attn_decode(
            query.data_ptr(), query.stride(0), query.stride(1), k_layer.data_ptr(), v_layer.data_ptr(),
            k_layer.stride(0), k_layer.stride(1), block_tables.data_ptr(), block_tables.stride(0), max_blocks,
            seq_lens.data_ptr(), bsz, hq, hkv, d, bs, nb, float(scaling), out.data_ptr(), out.stride(0),
            out.stride(1), ws.data_ptr(), nbytes, _CHUNK_TOKENS,
            _DTYPE_FLAGS[query.dtype] | (MX_PA_SHARED_BLOCKS if shared_blocks else 0) | plan,
            _hip.stream_handle(query.device),
        ),
        "mx_paged_attn_decode",
    )
    return out


def paged_attention_decode_batched(query: torch.Tensor, metadata: PagedDecodeBatchMetadata, num_kv_groups: int,
                                   scaling: float) -> torch.Tensor:
    """Batched decode: ``query [B, heads, 1, dim]`` -> ``[B, heads, 1, dim]`` (``:745-775``)."""
    if query.shape[0] != metadata.block_tables.shape[0]:
        raise ValueError("query batch size must match block_tables rows")
    _hip.require_device_tensor(query, "query")
    pool = metadata.pool
    pool._ensure_pools()
    k_layer = pool.k_layer_view(metadata.layer_idx)
    v_layer = pool.v_layer_view(metadata.layer_idx)
    return _decode(query, k_layer, v_layer, metadata.block_tables, metadata.seq_lens, scaling, num_kv_groups,
                   shared_blocks=metadata.shared_blocks)


def paged_attention_decode(query: torch.Tensor, pool: "GpuKVBlockPool", layer_idx: int, block_ids: list[int],
                           seq_len: int, num_kv_groups: int, scaling: float,
                           block_table: torch.Tensor | None = None) -> torch.Tensor:
    """Decode-step attention for batch=1 (``:778-802``)."""
    if seq_len <= 0:
        raise ValueError("seq_len must be positive for paged decode")
    num_logical = math.ceil(seq_len / pool.block_size_tokens)
    if block_table is None:
        table = torch.tensor(block_ids[:num_logical], device=query.device, dtype=torch.int32)
    else:
        table = block_table[:num_logical]
    meta = PagedDecodeBatchMetadata(
        pool=pool,
        layer_idx=layer_idx,
        block_tables=table.unsqueeze(0),
        seq_lens=torch.tensor([seq_len], device=query.device, dtype=torch.int32),
    )
    return paged_attention_decode_batched(query, meta, num_kv_groups, scaling)


def warmup_paged_attention_kernel(pool: "GpuKVBlockPool", *, num_heads: int, num_kv_groups: int, head_dim: int,
                                  block_ids: list[int], seq_len: int = 16) -> None:
    """Load the library and run one tiny decode (``:118-143``)."""
    if not hip_kernel_available() or pool.device.type != "cuda":
        return
    query = torch.zeros(1, num_heads, 1, head_dim, device=pool.device, dtype=pool.dtype)
    paged_attention_decode(query=query, pool=pool, layer_idx=0, block_ids=block_ids, seq_len=seq_len,
                           num_kv_groups=num_kv_groups, scaling=head_dim**-0.5,
                           block_table=torch.tensor(block_ids, device=pool.device, dtype=torch.int32))
    torch.cuda.synchronize(pool.device)


def reference_sdpa_attention(query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scaling: float,
                             num_kv_groups: int) -> torch.Tensor:
    """API-compatible export of the reference's SDPA helper (``:805-817``).

    Kept because callers import it from this module; the decode path above
    never calls it.
    """
    if num_kv_groups > 1:
        keys = keys.repeat_interleave(num_kv_groups, dim=1)
        values = values.repeat_interleave(num_kv_groups, dim=1)
    attn = torch.matmul(query, keys.transpose(2, 3).contiguous()) * scaling
    attn = F.softmax(attn, dim=-1, dtype=torch.float32).to(query.dtype)
    return torch.matmul(attn, values)
