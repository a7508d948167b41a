"""Host wrappers of the decode-step glue kernels of libmxdecode.

* :func:`kv_append` — scatter new K/V states into a layer of a
  :class:`GpuKVBlockPool` (``GpuKVBlockPool.write_tokens_batch`` semantics,
  ``runtime/phase2/paged_kv_kernel.py:176-227``) in one launch;
* :func:`qkv_rope_append` — rotate q and k of a fused QKV projection output and
  append k, v at each row's position (the HF decoder layer's
  ``apply_rotary_pos_emb`` + ``BlockPagedBatchLayer.update`` write,
  ``runtime/phase2/paged_kv_cache.py:121-157``);
* :func:`add_rmsnorm` — residual add fused with RMSNorm;
* :func:`qkv_rope_append_splits` / :func:`add_rmsnorm_splits` — the same, reading
  the producing linear's split-K partials (``int8_linear_partials``) and
  forming its fp16 output on the fly;
* :func:`silu_mul` — SwiGLU's ``silu(gate) * up``;
* :func:`swiglu_interleaved` — the same for the interleaved gate||up projection, from its
  fp16 output or its split-K partials;
* :func:`rope_table` — the fp32 ``(cos, sin)`` table the fused RoPE reads,
  computed like transformers' default rotary embedding
  (``inv_freq = theta ** -(2i / D)``, angle ``pos * inv_freq`` in fp32).

All take device tensors and enqueue on the current stream; no call
synchronises or allocates except for the returned outputs when ``out`` is
omitted. Errors raise ``ValueError`` (bad arguments) or ``RuntimeError``.
"""

from __future__ import annotations

import torch

from . import _hip


def _i32(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    if t.dtype != torch.int32 or t.device != device or not t.is_contiguous():
        t = t.to(device=device, dtype=torch.int32).contiguous()
    return t


def _rows16(t: torch.Tensor) -> torch.Tensor:
    """2-D fp16 view with unit inner stride and 16-byte aligned rows (copied into rows padded to a
    multiple of 8 elements if needed)."""
    if t.stride(-1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
        n = int(t.shape[-1])
        buf = torch.empty(int(t.shape[0]), (n + 7) // 8 * 8, dtype=t.dtype, device=t.device)
        buf[:, :n].copy_(t)
        t = buf[:, :n]
    return t


def _lens_ptr(lens_out: torch.Tensor | None, b: int):
    if lens_out is None:
        return None
    if lens_out.dtype != torch.int32 or not lens_out.is_contiguous() or lens_out.numel() < b:
        raise ValueError("lens_out must be a contiguous int32 tensor of at least B elements")
    return lens_out.data_ptr()


def _used_ptr(used_blocks: torch.Tensor | None, nb: int, dev: torch.device):
    if used_blocks is None:
        return None
    if (used_blocks.dtype != torch.uint8 or used_blocks.numel() < nb or not used_blocks.is_contiguous()
            or used_blocks.device != dev):
        raise ValueError("used_blocks must be a contiguous uint8 device tensor of num_blocks entries")
    return used_blocks.data_ptr()


_argmax_workspaces: dict[tuple, torch.Tensor] = {}


def argmax_workspace(device: torch.device, m: int, n: int) -> torch.Tensor:
    """The chunk keys of ``mx_argmax_rows_split`` for ``[m, n]`` logits, cached per device and
    shape (created outside graph capture, like the attention workspaces)."""
    key = (torch.device(device), int(m), int(n))
    ws = _argmax_workspaces.get(key)
    if ws is None:
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("argmax workspace must be created before graph capture; run one eager call first")
        nbytes = int(_hip.load().mx_argmax_workspace_bytes(int(m), int(n)))
        ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=device)
        _argmax_workspaces[key] = ws
    return ws


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None, seq_lens: torch.Tensor | None = None,
                split: bool = True) -> torch.Tensor:
    """Greedy tokens ``[M]`` (int64) of fp16 ``logits [M, N]``; ``seq_lens`` (int32) is advanced by one.
    ``split`` (default) reduces each row in 4096-logit chunks across workgroups
    (``mx_argmax_rows_split``); ``split=False`` runs one workgroup per row (``mx_argmax_rows``).
    Both give torch.argmax's index."""
    _hip.require_device_tensor(logits, "logits")
    if logits.dtype != torch.float16 or logits.dim() != 2:
        raise ValueError("argmax_rows expects fp16 logits [M, N]")
    lg = _rows16(logits)
    m, n = (int(v) for v in lg.shape)
    out = torch.empty(m, dtype=torch.int64, device=lg.device) if out is None else out
    if out.dtype != torch.int64 or not out.is_contiguous() or out.numel() < m:
        raise ValueError("out must be a contiguous int64 tensor of M elements")
    if seq_lens is not None and (seq_lens.dtype != torch.int32 or not seq_lens.is_contiguous()):
        raise ValueError("seq_lens must be a contiguous int32 tensor")
    lens_p = seq_lens.data_ptr() if seq_lens is not None else None
    lib = _hip.load()
    if split and 0 < m <= 65535:
        ws = argmax_workspace(lg.device, m, n)
        _hip.check(lib.mx_argmax_rows_split(lg.data_ptr(), lg.stride(0), m, n, out.data_ptr(), lens_p, ws.data_ptr(),
                                            ws.numel(), _hip.stream_handle(lg.device)), "mx_argmax_rows_split")
    else:
        _hip.check(lib.mx_argmax_rows(lg.data_ptr(), lg.stride(0), m, n, out.data_ptr(), lens_p,
                                      _hip.stream_handle(lg.device)), "mx_argmax_rows")
    return out


def rope_table(max_pos: int, head_dim: int, theta: float, device: torch.device | str) -> torch.Tensor:
    """``[max_pos, head_dim // 2, 2]`` fp32 ``(cos, sin)`` of ``pos * theta ** -(2i / head_dim)``."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim))
    pos = torch.arange(max_pos, dtype=torch.float32)
    ang = pos[:, None] * inv_freq[None, :half]
    return torch.stack((ang.cos(), ang.sin()), dim=-1).contiguous().to(device)


def kv_append(k_layer: torch.Tensor, v_layer: torch.Tensor, block_tables: torch.Tensor, start_pos: torch.Tensor,
              key_states: torch.Tensor, value_states: torch.Tensor, err: torch.Tensor | None = None,
              used_blocks: torch.Tensor | None = None) -> None:
    """Write ``key/value_states [B, Hkv, T, D]`` at positions ``start_pos[b] + t`` of each row.

    ``k_layer``/``v_layer`` are per-layer pool views ``[num_blocks, Hkv, bs, D]``.
    Slots outside the table or the pool are skipped and flagged in ``err``
    (an int32 device word, OR-ed with 1) when given. ``used_blocks`` (uint8
    ``[num_blocks]``, optional) gets 1 at every block a token was written to.
    """
    _hip.require_device_tensor(key_states, "key_states")
    dev = k_layer.device
    if key_states.shape != value_states.shape or key_states.dim() != 4:
        raise ValueError("key_states and value_states must both be [B, Hkv, T, D]")
    if key_states.dtype != k_layer.dtype or k_layer.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("kv_append supports fp16 or bf16 states and pools of the same dtype")
    b, hkv, t, d = key_states.shape
    nb, hkv_p, bs, d_p = k_layer.shape
    if (hkv, d) != (hkv_p, d_p) or k_layer.stride() != v_layer.stride():
        raise ValueError("states do not match the pool layout")
    if k_layer.stride(3) != 1 or k_layer.stride(2) != d:
        raise ValueError("pool layer views must be contiguous within a (block, kv-head) run")
    if key_states.stride(3) != 1 or value_states.stride() != key_states.stride():
        key_states = key_states.contiguous()
        value_states = value_states.contiguous()
    tables = _i32(block_tables, dev)
    if tables.dim() != 2 or tables.shape[0] != b:
        raise ValueError("block_tables must be [B, max_blocks]")
    starts = _i32(start_pos.reshape(-1), dev)
    used = _used_ptr(used_blocks, nb, dev)
    lib = _hip.load()
    _hip.check(lib.mx_kv_append(
        key_states.data_ptr(), value_states.data_ptr(), key_states.stride(0), key_states.stride(1),
        key_states.stride(2), b, t, hkv, d, tables.data_ptr(), tables.stride(0), int(tables.shape[1]),
        starts.data_ptr(), k_layer.data_ptr(), v_layer.data_ptr(), k_layer.stride(0), k_layer.stride(1), bs, nb,
        err.data_ptr() if err is not None else None, used, _hip.stream_handle(dev)), "mx_kv_append")


def qkv_rope_append(qkv: torch.Tensor, rope: torch.Tensor, positions: torch.Tensor, q_out: torch.Tensor,
                    k_layer: torch.Tensor, v_layer: torch.Tensor, block_tables: torch.Tensor, num_heads: int,
                    num_kv_heads: int, err: torch.Tensor | None = None,
                    lens_out: torch.Tensor | None = None, used_blocks: torch.Tensor | None = None) -> torch.Tensor:
    """Rotate q, k of ``qkv [B, (Hq + 2 Hkv) * D]`` at ``positions [B]``; q -> ``q_out``, k, v -> the pool.

    ``lens_out`` (int32 ``[B]``, optional) receives ``positions + 1``; ``used_blocks`` (uint8
    ``[num_blocks]``, optional) gets 1 at every block a token was written to, as in :func:`kv_append`.
    """
    _hip.require_device_tensor(qkv, "qkv")
    dev = qkv.device
    nb, hkv, bs, d = k_layer.shape
    if hkv != num_kv_heads or qkv.shape[-1] != (num_heads + 2 * num_kv_heads) * d:
        raise ValueError("qkv width does not match (Hq + 2 Hkv) * D of the pool")
    if rope.dtype != torch.float32 or rope.dim() != 3 or rope.shape[1:] != (d // 2, 2) or not rope.is_contiguous():
        raise ValueError("rope must be a contiguous fp32 [max_pos, D/2, 2] table")
    if q_out.shape[-1] != num_heads * d:
        raise ValueError("q_out must be [B, Hq * D]")
    tables = _i32(block_tables, dev)
    pos = _i32(positions.reshape(-1), dev)
    qkv2 = _rows16(qkv.reshape(-1, qkv.shape[-1]))
    b = int(qkv2.shape[0])
    if tables.shape[0] != b or pos.shape[0] != b or q_out.reshape(-1, q_out.shape[-1]).shape[0] != b:
        raise ValueError("batch dimension mismatch")
    q2 = q_out.reshape(b, -1)
    if q2.data_ptr() != q_out.data_ptr() or q2.stride(-1) != 1:
        raise ValueError("q_out must be a row-major [B, Hq * D] buffer")
    lib = _hip.load()
    _hip.check(lib.mx_qkv_rope_append(
        qkv2.data_ptr(), qkv2.stride(0), b, num_heads, num_kv_heads, d, rope.data_ptr(), int(rope.shape[0]),
        pos.data_ptr(), q2.data_ptr(), q2.stride(0), k_layer.data_ptr(), v_layer.data_ptr(), k_layer.stride(0),
        k_layer.stride(1), tables.data_ptr(), tables.stride(0), int(tables.shape[1]), bs, nb,
        err.data_ptr() if err is not None else None, _lens_ptr(lens_out, b), _used_ptr(used_blocks, nb, dev),
        _hip.stream_handle(dev)), "mx_qkv_rope_append")
    return q_out


def qkv_rope_append_splits(partials: torch.Tensor, splits: int, bias: torch.Tensor | None, rope: torch.Tensor,
                           positions: torch.Tensor, q_out: torch.Tensor, k_layer: torch.Tensor,
                           v_layer: torch.Tensor, block_tables: torch.Tensor, num_heads: int, num_kv_heads: int,
                           err: torch.Tensor | None = None, lens_out: torch.Tensor | None = None,
                           used_blocks: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`qkv_rope_append` with the QKV projection as fp32 split partials ``[splits, B, width]``
    (16-byte aligned, as is ``bias``)."""
    _hip.require_device_tensor(partials, "partials")
    dev = partials.device
    nb, hkv, bs, d = k_layer.shape
    width = (num_heads + 2 * num_kv_heads) * d
    b = int(q_out.shape[0])
    if hkv != num_kv_heads or partials.dtype != torch.float32 or partials.numel() < splits * b * width:
        raise ValueError("partials must be fp32 [splits, B, (Hq + 2 Hkv) * D]")
    if rope.dtype != torch.float32 or rope.dim() != 3 or rope.shape[1:] != (d // 2, 2) or not rope.is_contiguous():
        raise ValueError("rope must be a contiguous fp32 [max_pos, D/2, 2] table")
    tables = _i32(block_tables, dev)
    pos = _i32(positions.reshape(-1), dev)
    q2 = q_out.reshape(b, -1)
    lib = _hip.load()
    _hip.check(lib.mx_qkv_rope_append_splits(
        partials.data_ptr(), splits, bias.data_ptr() if bias is not None else None, b, num_heads, num_kv_heads, d,
        rope.data_ptr(), int(rope.shape[0]), pos.data_ptr(), q2.data_ptr(), q2.stride(0), k_layer.data_ptr(),
        v_layer.data_ptr(), k_layer.stride(0), k_layer.stride(1), tables.data_ptr(), tables.stride(0),
        int(tables.shape[1]), bs, nb, err.data_ptr() if err is not None else None, _lens_ptr(lens_out, b),
        _used_ptr(used_blocks, nb, dev), _hip.stream_handle(dev)), "mx_qkv_rope_append_splits")
    return q_out


QKV_ROPE_MAX_ROWS = 32


def qkv_linear_rope_append(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
                           rope: torch.Tensor, positions: torch.Tensor, q_out: torch.Tensor, k_layer: torch.Tensor,
                           v_layer: torch.Tensor, block_tables: torch.Tensor, num_heads: int, num_kv_heads: int,
                           err: torch.Tensor | None = None, lens_out: torch.Tensor | None = None,
                           used_blocks: torch.Tensor | None = None) -> torch.Tensor:
    """The int8 QKV projection of ``x [B, K]`` (packed fused-QKV weight, ``B <= 32``) and
    :func:`qkv_rope_append_splits` in one launch (``mx_w8a16_qkv_rope_append``)."""
    _hip.require_device_tensor(x, "x")
    dev = x.device
    nb, hkv, bs, d = k_layer.shape
    x2 = _rows16(x.reshape(-1, x.shape[-1]))
    b, k = (int(v) for v in x2.shape)
    if hkv != num_kv_heads:
        raise ValueError("num_kv_heads does not match the pool")
    if not 1 <= b <= QKV_ROPE_MAX_ROWS:
        raise ValueError(f"the fused QKV + RoPE launch takes 1..{QKV_ROPE_MAX_ROWS} rows, got {b}")
    n = (num_heads + 2 * num_kv_heads) * d
    if scale.numel() != n or (bias is not None and bias.numel() != n):
        raise ValueError("scale (and bias) must have (Hq + 2 Hkv) * D entries")
    if packed.dtype != torch.uint8 or packed.numel() != n * k or not packed.is_contiguous():
        raise ValueError(f"packed must be the contiguous uint8 tile layout of a [{n}, {k}] weight")
    for t, name in ((packed, "packed"), (scale, "scale")) + (((bias, "bias"),) if bias is not None else ()):
        _hip.require_device_tensor(t, name)
    if rope.dtype != torch.float32 or rope.dim() != 3 or rope.shape[1:] != (d // 2, 2) or not rope.is_contiguous():
        raise ValueError("rope must be a contiguous fp32 [max_pos, D/2, 2] table")
    tables = _i32(block_tables, dev)
    pos = _i32(positions.reshape(-1), dev)
    if tables.shape[0] != b or pos.shape[0] != b:
        raise ValueError("batch dimension mismatch")
    q2 = q_out.reshape(b, -1)
    if q2.data_ptr() != q_out.data_ptr() or q2.stride(-1) != 1 or q2.shape[-1] != num_heads * d:
        raise ValueError("q_out must be a row-major [B, Hq * D] buffer")
    lib = _hip.load()
    _hip.check(lib.mx_w8a16_qkv_rope_append(
        x2.data_ptr(), b, k, x2.stride(0), packed.data_ptr(), scale.data_ptr(),
        bias.data_ptr() if bias is not None else None, num_heads, num_kv_heads, d, rope.data_ptr(),
        int(rope.shape[0]), pos.data_ptr(), q2.data_ptr(), q2.stride(0), k_layer.data_ptr(), v_layer.data_ptr(),
        k_layer.stride(0), k_layer.stride(1), tables.data_ptr(), tables.stride(0), int(tables.shape[1]), bs, nb,
        err.data_ptr() if err is not None else None, _lens_ptr(lens_out, b), _used_ptr(used_blocks, nb, dev),
        _hip.stream_handle(dev)), "mx_w8a16_qkv_rope_append")
    return q_out


def add_rmsnorm_splits(partials: torch.Tensor, splits: int, bias: torch.Tensor | None, weight: torch.Tensor,
                       eps: float, out: torch.Tensor, residual: torch.Tensor | None = None,
                       residual_out: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`add_rmsnorm` with x as the producing linear's fp32 split partials ``[splits, M, H]``."""
    _hip.require_device_tensor(partials, "partials")
    m, h = (int(v) for v in out.shape)
    if partials.dtype != torch.float32 or partials.numel() < splits * m * h:
        raise ValueError("partials must be fp32 [splits, M, H]")
    r2 = _rows16(residual.reshape(m, h)) if residual is not None else None
    ro2 = residual_out.view(m, h) if residual_out is not None else None
    lib = _hip.load()
    _hip.check(lib.mx_add_rmsnorm_splits(
        partials.data_ptr(), splits, bias.data_ptr() if bias is not None else None,
        r2.data_ptr() if r2 is not None else None, r2.stride(0) if r2 is not None else 0, weight.data_ptr(), m, h,
        float(eps), out.data_ptr(), out.stride(0), ro2.data_ptr() if ro2 is not None else None,
        ro2.stride(0) if ro2 is not None else 0, _hip.stream_handle(partials.device)), "mx_add_rmsnorm_splits")
    return out


def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
                out: torch.Tensor | None = None, residual_out: torch.Tensor | None = None,
                rows: torch.Tensor | None = None) -> torch.Tensor:
    """``h = x (+ residual)``; ``residual_out = h``; returns ``RMSNorm(h) * weight`` (fp16 ``[M, H]``).

    With ``rows`` (int64 ``[M]``), row m of x is ``x[rows[m]]`` (an embedding lookup); an index
    outside ``[0, len(x))`` reads a zero row (memory-safe; no device-side assert as in torch).
    """
    _hip.require_device_tensor(x, "x")
    if x.dtype != torch.float16 or weight.dtype != torch.float16:
        raise ValueError("add_rmsnorm supports fp16")
    x2 = _rows16(x.reshape(-1, x.shape[-1]))
    m, h = x2.shape
    if rows is not None:
        if rows.dtype != torch.int64 or not rows.is_contiguous():
            raise ValueError("rows must be a contiguous int64 tensor")
        m = int(rows.numel())
    r2 = _rows16(residual.reshape(m, h)) if residual is not None else None
    out = torch.empty((m, h), dtype=x2.dtype, device=x2.device) if out is None else out
    o2 = out.view(m, h)
    ro2 = residual_out.view(m, h) if residual_out is not None else None
    w = weight.contiguous()
    lib = _hip.load()
    _hip.check(lib.mx_add_rmsnorm(
        x2.data_ptr(), x2.stride(0), rows.data_ptr() if rows is not None else None, int(x2.shape[0]),
        r2.data_ptr() if r2 is not None else None, r2.stride(0) if r2 is not None else 0,
        w.data_ptr(), m, h, float(eps), o2.data_ptr(), o2.stride(0),
        ro2.data_ptr() if ro2 is not None else None, ro2.stride(0) if ro2 is not None else 0,
        _hip.stream_handle(x.device)), "mx_add_rmsnorm")
    return out


def swiglu_interleaved(gate_up: torch.Tensor | None, inter: int, partials: torch.Tensor | None = None,
                       splits: int = 0, bias: torch.Tensor | None = None, rows: int | None = None,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(g) * u`` of the interleaved gate||up projection (``gateup_interleave`` row order).

    From its fp16 output ``gate_up [M, 2*inter]``, or (``gate_up=None``) from its split-K
    ``partials`` (``[splits, rows, 2*inter]`` fp32, :func:`int8_linear_partials`) plus ``bias``,
    rounded as the projection's own output. Returns fp16 ``[M, inter]``.
    """
    if (gate_up is None) == (partials is None):
        raise ValueError("give exactly one of gate_up and partials")
    if gate_up is not None:
        _hip.require_device_tensor(gate_up, "gate_up")
        g2 = _rows16(gate_up.reshape(-1, gate_up.shape[-1]))
        m = int(g2.shape[0])
        if g2.dtype != torch.float16 or g2.shape[1] != 2 * inter:
            raise ValueError("gate_up must be fp16 [M, 2*inter]")
        dev = g2.device
    else:
        _hip.require_device_tensor(partials, "partials")
        if rows is None or partials.dtype != torch.float32 or partials.numel() < splits * rows * 2 * inter:
            raise ValueError("partials must be fp32 [splits, rows, 2*inter] (give rows and splits)")
        m, dev = int(rows), partials.device
    out = torch.empty(m, inter, dtype=torch.float16, device=dev) if out is None else out
    o2 = out.view(m, inter)
    b = bias.contiguous() if bias is not None else None
    _hip.check(_hip.load().mx_swiglu_interleaved(
        g2.data_ptr() if gate_up is not None else None, g2.stride(0) if gate_up is not None else 0,
        partials.data_ptr() if partials is not None else None, int(splits), b.data_ptr() if b is not None else None,
        m, int(inter), o2.data_ptr(), o2.stride(0), _hip.stream_handle(dev)), "mx_swiglu_interleaved")
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gate_up[:, :I]) * gate_up[:, I:]`` for fp16 ``gate_up [M, 2I]``."""
    _hip.require_device_tensor(gate_up, "gate_up")
    if gate_up.dtype != torch.float16:
        raise ValueError("silu_mul supports fp16")
    g2 = _rows16(gate_up.reshape(-1, gate_up.shape[-1]))
    m, two_i = g2.shape
    if two_i % 2:
        raise ValueError("gate_up width must be even")
    i = two_i // 2
    out = torch.empty((m, i), dtype=torch.float16, device=gate_up.device) if out is None else out
    o2 = out.view(m, i)
    lib = _hip.load()
    _hip.check(lib.mx_silu_mul(g2.data_ptr(), g2.stride(0), m, i, o2.data_ptr(), o2.stride(0),
                               _hip.stream_handle(gate_up.device)), "mx_silu_mul")
    return out
