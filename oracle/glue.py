"""CPU restatement of the decode-step glue (torch on the CPU).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* :func:`append_tokens` — ``GpuKVBlockPool.write_tokens_batch``
  (``runtime/phase2/paged_kv_kernel.py:176-227``): token ``t`` of row ``b`` goes
  to ``pos = start[b] + t``, block ``table[b, pos // bs]``, offset ``pos % bs``;
  a per-token loop as in the reference (``:217-227``). Out-of-range slots are
  skipped and reported (the reference raises; the device kernel flags).
* :func:`rope_rotate_half` — transformers' ``apply_rotary_pos_emb`` with the
  default rotary embedding (``inv_freq = theta ** -(2i / D)``, pairs ``i`` and
  ``i + D/2``); angles rounded to fp32 as transformers forms them, cos/sin and
  the rotation in float64.
* :func:`add_rmsnorm` / :func:`silu_mul` — transformers' Qwen2/Llama RMSNorm and
  SwiGLU MLP product with fp16 storage at the points where an fp16 model
  rounds (the residual sum, the normalised value, the products), fp32 math.

Parity pins (``tests/test_oracle_glue.py``): ``append_tokens`` against the pool
oracle's ``write_tokens`` and the reference's round-trip KAT shape;
``rope_rotate_half`` against transformers' own rotary embedding +
``apply_rotary_pos_emb`` (library code), identity at position 0, pair-norm
preservation and angle additivity; ``add_rmsnorm`` and ``silu_mul`` against
transformers' ``Qwen2RMSNorm`` / ``Qwen2MLP`` run in fp16-rounded fp32 and
against closed forms (a constant row normalises to ``sign * weight``,
``silu(0) = 0``).
"""

from __future__ import annotations

import torch


def append_tokens(k_layer: torch.Tensor, v_layer: torch.Tensor, block_tables: torch.Tensor, start_pos,
                  key_states: torch.Tensor, value_states: torch.Tensor) -> list[tuple[int, int]]:
    """Write ``[B, Hkv, T, D]`` states into ``[nb, Hkv, bs, D]`` views; returns skipped ``(b, t)``."""
    nb, _, bs, _ = k_layer.shape
    max_blocks = int(block_tables.shape[1])
    skipped = []
    for b in range(key_states.shape[0]):
        for t in range(key_states.shape[2]):
            pos = int(start_pos[b]) + t
            lb = pos // bs
            phys = int(block_tables[b, lb]) if 0 <= pos and lb < max_blocks else -1
            if phys < 0 or phys >= nb:
                skipped.append((b, t))
                continue
            k_layer[phys, :, pos % bs, :] = key_states[b, :, t, :].to(k_layer.dtype)
            v_layer[phys, :, pos % bs, :] = value_states[b, :, t, :].to(v_layer.dtype)
    return skipped


def rope_angles(positions, head_dim: int, theta: float) -> torch.Tensor:
    """``[len(positions), D/2]`` angles ``pos * theta ** -(2i / D)``, rounded to fp32 as
    transformers' default rotary embedding forms them (fp32 ``inv_freq`` times fp32
    positions), returned as float64."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim))
    ang = torch.as_tensor(positions).to(torch.float32).reshape(-1, 1) * inv.reshape(1, -1)
    return ang.to(torch.float64)


def rope_rotate_half(x: torch.Tensor, positions, theta: float) -> torch.Tensor:
    """Rotate ``x [B, H, D]`` at ``positions [B]``: ``x * cos + rotate_half(x) * sin`` (float64)."""
    d = x.shape[-1]
    ang = rope_angles(positions, d, theta)
    cos = torch.cat((ang.cos(), ang.cos()), dim=-1).unsqueeze(1)
    sin = torch.cat((ang.sin(), ang.sin()), dim=-1).unsqueeze(1)
    xd = x.to(torch.float64)
    rot = torch.cat((-xd[..., d // 2:], xd[..., : d // 2]), dim=-1)
    return xd * cos + rot * sin


def _f16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float16).to(torch.float32)


def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None
                ) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns ``(out, h)`` as fp16-valued fp32 tensors: ``h = fp16(x + residual)``,
    ``out = fp16(fp16(h * rsqrt(mean(h^2) + eps)) * weight)``."""
    h = x.float() if residual is None else _f16(x.float() + residual.float())
    r = torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return _f16(_f16(h * r) * weight.float()), h


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """``fp16(fp16(silu(g)) * u)`` for ``gate_up = [g | u]`` (fp16-valued fp32 result)."""
    i = gate_up.shape[-1] // 2
    g = gate_up[..., :i].float()
    u = gate_up[..., i:].float()
    return _f16(_f16(g / (1.0 + torch.exp(-g))) * u)
