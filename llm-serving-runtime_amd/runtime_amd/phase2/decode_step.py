"""One batched decode step of an int8 (W8A16) decoder over the paged KV pool.

This is the path ``TransformersBackend._paged_decode_step`` drives through an HF
model (``runtime/phase2/worker_server.py:733-794``): per decoder layer the
q/k/v, o, gate/up and down projections (the quantized-linear slot,
``:194-205``), the K/V write of the new token into its block
(``paged_kv_cache.py:121-170`` -> ``paged_kv_kernel.py:176-227``) and paged
decode attention (``block_paged_attention.py:37-48``), then greedy argmax
(``worker_server.py:786``). Projections and attention run on the HIP kernels
of libmxdecode; normalisation, rotary embedding, the KV write and SwiGLU are
torch glue on the same stream. Every tensor the step touches is allocated
before the first step, so a whole step can be captured in one HIP graph.

Architecture is Llama / Qwen2 style: RMSNorm, fused QKV (optional bias, as in
Qwen2), RoPE, GQA, fused gate||up with SiLU, untied int8 lm_head.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .int8_linear import int8_linear, pack_weight, quantize_weight
from .paged_attention_hip import _decode as _paged_decode


@dataclass(frozen=True)
class DecoderShape:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5
    qkv_bias: bool = False

    @property
    def qkv_out(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    @property
    def group(self) -> int:
        return self.heads // self.kv_heads


LLAMA3_8B = DecoderShape(hidden=4096, layers=32, heads=32, kv_heads=8, head_dim=128, intermediate=14336, vocab=128256,
                         rope_theta=500000.0, rms_eps=1e-5)
QWEN2_05B = DecoderShape(hidden=896, layers=24, heads=14, kv_heads=2, head_dim=64, intermediate=4864, vocab=151936,
                         rope_theta=1000000.0, rms_eps=1e-6, qkv_bias=True)


@dataclass
class _Layer:
    ln_in: torch.Tensor
    ln_post: torch.Tensor
    qkv: tuple
    o: tuple
    gate_up: tuple
    down: tuple


def _quantized(n: int, k: int, gen: torch.Generator, device: torch.device, std: float) -> tuple:
    w = torch.randn(n, k, generator=gen, device=device, dtype=torch.float32) * std
    q, s = quantize_weight(w)
    del w
    return pack_weight(q), s, n


class Int8DecodeModel:
    """Random-init int8 decoder (weights quantized with the build's format on the device)."""

    def __init__(self, shape: DecoderShape, device: torch.device | str = "cuda", seed: int = 0, std: float = 0.02,
                 layers: int | None = None) -> None:
        self.shape = shape
        self.device = torch.device(device)
        self.n_layers = layers if layers is not None else shape.layers
        gen = torch.Generator(device=self.device).manual_seed(seed)
        s = shape
        self.embed = (torch.randn(s.vocab, s.hidden, generator=gen, device=self.device) * std).to(torch.float16)
        self.layers: list[_Layer] = []
        for _ in range(self.n_layers):
            qkv = _quantized(s.qkv_out, s.hidden, gen, self.device, std)
            if s.qkv_bias:
                qkv = (*qkv, (torch.randn(s.qkv_out, generator=gen, device=self.device) * std).to(torch.float16))
            else:
                qkv = (*qkv, None)
            self.layers.append(_Layer(
                ln_in=torch.ones(s.hidden, dtype=torch.float16, device=self.device),
                ln_post=torch.ones(s.hidden, dtype=torch.float16, device=self.device),
                qkv=qkv,
                o=(*_quantized(s.hidden, s.heads * s.head_dim, gen, self.device, std), None),
                gate_up=(*_quantized(2 * s.intermediate, s.hidden, gen, self.device, std), None),
                down=(*_quantized(s.hidden, s.intermediate, gen, self.device, std), None),
            ))
        self.ln_final = torch.ones(s.hidden, dtype=torch.float16, device=self.device)
        self.lm_head = (*_quantized(s.vocab, s.hidden, gen, self.device, std), None)
        half = s.head_dim // 2
        self.inv_freq = 1.0 / (s.rope_theta ** (torch.arange(0, half, device=self.device, dtype=torch.float32) / half))

    # --- byte accounting (algorithmic HBM bytes of one step) -------------------
    def linear_bytes(self, batch: int) -> dict[str, int]:
        s = self.shape

        def lb(n, k, bias=False):
            return n * k + 2 * n + 2 * batch * k + 2 * batch * n + (2 * n if bias else 0)

        return {
            "qkv": lb(s.qkv_out, s.hidden, s.qkv_bias),
            "o": lb(s.hidden, s.heads * s.head_dim),
            "gate_up": lb(2 * s.intermediate, s.hidden),
            "down": lb(s.hidden, s.intermediate),
            "lm_head": lb(s.vocab, s.hidden),
        }

    # --- glue -------------------------------------------------------------------
    def _rms(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.shape.rms_eps)
        return w * xf.to(torch.float16)

    def _rope(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        # x [B, H, D], pos [B] int -> rotate-half RoPE (HF Llama/Qwen2 convention).
        freqs = pos.float().unsqueeze(-1) * self.inv_freq.unsqueeze(0)  # [B, D/2]
        emb = torch.cat((freqs, freqs), dim=-1)
        cos = emb.cos().to(x.dtype).unsqueeze(1)
        sin = emb.sin().to(x.dtype).unsqueeze(1)
        half = x.shape[-1] // 2
        rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
        return x * cos + rot * sin

    def step(self, tokens: torch.Tensor, pool, block_tables: torch.Tensor, seq_lens: torch.Tensor,
             timers: dict | None = None) -> torch.Tensor:
        """Decode one token per row. ``seq_lens`` holds the KV length BEFORE this token and is
        advanced in place. Returns the greedy next tokens ``[B]`` (int64, on device)."""
        s = self.shape
        bsz = int(tokens.shape[0])
        bs = pool.block_size_tokens
        pos = seq_lens.to(torch.int64)
        rows = torch.arange(bsz, device=self.device)
        phys = block_tables.to(torch.int64)[rows, torch.div(pos, bs, rounding_mode="floor")]
        off = pos % bs
        attn_lens = (seq_lens + 1).to(torch.int32)
        h = self.embed.index_select(0, tokens)
        nq, nkv = s.heads * s.head_dim, s.kv_heads * s.head_dim
        for li, layer in enumerate(self.layers):
            x = self._rms(h, layer.ln_in)
            qkv = self._lin(x, layer.qkv, timers, "qkv")
            q = self._rope(qkv[:, :nq].view(bsz, s.heads, s.head_dim), pos)
            k = self._rope(qkv[:, nq:nq + nkv].view(bsz, s.kv_heads, s.head_dim), pos)
            v = qkv[:, nq + nkv:].view(bsz, s.kv_heads, s.head_dim)
            k_layer = pool.k_layer_view(li)
            v_layer = pool.v_layer_view(li)
            k_layer[phys, :, off, :] = k
            v_layer[phys, :, off, :] = v
            ev = self._tick(timers, "attn")
            attn = _paged_decode(q.unsqueeze(2), k_layer, v_layer, block_tables, attn_lens, s.head_dim**-0.5,
                                 s.group)
            self._tock(timers, "attn", ev)
            h = h + self._lin(attn.view(bsz, nq), layer.o, timers, "o")
            x = self._rms(h, layer.ln_post)
            gu = self._lin(x, layer.gate_up, timers, "gate_up")
            a = torch.nn.functional.silu(gu[:, :s.intermediate]) * gu[:, s.intermediate:]
            h = h + self._lin(a, layer.down, timers, "down")
        x = self._rms(h, self.ln_final)
        logits = self._lin(x, self.lm_head, timers, "lm_head")
        seq_lens.add_(1)
        return logits.argmax(dim=-1)

    def _lin(self, x, w, timers, name):
        packed, scale, n, bias = w
        ev = self._tick(timers, name)
        y = int8_linear(x, packed, scale, bias, n)
        self._tock(timers, name, ev)
        return y

    @staticmethod
    def _tick(timers, name):
        if timers is None:
            return None
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return e

    @staticmethod
    def _tock(timers, name, start):
        if timers is None:
            return
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        timers.setdefault(name, []).append((start, e))


def make_contexts(batch: int, lo: int, hi: int, block_size: int, pool_blocks: int, headroom: int, seed: int = 0
                  ) -> tuple[torch.Tensor, torch.Tensor]:
    """Seeded context lengths ~ U[lo, hi] and disjoint block tables from one randperm(pool_blocks).

    Each row gets ``ceil((len + headroom) / block_size)`` blocks so ``headroom``
    decode steps fit without reallocation.
    """
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g)
    perm = torch.randperm(pool_blocks, generator=g)
    need = [math.ceil((int(x) + headroom) / block_size) for x in lens]
    if sum(need) > pool_blocks:
        raise ValueError("pool too small for the requested contexts")
    tables = torch.zeros(batch, max(need), dtype=torch.int32)
    used = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    return lens.to(torch.int32), tables
