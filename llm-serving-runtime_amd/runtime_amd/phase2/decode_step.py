"""One batched decode step of an int8 (W8A16) decoder over the paged KV pool.

This is the path ``TransformersBackend._paged_decode_step`` drives through an HF
model (``runtime/phase2/worker_server.py:733-794``), without the HF module
tree: per decoder layer the fused q/k/v, o, gate/up and down projections (the
quantized-linear slot, ``:194-205``), the K/V write of the new token into its
block (``paged_kv_cache.py:121-170`` -> ``paged_kv_kernel.py:176-227``) and
paged decode attention (``block_paged_attention.py:37-48``), then greedy
argmax (``worker_server.py:786``). Every op is a libmxdecode kernel on the
current stream:

    x = RMSNorm(h)                         mx_add_rmsnorm (fused with the residual add
                                           of the previous layer's MLP)
    qkv = x Wqkv^T (+b)                    mx_w8a16_qkv_rope_append (one launch for
    q, K/V slot <- RoPE(qkv), v            both lines at batch <= 32; else
                                           mx_w8a16_linear + mx_qkv_rope_append)
    a = paged_attention(q, pool)           mx_paged_attn_decode
    h += a Wo^T;  x = RMSNorm(h)           mx_w8a16_linear, mx_add_rmsnorm
    a = silu(x Wg^T) * (x Wu^T)            mx_w8a16_gateup_swiglu (gate and up rows
                                           interleaved by 8, product in the epilogue;
                                           K is never split, the VALU GEMV takes <= 4 rows)
    h += a Wdown^T                         mx_w8a16_linear (+ the next add_rmsnorm)
    logits = RMSNorm(h) Wlm^T; argmax      mx_add_rmsnorm, mx_w8a16_linear, mx_argmax_rows_split

The first norm gathers the embedding rows of the step's tokens itself, layer
0's RoPE kernel writes the attention lengths (positions + 1) and the argmax
kernel advances ``seq_lens``, so no torch kernel runs inside a step.

A projection whose shape splits K (``mx_w8a16_splits`` > 1: qkv, o and down at
batch 32) writes fp32 split partials instead (``mx_w8a16_linear_partials``)
and the kernel that consumes it (``mx_qkv_rope_append_splits`` /
``mx_add_rmsnorm_splits``) sums them, adds the bias and rounds to fp16 at the
point the linear would have, so no reduce launch sits between the two.

Activations live in per-batch-size buffers allocated on the first step, so a
whole step can be captured in one HIP graph and replayed. Architecture is
Llama / Qwen2 style (pre-norm, rotate-half RoPE, GQA, SwiGLU, untied int8
lm_head); :meth:`Int8DecodeModel.from_hf` loads the weights of an HF
``LlamaForCausalLM`` / ``Qwen2ForCausalLM``. The gate||up weight is stored
with gate and up rows interleaved in groups of 8 (``gateup_interleave``), and
one ``mx_w8a16_gateup_swiglu`` launch per 128 rows writes ``silu(g) * u``
whatever the batch: it never splits K (on shapes whose plain projection would,
such as Qwen2-0.5B at batch 16, it runs unsplit), and at most 4 rows run on
the VALU GEMV with the product in its own epilogue.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .decode_glue import (QKV_ROPE_MAX_ROWS, add_rmsnorm, add_rmsnorm_splits, argmax_rows, qkv_linear_rope_append,
                          qkv_rope_append, qkv_rope_append_splits, rope_table)
from .int8_linear import (MLP_SYNC_ERR, MLP_SYNC_WORDS, gateup_interleave, int8_gateup_swiglu, int8_linear,
                          int8_linear_partials, int8_mlp_fused_partials, linear_splits, mlp_fusable,
                          pack_weight, quantize_weight)
from .paged_attention_hip import MX_PA_PLAN_READ, MX_PA_PLAN_WRITE
from .paged_attention_hip import _decode as _paged_decode
from .roofline import linear_hbm_bytes


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


@dataclass
class _Buffers:
    h: torch.Tensor       # residual stream [B, hidden]
    x: torch.Tensor       # normalised input of the next projection [B, hidden]
    qkv: torch.Tensor     # [B, qkv_out]
    q: torch.Tensor       # rotated queries [B, heads * head_dim]
    attn: torch.Tensor    # attention output [B, heads, 1, head_dim]
    o: torch.Tensor       # [B, hidden]
    act: torch.Tensor     # [B, intermediate], silu(gate) * up
    mlp: torch.Tensor     # [B, hidden]
    logits: torch.Tensor  # [B, vocab]
    part: torch.Tensor    # fp32 split partials of the current split projection (qkv, o, down)
    splits: dict          # projection name -> K splits of its plain launch at this batch size
    attn_lens: torch.Tensor  # int32 [B]
    next: torch.Tensor    # int64 [B], greedy tokens
    err: torch.Tensor     # int32 [1], OR of the append kernels' error bits
    mlp_sync: torch.Tensor  # int32 [MLP_SYNC_WORDS], the fused MLP launch's counters and error word
    mlp_fused: bool       # gate||up and down run as one launch at this batch size


def _quantize(w: torch.Tensor, device: torch.device) -> tuple:
    q, s = quantize_weight(w.to(device=device, dtype=torch.float32))
    return pack_weight(q), s, int(w.shape[0])


def _random_quantized(n: int, k: int, gen: torch.Generator, device: torch.device, std: float) -> tuple:
    w = torch.randn(n, k, generator=gen, device=device, dtype=torch.float32) * std
    out = _quantize(w, device)
    del w
    return out


class Int8DecodeModel:
    """int8 decoder for the native decode step: random init or weights loaded from HF."""

    def __init__(self, shape: DecoderShape, device: torch.device | str = "cuda", seed: int = 0, std: float = 0.02,
                 layers: int | None = None, max_positions: int = 32768, init: bool = True) -> None:
        self.shape = shape
        self.device = torch.device(device)
        self.n_layers = layers if layers is not None else shape.layers
        self.rope = rope_table(max_positions, shape.head_dim, shape.rope_theta, self.device)
        # QKV projection + RoPE + append as one launch where it applies (uses_fused_qkv);
        # False keeps the two-launch path (split partials or fp16 rows, then the RoPE kernel).
        self.fuse_qkv_rope = True
        # Set when block tables may alias block ids across rows (a shared prefix): the
        # attention kernel then keeps the default cache policy for K/V.
        self.shared_kv_blocks = False
        # Attention at layer 0 records each wave's tiles (MX_PA_PLAN_WRITE) and the later layers,
        # whose lengths and block tables are the same, start from that record (MX_PA_PLAN_READ):
        # one dependent memory round trip less per layer. Needs block size >= 16 and no aliasing.
        self.attn_plan = True
        # True: gate||up and down as one launch where the shape and device take it (mlp_fusable:
        # the Llama-3-8B MLP at batch 32), bit-identical to the two launches. Off: measured on
        # MI355X at batch 32 it took 48-50 us per layer against 39.6-41.3 us for the two launches
        # (bench.py --fuse-mlp); down cannot start before gate||up's slowest workgroups finish.
        self.fuse_mlp = False
        self._buffers: dict[int, _Buffers] = {}
        self.layers: list[_Layer] = []
        if not init:
            return
        gen = torch.Generator(device=self.device).manual_seed(seed)
        s = shape
        self.embed = (torch.randn(s.vocab, s.hidden, generator=gen, device=self.device) * std).to(torch.float16)
        for _ in range(self.n_layers):
            qkv = _random_quantized(s.qkv_out, s.hidden, gen, self.device, std)
            bias = (torch.randn(s.qkv_out, generator=gen, device=self.device) * std).to(torch.float16) \
                if s.qkv_bias else None
            self.layers.append(_Layer(
                ln_in=torch.ones(s.hidden, dtype=torch.float16, device=self.device),
                ln_post=torch.ones(s.hidden, dtype=torch.float16, device=self.device),
                qkv=(*qkv, bias),
                o=(*_random_quantized(s.hidden, s.heads * s.head_dim, gen, self.device, std), None),
                gate_up=(*_random_quantized(2 * s.intermediate, s.hidden, gen, self.device, std), None),
                down=(*_random_quantized(s.hidden, s.intermediate, gen, self.device, std), None),
            ))
        self.ln_final = torch.ones(s.hidden, dtype=torch.float16, device=self.device)
        self.lm_head = (*_random_quantized(s.vocab, s.hidden, gen, self.device, std), None)

    @classmethod
    def from_hf(cls, model, device: torch.device | str = "cuda", max_positions: int = 32768) -> "Int8DecodeModel":
        """Quantize an HF ``LlamaForCausalLM`` / ``Qwen2ForCausalLM`` (fp32 weights) into this layout.

        q/k/v are stacked into one projection (rows q, then k, then v) and
        gate/up into one with rows interleaved by 8 (``gateup_interleave``).
        Per-output-channel quantization is row-wise, so each stacked weight
        quantizes exactly as its parts would.
        Norms, biases and the embedding are stored in fp16; lm_head is int8.
        """
        cfg = model.config
        heads = int(cfg.num_attention_heads)
        head_dim = int(getattr(cfg, "head_dim", None) or cfg.hidden_size // heads)
        rope = getattr(cfg, "rope_parameters", None) or {}
        theta = float(rope.get("rope_theta", getattr(cfg, "rope_theta", 10000.0)))
        # The (cos, sin) table is transformers' default rotary embedding; a scaled variant
        # (llama3, yarn, linear, dynamic, ...) would load and decode with wrong phases.
        scaling = getattr(cfg, "rope_scaling", None) or {}
        for spec in (rope, scaling):
            kind = spec.get("rope_type", spec.get("type", "default")) if isinstance(spec, dict) else "default"
            if kind not in (None, "default"):
                raise ValueError(f"from_hf supports the default rotary embedding only, got rope_type={kind!r}")
        attn0 = model.model.layers[0].self_attn
        shape = DecoderShape(hidden=int(cfg.hidden_size), layers=int(cfg.num_hidden_layers), heads=heads,
                             kv_heads=int(cfg.num_key_value_heads), head_dim=head_dim,
                             intermediate=int(cfg.intermediate_size), vocab=int(cfg.vocab_size), rope_theta=theta,
                             rms_eps=float(cfg.rms_norm_eps), qkv_bias=attn0.q_proj.bias is not None)
        self = cls(shape, device=device, max_positions=max_positions, init=False)
        dev = self.device

        def f16(t):
            return t.detach().to(device=dev, dtype=torch.float16).contiguous()

        with torch.no_grad():
            self.embed = f16(model.model.embed_tokens.weight)
            for layer in model.model.layers:
                at, mlp = layer.self_attn, layer.mlp
                qkv_w = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight], dim=0)
                bias = None
                if at.q_proj.bias is not None:
                    bias = f16(torch.cat([at.q_proj.bias, at.k_proj.bias, at.v_proj.bias]))
                self.layers.append(_Layer(
                    ln_in=f16(layer.input_layernorm.weight),
                    ln_post=f16(layer.post_attention_layernorm.weight),
                    qkv=(*_quantize(qkv_w, dev), bias),
                    o=(*_quantize(at.o_proj.weight, dev), None),
                    gate_up=(*_quantize(gateup_interleave(mlp.gate_proj.weight, mlp.up_proj.weight), dev), None),
                    down=(*_quantize(mlp.down_proj.weight, dev), None),
                ))
            self.ln_final = f16(model.model.norm.weight)
            self.lm_head = (*_quantize(model.lm_head.weight, dev), None)
        return self

    # --- byte accounting (algorithmic HBM bytes of one step) -------------------
    def linear_bytes(self, batch: int) -> dict[str, int]:
        s = self.shape
        return {
            "qkv": linear_hbm_bytes(batch, s.qkv_out, s.hidden, s.qkv_bias),
            "o": linear_hbm_bytes(batch, s.hidden, s.heads * s.head_dim),
            # gate||up writes silu(g) * u only
            "gate_up": linear_hbm_bytes(batch, 2 * s.intermediate, s.hidden, out_cols=s.intermediate),
            "down": linear_hbm_bytes(batch, s.hidden, s.intermediate),
            "lm_head": linear_hbm_bytes(batch, s.vocab, s.hidden),
        }

    def buffers(self, batch: int) -> _Buffers:
        buf = self._buffers.get(batch)
        if buf is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("decode buffers must be allocated before graph capture; run one eager step")
            s, dev, f16 = self.shape, self.device, torch.float16

            def e(*shape):
                return torch.empty(*shape, dtype=f16, device=dev)

            shapes = {"qkv": (s.qkv_out, s.hidden), "o": (s.hidden, s.heads * s.head_dim),
                      "gate_up": (2 * s.intermediate, s.hidden), "down": (s.hidden, s.intermediate),
                      "lm_head": (s.vocab, s.hidden)}
            splits = {k: linear_splits(batch, n, kk) for k, (n, kk) in shapes.items()}
            # gate||up runs unsplit with its SwiGLU epilogue and lm_head writes fp16 logits: only
            # qkv (where not fused with RoPE), o and down write split partials.
            part_elems = max([splits[k] * batch * shapes[k][0] for k in ("qkv", "o", "down") if splits[k] > 1]
                             + [4])
            buf = _Buffers(h=e(batch, s.hidden), x=e(batch, s.hidden), qkv=e(batch, s.qkv_out),
                           q=e(batch, s.heads * s.head_dim), attn=e(batch, s.heads, 1, s.head_dim),
                           o=e(batch, s.hidden), act=e(batch, s.intermediate),
                           mlp=e(batch, s.hidden), logits=e(batch, s.vocab),
                           part=torch.empty(part_elems, dtype=torch.float32, device=dev), splits=splits,
                           attn_lens=torch.zeros(batch, dtype=torch.int32, device=dev),
                           next=torch.zeros(batch, dtype=torch.int64, device=dev),
                           err=torch.zeros(1, dtype=torch.int32, device=dev),
                           mlp_sync=torch.zeros(MLP_SYNC_WORDS, dtype=torch.int32, device=dev),
                           mlp_fused=mlp_fusable(batch, s.hidden, s.intermediate, s.hidden))
            self._buffers[batch] = buf
        return buf

    def error_flag(self) -> int:
        """OR of the KV-append error bits since the buffers were created (one host sync each), with
        bit 16 set if a fused MLP launch gave up waiting for its activations."""
        flag = 0
        for buf in self._buffers.values():
            flag |= int(buf.err.item())
            if int(buf.mlp_sync[MLP_SYNC_ERR].item()):
                flag |= 16
        return flag

    def step(self, tokens: torch.Tensor, pool, block_tables: torch.Tensor, seq_lens: torch.Tensor,
             timers: dict | None = None, return_logits: bool = False, out: torch.Tensor | None = None):
        """Decode one token per row. ``tokens`` (int64) are this step's inputs; ``seq_lens``
        (int32) holds the KV length BEFORE this token (= the token's position) and is advanced in
        place. Returns the greedy next tokens ``[B]`` (int64, on device; written to ``out`` if
        given, which may be ``tokens`` itself), and the fp16 logits ``[B, vocab]`` with
        ``return_logits``."""
        s = self.shape
        bsz = int(tokens.shape[0])
        buf = self.buffers(bsz)
        if seq_lens.dtype != torch.int32 or block_tables.dtype != torch.int32 or tokens.dtype != torch.int64:
            raise ValueError("seq_lens and block_tables must be int32 and tokens int64 device tensors")
        eps = s.rms_eps
        plan = self.attn_plan and not self.shared_kv_blocks and pool.block_size_tokens >= 16
        sp = buf.splits
        for li, layer in enumerate(self.layers):
            if li == 0:  # h = embed[tokens]; x = RMSNorm(h)
                add_rmsnorm(self.embed, layer.ln_in, eps, out=buf.x, residual_out=buf.h, rows=tokens)
            else:
                self._norm_after_down(buf, layer.ln_in)
            lens_out = buf.attn_lens if li == 0 else None
            k_layer = pool.k_layer_view(li)
            v_layer = pool.v_layer_view(li)
            used = pool._used_map  # the pool's block-usage accounting, marked by the K/V append
            if self.uses_fused_qkv(bsz):
                ev = self._tick(timers, "qkv")
                packed, scale, _, bias = layer.qkv
                qkv_linear_rope_append(buf.x, packed, scale, bias, self.rope, seq_lens, buf.q, k_layer, v_layer,
                                       block_tables, s.heads, s.kv_heads, err=buf.err, lens_out=lens_out,
                                       used_blocks=used)
                self._tock(timers, "qkv", ev)
            elif sp["qkv"] > 1:
                self._partials(buf.x, layer.qkv, buf.part, timers, "qkv")
                qkv_rope_append_splits(buf.part, sp["qkv"], layer.qkv[3], self.rope, seq_lens, buf.q, k_layer,
                                       v_layer, block_tables, s.heads, s.kv_heads, err=buf.err, lens_out=lens_out,
                                       used_blocks=used)
            else:
                self._lin(buf.x, layer.qkv, buf.qkv, timers, "qkv")
                qkv_rope_append(buf.qkv, self.rope, seq_lens, buf.q, k_layer, v_layer, block_tables, s.heads,
                                s.kv_heads, err=buf.err, lens_out=lens_out, used_blocks=used)
            ev = self._tick(timers, "attn")
            _paged_decode(buf.q.view(bsz, s.heads, 1, s.head_dim), k_layer, v_layer, block_tables, buf.attn_lens,
                          s.head_dim ** -0.5, s.group, out=buf.attn, shared_blocks=self.shared_kv_blocks,
                          plan=(MX_PA_PLAN_WRITE if li == 0 else MX_PA_PLAN_READ) if plan else 0)
            self._tock(timers, "attn", ev)
            if sp["o"] > 1:
                self._partials(buf.attn.view(bsz, -1), layer.o, buf.part, timers, "o")
                add_rmsnorm_splits(buf.part, sp["o"], layer.o[3], layer.ln_post, eps, buf.x, residual=buf.h,
                                   residual_out=buf.h)
            else:
                self._lin(buf.attn.view(bsz, -1), layer.o, buf.o, timers, "o")
                add_rmsnorm(buf.o, layer.ln_post, eps, residual=buf.h, out=buf.x, residual_out=buf.h)
            if self.fuse_mlp and buf.mlp_fused:
                ev = self._tick(timers, "mlp")
                int8_mlp_fused_partials(buf.x, layer.gate_up, layer.down, buf.act, buf.part, buf.mlp_sync)
                self._tock(timers, "mlp", ev)
            else:
                self._gate_up(buf, layer.gate_up, bsz, timers)
                if sp["down"] > 1:
                    self._partials(buf.act, layer.down, buf.part, timers, "down")
                else:
                    self._lin(buf.act, layer.down, buf.mlp, timers, "down")
        self._norm_after_down(buf, self.ln_final)
        self._lin(buf.x, self.lm_head, buf.logits, timers, "lm_head")
        nxt = argmax_rows(buf.logits, out=buf.next if out is None else out, seq_lens=seq_lens)
        return (nxt, buf.logits) if return_logits else nxt

    def uses_fused_qkv(self, bsz: int) -> bool:
        """Whether the step's QKV projection and RoPE + append run as one launch at this batch."""
        return self.fuse_qkv_rope and bsz <= QKV_ROPE_MAX_ROWS and self.shape.head_dim in (64, 128)

    def _norm_after_down(self, buf: _Buffers, weight: torch.Tensor) -> None:
        """x = RMSNorm(h + down output) * weight; h updated in place."""
        eps = self.shape.rms_eps
        if buf.splits["down"] > 1:
            add_rmsnorm_splits(buf.part, buf.splits["down"], None, weight, eps, buf.x, residual=buf.h,
                               residual_out=buf.h)
        else:
            add_rmsnorm(buf.mlp, weight, eps, residual=buf.h, out=buf.x, residual_out=buf.h)

    def _gate_up(self, buf: _Buffers, w, bsz: int, timers) -> None:
        """act = silu(gate) * up from the interleaved gate||up weight, one launch per 128 rows."""
        packed, scale, n, bias = w
        ev = self._tick(timers, "gate_up")
        int8_gateup_swiglu(buf.x, packed, scale, bias, n // 2, out=buf.act)
        self._tock(timers, "gate_up", ev)

    def _partials(self, x, w, part, timers, name):
        packed, scale, n, _ = w
        ev = self._tick(timers, name)
        int8_linear_partials(x, packed, scale, n, part)
        self._tock(timers, name, ev)

    def _lin(self, x, w, out, timers, name):
        packed, scale, n, bias = w
        ev = self._tick(timers, name)
        int8_linear(x, packed, scale, bias, n, out=out)
        self._tock(timers, name, ev)

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
