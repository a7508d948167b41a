"""Pins of the glue oracle against transformers' own modules and closed forms (CPU)."""

from __future__ import annotations

import math

import torch

from oracle import glue as og
from oracle import kv_pool as okv


def test_append_tokens_matches_pool_oracle_and_flags_out_of_range():
    g = torch.Generator().manual_seed(0)
    nb, hkv, bs, d = 12, 2, 4, 8
    k_a = torch.zeros(nb, hkv, bs, d)
    v_a = torch.zeros_like(k_a)
    tables = torch.tensor([[3, 7, 1], [5, 0, 9]], dtype=torch.int32)
    start = [2, 4]
    ks = torch.randn(2, hkv, 5, d, generator=g)
    vs = torch.randn(2, hkv, 5, d, generator=g)
    skipped = og.append_tokens(k_a, v_a, tables, start, ks, vs)
    assert skipped == []
    for b, (row, n) in enumerate((([3, 7, 1], 7), ([5, 0, 9], 9))):
        k, v = okv.gather_layer_view(k_a, v_a, row, n)
        torch.testing.assert_close(k[0, :, start[b]:], ks[b], atol=0, rtol=0)
        torch.testing.assert_close(v[0, :, start[b]:], vs[b], atol=0, rtol=0)
    # Past the table (row 1 position 12 -> logical block 3) and a bad physical id.
    skipped = og.append_tokens(k_a, v_a, torch.tensor([[3, 7, 1], [5, 99, 0]], dtype=torch.int32), [10, 3], ks, vs)
    assert (0, 2) in skipped and (1, 1) in skipped and (0, 1) not in skipped


def test_rope_matches_transformers_rotary_embedding():
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding, apply_rotary_pos_emb

    cfg = Qwen2Config(hidden_size=256, num_attention_heads=4, num_key_value_heads=2, rope_theta=1e6)
    rot = Qwen2RotaryEmbedding(cfg)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 4, 64, generator=g)
    pos = torch.tensor([0, 5, 4000])
    cos, sin = rot(x, pos.view(3, 1))  # [3, 1, 64]
    q, _ = apply_rotary_pos_emb(x.unsqueeze(2), x.unsqueeze(2), cos, sin, unsqueeze_dim=1)
    ours = og.rope_rotate_half(x, pos, 1e6)
    torch.testing.assert_close(ours.float(), q.squeeze(2), atol=2e-6, rtol=1e-6)


def test_rope_closed_forms():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 3, 16, generator=g, dtype=torch.float64)
    torch.testing.assert_close(og.rope_rotate_half(x, [0, 0], 1e4), x, atol=0, rtol=0)
    y = og.rope_rotate_half(x, [7, 123], 1e4)
    pair = lambda t: t[..., :8] ** 2 + t[..., 8:] ** 2  # noqa: E731
    torch.testing.assert_close(pair(y), pair(x), atol=1e-12, rtol=1e-12)
    z = og.rope_rotate_half(og.rope_rotate_half(x, [3, 40], 1e4).to(torch.float64), [4, 60], 1e4)
    # Angle additivity, up to the fp32 rounding of the angles.
    torch.testing.assert_close(z, og.rope_rotate_half(x, [7, 100], 1e4), atol=1e-4, rtol=0)
    # A planted sign slip in rotate_half breaks norm preservation.
    ang = og.rope_angles([7], 16, 1e4)
    bad = x[0] * torch.cat((ang.cos(), ang.cos()), -1) + torch.cat((x[0, :, 8:], x[0, :, :8]), -1) * torch.cat(
        (ang.sin(), ang.sin()), -1)
    assert (pair(bad) - pair(x[0])).abs().max() > 1e-3


def test_add_rmsnorm_matches_transformers_module():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 96, generator=g).half()
    res = torch.randn(4, 96, generator=g).half()
    w = (1 + 0.1 * torch.randn(96, generator=g)).half()
    norm = Qwen2RMSNorm(96, eps=1e-6)
    norm.weight.data = w.clone()
    h16 = (x.float() + res.float()).half()  # fp16 residual add as an fp16 model does it
    ref = norm(h16)  # HF: fp32 normalise, cast to fp16, * fp16 weight
    out, h = og.add_rmsnorm(x, w, 1e-6, residual=res)
    torch.testing.assert_close(h, h16.float(), atol=0, rtol=0)
    torch.testing.assert_close(out, ref.float(), atol=0, rtol=0)
    # Closed form: a constant row normalises to sign * weight.
    c = torch.full((1, 96), -3.0)
    out_c, _ = og.add_rmsnorm(c, w, 0.0)
    torch.testing.assert_close(out_c[0], (-w.float()).half().float(), atol=0, rtol=0)


def test_silu_mul_matches_transformers_mlp_product():
    g = torch.Generator().manual_seed(4)
    gu = torch.randn(3, 64, generator=g).half()
    gate, up = gu[:, :32], gu[:, 32:]
    ref = torch.nn.functional.silu(gate.float()).half().float() * up.float()
    torch.testing.assert_close(og.silu_mul(gu), ref.half().float(), atol=0, rtol=0)
    zero = og.silu_mul(torch.cat((torch.zeros(1, 4), torch.ones(1, 4)), -1))
    assert float(zero.abs().max()) == 0.0
    big = og.silu_mul(torch.tensor([[20.0, 2.0]]))
    assert math.isclose(float(big[0, 0]), 40.0, rel_tol=1e-3)
