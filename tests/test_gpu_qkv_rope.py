"""Fused QKV projection + RoPE + KV append (``mx_w8a16_qkv_rope_append``).

* Where the two-launch path splits the QKV projection 8 ways (Llama-3-8B dims, 5..32 rows),
  the fused launch is bit for bit the two-launch path (``mx_w8a16_linear_partials`` then
  ``mx_qkv_rope_append_splits``): q, every byte of the K/V layers, the error word and the
  lengths. Its 8 waves accumulate the same k ranges with the same MFMA sequence, and the
  epilogue sums and rounds as the split consumer does.
* Elsewhere (Qwen2-0.5B dims with bias, GEMV-sized batches) the projection sums in another
  order, so the bar is the fp16 one of the two-launch path: atol/rtol 1e-2 against the fp32
  oracle (int8 linear, then rotate-half RoPE in float64); v within 1 fp16 ulp of the
  two-launch output, and q, k within 2 ulps of the projection's largest magnitude (a 1-ulp
  change of a rotated pair moves its outputs by at most sqrt(2) such ulps, plus the final
  rounding; a per-element ulp bar would fail where the rotation cancels to near zero).
* Positions outside the RoPE table and slots outside a row's table raise the same error bits
  and leave the same memory untouched; more than 32 rows are refused.
* The decode step with the fused launch gives the two-launch step's logits bit for bit at
  batch 32 on the Llama-3-8B dims.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import glue as og
from oracle import int8_quant

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _ulps(a: torch.Tensor, b: torch.Tensor) -> int:
    def key(t):
        i = t.to(torch.float16).view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return int((key(a.cpu()) - key(b.cpu())).abs().max())


def _setup(hq, hkv, d, hidden, m, with_bias, seed, max_pos=4096, nb=None, bs=16):
    from runtime_amd.phase2.decode_glue import rope_table
    from runtime_amd.phase2.int8_linear import pack_weight, quantize_weight

    g = torch.Generator(device=DEV).manual_seed(seed)
    n = (hq + 2 * hkv) * d
    q8, s8 = quantize_weight(torch.randn(n, hidden, generator=g, device=DEV) * 0.02)
    bias = (torch.randn(n, generator=g, device=DEV) * 0.1).half() if with_bias else None
    x = torch.randn(m, hidden, generator=g, device=DEV).half()
    rope = rope_table(max_pos, d, 5e5, DEV)
    gc = torch.Generator().manual_seed(seed)
    pos = torch.randint(0, 1000, (m,), generator=gc, dtype=torch.int32)
    per_row = 64
    nb = nb or m * per_row + 3
    tables = torch.randperm(nb, generator=gc)[:m * per_row].to(torch.int32).view(m, per_row)
    return dict(q8=q8, s8=s8, packed=pack_weight(q8), bias=bias, x=x, rope=rope, pos=pos.to(DEV),
                tables=tables.to(DEV), nb=nb, bs=bs, n=n)


def _pool_layer(nb, hkv, bs, d, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn(nb, hkv, bs, d, generator=g, device=DEV).half()
    v = torch.randn(nb, hkv, bs, d, generator=g, device=DEV).half()
    return k, v


def _fused(c, hq, hkv, d, k, v, lens=None, err=None):
    from runtime_amd.phase2.decode_glue import qkv_linear_rope_append

    q_out = torch.full((c["x"].shape[0], hq * d), 3.0, dtype=torch.float16, device=DEV)
    qkv_linear_rope_append(c["x"], c["packed"], c["s8"], c["bias"], c["rope"], c["pos"], q_out, k, v, c["tables"],
                           hq, hkv, err=err, lens_out=lens)
    return q_out


def _two_launch(c, hq, hkv, d, k, v, lens=None, err=None):
    from runtime_amd.phase2.decode_glue import qkv_rope_append, qkv_rope_append_splits
    from runtime_amd.phase2.int8_linear import int8_linear, int8_linear_partials, linear_splits

    m, hidden = c["x"].shape
    q_out = torch.full((m, hq * d), 3.0, dtype=torch.float16, device=DEV)
    splits = linear_splits(m, c["n"], hidden)
    if splits > 1 and m > 4:
        part = torch.empty(splits * m * c["n"], dtype=torch.float32, device=DEV)
        int8_linear_partials(c["x"], c["packed"], c["s8"], c["n"], part)
        qkv_rope_append_splits(part, splits, c["bias"], c["rope"], c["pos"], q_out, k, v, c["tables"], hq, hkv,
                               err=err, lens_out=lens)
    else:
        qkv = int8_linear(c["x"], c["packed"], c["s8"], c["bias"], c["n"])
        qkv_rope_append(qkv, c["rope"], c["pos"], q_out, k, v, c["tables"], hq, hkv, err=err, lens_out=lens)
    return q_out


@pytest.mark.parametrize("m", [5, 16, 32])
@pytest.mark.parametrize("with_bias", [False, True])
def test_fused_equals_split_path_bit_exact(m, with_bias):
    from runtime_amd.phase2.int8_linear import linear_splits

    hq, hkv, d, hidden = 32, 8, 128, 4096
    c = _setup(hq, hkv, d, hidden, m, with_bias, seed=10 + m)
    assert linear_splits(m, c["n"], hidden) == 8
    outs = []
    for fn in (_fused, _two_launch):
        k, v = _pool_layer(c["nb"], hkv, c["bs"], d, seed=4)
        lens = torch.full((m,), -1, dtype=torch.int32, device=DEV)
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        q = fn(c, hq, hkv, d, k, v, lens=lens, err=err)
        outs.append((q, k, v, lens, err))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert outs[0][3].cpu().tolist() == (c["pos"] + 1).cpu().tolist()
    assert int(outs[0][4].item()) == 0


@pytest.mark.parametrize("m", [1, 3, 16])
def test_fused_qwen_dims_with_bias_vs_oracle(m):
    hq, hkv, d, hidden = 14, 2, 64, 896
    c = _setup(hq, hkv, d, hidden, m, True, seed=20 + m)
    kf, vf = _pool_layer(c["nb"], hkv, c["bs"], d, seed=5)
    kt, vt = kf.clone(), vf.clone()
    before_k, before_v = kf.clone(), vf.clone()
    q_f = _fused(c, hq, hkv, d, kf, vf)
    q_t = _two_launch(c, hq, hkv, d, kt, vt)
    qkv = torch.from_numpy(int8_quant.linear_ref_fp32(c["x"].cpu().numpy(), c["q8"].cpu().numpy(),
                                                      c["s8"].cpu().numpy(), c["bias"].cpu().numpy()))
    ulp = 2.0 ** (float(np.floor(np.log2(float(qkv.abs().max())))) - 10)
    assert float((q_f.float() - q_t.float()).abs().max()) <= 2 * ulp
    assert float((kf.float() - kt.float()).abs().max()) <= 2 * ulp
    assert _ulps(vf, vt) <= 1
    pos = c["pos"].cpu()
    q_ref = og.rope_rotate_half(qkv[:, :hq * d].view(m, hq, d).double(), pos.tolist(), 5e5)
    torch.testing.assert_close(q_f.view(m, hq, d).float().cpu(), q_ref.float(), atol=1e-2, rtol=1e-2)
    k_ref = og.rope_rotate_half(qkv[:, hq * d:(hq + hkv) * d].view(m, hkv, d).double(), pos.tolist(), 5e5)
    v_ref = qkv[:, (hq + hkv) * d:].view(m, hkv, d)
    touched = torch.zeros(c["nb"], c["bs"], dtype=torch.bool)
    tables = c["tables"].cpu()
    for r in range(m):
        p = int(pos[r])
        phys = int(tables[r, p // c["bs"]])
        touched[phys, p % c["bs"]] = True
        torch.testing.assert_close(kf[phys, :, p % c["bs"]].float().cpu(), k_ref[r].float(), atol=1e-2, rtol=1e-2)
        torch.testing.assert_close(vf[phys, :, p % c["bs"]].float().cpu(), v_ref[r].float(), atol=1e-2, rtol=1e-2)
    mask = ~touched[:, None, :, None].expand(c["nb"], hkv, c["bs"], d).to(DEV)
    assert torch.equal(kf[mask], before_k[mask]) and torch.equal(vf[mask], before_v[mask])


def test_fused_positions_outside_tables_and_lengths():
    """Row 0's position is past the RoPE table (bit 2, q = 0, no K/V), row 1's slot is past its
    block table (bit 1, no K/V), row 2 appends; lens_out = positions + 1 for every row."""
    hq, hkv, d, hidden = 4, 2, 64, 256
    c = _setup(hq, hkv, d, hidden, 3, False, seed=30, max_pos=64)
    c["pos"] = torch.tensor([64, 40, 5], dtype=torch.int32, device=DEV)
    c["tables"] = torch.tensor([[1, 2], [3, 4], [5, 6]], dtype=torch.int32, device=DEV)
    outs = []
    for fn in (_fused, _two_launch):
        k, v = _pool_layer(16, hkv, 16, d, seed=6)
        before = (k.clone(), v.clone())
        lens = torch.full((3,), -5, dtype=torch.int32, device=DEV)
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        q = fn(c, hq, hkv, d, k, v, lens=lens, err=err)
        outs.append((q, k, v, lens, err, before))
    qf, kf, vf, lens, err, (k0, v0) = outs[0]
    assert int(err.item()) == 3 and lens.cpu().tolist() == [65, 41, 6]
    assert float(qf[0].abs().max()) == 0.0
    changed = (kf != k0).any(dim=(1, 2, 3)).cpu()
    assert changed.tolist() == [i == 5 for i in range(16)]  # only row 2's block 5 (position 5)
    assert torch.equal(vf[:5], v0[:5]) and torch.equal(vf[6:], v0[6:])
    for a, b in zip(outs[0][:5], outs[1][:5]):
        assert _ulps(a, b) <= 2 if a.dtype == torch.float16 else torch.equal(a, b)


def test_fused_rejects_bad_arguments():
    """More than 32 rows, a packed weight or bias of the wrong size: ValueError before any launch."""
    hq, hkv, d, hidden = 4, 2, 64, 256
    c = _setup(hq, hkv, d, hidden, 33, False, seed=40)
    k, v = _pool_layer(c["nb"], hkv, c["bs"], d, seed=7)
    with pytest.raises(ValueError):
        _fused(c, hq, hkv, d, k, v)
    c = _setup(hq, hkv, d, hidden, 4, False, seed=41)
    for key, bad in (("packed", c["packed"][:-64]), ("bias", torch.zeros(c["n"] - 16, dtype=torch.float16,
                                                                          device=DEV))):
        with pytest.raises(ValueError):
            _fused({**c, key: bad}, hq, hkv, d, k, v)


@pytest.mark.timeout(600)
def test_decode_step_fused_equals_two_launch_step():
    """Three decode steps at batch 32 on the Llama-3-8B dims (2 layers, 32768-token vocab): the
    step with the fused QKV launch and the step with the split path agree bit for bit."""
    from runtime_amd.phase2.decode_step import LLAMA3_8B, DecoderShape, Int8DecodeModel, make_contexts
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    s0 = LLAMA3_8B
    shape = DecoderShape(hidden=s0.hidden, layers=2, heads=s0.heads, kv_heads=s0.kv_heads, head_dim=s0.head_dim,
                         intermediate=s0.intermediate, vocab=32768, rope_theta=s0.rope_theta, rms_eps=s0.rms_eps)
    model = Int8DecodeModel(shape, device=DEV, seed=3, max_positions=2048)
    assert model.uses_fused_qkv(32)
    lens, tables = make_contexts(32, 64, 700, 16, 2048, headroom=4, seed=3)
    results = []
    for fused in (True, False):
        model.fuse_qkv_rope = fused
        pool = GpuKVBlockPool(num_blocks=2048, block_size_tokens=16, num_layers=2, num_kv_heads=shape.kv_heads,
                              head_dim=shape.head_dim, dtype=torch.float16, device=DEV)
        pool._ensure_pools()
        g = torch.Generator(device=DEV).manual_seed(8)
        pool._k_pool.copy_(torch.randn(pool._k_pool.shape, generator=g, device=DEV).half())
        pool._v_pool.copy_(torch.randn(pool._v_pool.shape, generator=g, device=DEV).half())
        seq = lens.to(DEV).clone()
        tokens = torch.arange(32, dtype=torch.int64, device=DEV) * 101
        logits = []
        for _ in range(3):
            tokens, lg = model.step(tokens, pool, tables.to(DEV), seq, return_logits=True, out=tokens)
            logits.append(lg.clone())
        results.append((torch.stack(logits), tokens.clone(), seq.clone(), pool._k_pool.clone(), pool._v_pool.clone()))
    model.fuse_qkv_rope = True
    for a, b in zip(*results):
        assert torch.equal(a, b)
    assert np.isfinite(results[0][0].float().cpu().numpy()).all()
