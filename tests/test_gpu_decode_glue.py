"""Glue kernels (KV append, fused RoPE + append, add + RMSNorm, SiLU * up) vs the CPU oracle.

Bars: index/byte work (where a token lands, what is copied) bit-exact, and
so is the fp16 residual sum (one rounding of an exact fp32 sum). Arithmetic
outputs stay within the stated atol 1e-2 / rtol 1e-2 and within a few fp16
ulps of the oracle, which rounds at the same points:

* RoPE (one rounding of an fp32 result; oracle from float64): 1 ulp;
* RMSNorm and SiLU * up round twice (``n = fp16(h * r)`` then ``fp16(n * w)``;
  ``s = fp16(silu(g))`` then ``fp16(s * u)``). The reduction order (RMSNorm) or
  ``exp`` (SiLU) can move the first rounding by 1 ulp of ``n``; scaled by ``w``
  that shifts the exact product by less than 2 ulps of the output
  (``|n w| >= |w| 2^e(n)``), so the bar is 2 ulps.
"""

from __future__ import annotations

import pytest
import torch

from oracle import glue as og

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _ulps(a: torch.Tensor, b: torch.Tensor) -> int:
    """Largest distance in fp16 units in the last place between two fp16-valued tensors."""
    def key(t):
        i = t.to(torch.float16).view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return int((key(a.cpu()) - key(b.cpu())).abs().max())


def _close(dev: torch.Tensor, ref: torch.Tensor, max_ulps: int = 1) -> None:
    torch.testing.assert_close(dev.float().cpu(), ref.float().cpu(), atol=1e-2, rtol=1e-2)
    assert _ulps(dev, ref) <= max_ulps


def _pool(nb, hkv, bs, d, layers=2, seed=0):
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    pool = GpuKVBlockPool(num_blocks=nb, block_size_tokens=bs, num_layers=layers, num_kv_heads=hkv, head_dim=d,
                          dtype=torch.float16, device=DEV)
    pool._ensure_pools()
    g = torch.Generator(device=DEV).manual_seed(seed)
    pool._k_pool.copy_(torch.randn(pool._k_pool.shape, generator=g, device=DEV).half())
    pool._v_pool.copy_(torch.randn(pool._v_pool.shape, generator=g, device=DEV).half())
    return pool


@pytest.mark.parametrize("T,transposed", [(1, False), (1, True), (7, True), (19, False)])
def test_kv_append_bit_exact(T, transposed):
    from runtime_amd.phase2.decode_glue import kv_append

    nb, hkv, bs, d, b = 64, 2, 16, 64, 3
    pool = _pool(nb, hkv, bs, d)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(T)).tolist()
    tables = torch.tensor([perm[0:4], perm[4:8], perm[8:12]], dtype=torch.int32)
    start = torch.tensor([0, 17, 40], dtype=torch.int32)
    g = torch.Generator(device=DEV).manual_seed(5)
    if transposed:  # HF's [B, T, Hkv, D] projection viewed as [B, Hkv, T, D]
        ks = torch.randn(b, T, hkv, d, generator=g, device=DEV).half().transpose(1, 2)
        vs = torch.randn(b, T, hkv, d, generator=g, device=DEV).half().transpose(1, 2)
    else:
        ks = torch.randn(b, hkv, T, d, generator=g, device=DEV).half()
        vs = torch.randn(b, hkv, T, d, generator=g, device=DEV).half()
    k_ref = pool.k_layer_view(1).cpu().clone()
    v_ref = pool.v_layer_view(1).cpu().clone()
    assert og.append_tokens(k_ref, v_ref, tables, start.tolist(), ks.cpu(), vs.cpu()) == []
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kv_append(pool.k_layer_view(1), pool.v_layer_view(1), tables.to(DEV), start.to(DEV), ks, vs, err=err)
    assert torch.equal(pool.k_layer_view(1).cpu(), k_ref)
    assert torch.equal(pool.v_layer_view(1).cpu(), v_ref)
    assert int(err.item()) == 0


def test_kv_append_skips_and_flags_out_of_range_slots():
    from runtime_amd.phase2.decode_glue import kv_append

    nb, hkv, bs, d = 16, 1, 16, 64
    pool = _pool(nb, hkv, bs, d)
    tables = torch.tensor([[3, 4], [5, 99]], dtype=torch.int32)  # row 1: bad physical id for block 1
    start = torch.tensor([30, 14], dtype=torch.int32)  # row 0: positions 30..33 pass the 2-block table
    ks = torch.randn(2, hkv, 4, d, device=DEV).half()
    k_ref = pool.k_layer_view(0).cpu().clone()
    v_ref = pool.v_layer_view(0).cpu().clone()
    skipped = og.append_tokens(k_ref, v_ref, tables, start.tolist(), ks.cpu(), ks.cpu())
    assert len(skipped) == 4
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kv_append(pool.k_layer_view(0), pool.v_layer_view(0), tables.to(DEV), start.to(DEV), ks, ks, err=err)
    assert torch.equal(pool.k_layer_view(0).cpu(), k_ref) and torch.equal(pool.v_layer_view(0).cpu(), v_ref)
    assert int(err.item()) == 1


def test_pool_write_tokens_batch_uses_kernel_and_keeps_reference_errors():
    nb, hkv, bs, d = 32, 2, 16, 128
    pool = _pool(nb, hkv, bs, d)
    tables = torch.tensor([[7, 2, 9], [1, 0, 4]], dtype=torch.int32, device=DEV)
    start = torch.tensor([5, 30], dtype=torch.int64, device=DEV)
    ks = torch.randn(2, hkv, 3, d, device=DEV).half()
    vs = torch.randn(2, hkv, 3, d, device=DEV).half()
    k_ref = pool.k_layer_view(0).cpu().clone()
    v_ref = pool.v_layer_view(0).cpu().clone()
    og.append_tokens(k_ref, v_ref, tables.cpu(), start.tolist(), ks.cpu(), vs.cpu())
    pool.write_tokens_batch(0, tables, start, ks, vs)
    pool.check_write_errors()
    assert torch.equal(pool.k_layer_view(0).cpu(), k_ref) and torch.equal(pool.v_layer_view(0).cpu(), v_ref)
    # Row 1 at positions 47..49 runs past its 3 blocks: the write is queued without a host sync,
    # the slots inside the table are written, and the reference's IndexError comes from the check.
    pool.write_tokens_batch(0, tables, torch.tensor([5, 47], device=DEV), ks, vs)
    with pytest.raises(IndexError):
        pool.check_write_errors()
    assert torch.equal(pool.k_layer_view(0)[4, :, 15].cpu(), ks[1, :, 0].cpu())


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64)])
def test_qkv_rope_append(hq, hkv, d):
    from runtime_amd.phase2.decode_glue import qkv_rope_append, rope_table

    b, nb, bs, theta, max_pos = 9, 80, 16, 5e5, 4096
    pool = _pool(nb, hkv, bs, d, seed=1)
    rope = rope_table(max_pos, d, theta, DEV)
    g = torch.Generator().manual_seed(2)
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=g).half()
    positions = torch.tensor([0, 1, 15, 16, 100, 511, 512, 2000, max_pos - 1], dtype=torch.int32)
    tables = torch.randperm(nb, generator=g)[:b * 8].to(torch.int32).view(b, 8)  # 8 distinct blocks a row
    keep = torch.tensor([int(p) // bs < 8 for p in positions])  # rows whose slot fits the table
    q_out = torch.empty(b, hq * d, dtype=torch.float16, device=DEV)
    k_before = pool.k_layer_view(1).cpu().clone()
    v_before = pool.v_layer_view(1).cpu().clone()
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    qkv_rope_append(qkv.to(DEV), rope, positions.to(DEV), q_out, pool.k_layer_view(1), pool.v_layer_view(1),
                    tables.to(DEV), hq, hkv, err=err)
    assert int(err.item()) == (0 if bool(keep.all()) else 1)

    q_ref = og.rope_rotate_half(qkv[:, :hq * d].view(b, hq, d).float(), positions, theta)
    _close(q_out.view(b, hq, d), q_ref.float())
    k_rot = og.rope_rotate_half(qkv[:, hq * d:(hq + hkv) * d].view(b, hkv, d).float(), positions, theta)
    v_new = qkv[:, (hq + hkv) * d:].view(b, hkv, d)
    k_after = pool.k_layer_view(1).cpu()
    v_after = pool.v_layer_view(1).cpu()
    touched = torch.zeros(nb, bs, dtype=torch.bool)
    for r in range(b):
        p = int(positions[r])
        if not keep[r]:
            continue
        phys = int(tables[r, p // bs])
        touched[phys, p % bs] = True
        _close(k_after[phys, :, p % bs], k_rot[r].float())
        assert torch.equal(v_after[phys, :, p % bs], v_new[r])
    # Nothing else in the layer changed.
    mask = ~touched[:, None, :, None].expand_as(k_after)
    assert torch.equal(k_after[mask], k_before[mask]) and torch.equal(v_after[mask], v_before[mask])


def test_qkv_rope_append_position_outside_table():
    from runtime_amd.phase2.decode_glue import qkv_rope_append, rope_table

    hq, hkv, d = 4, 2, 64
    pool = _pool(8, hkv, 16, d)
    rope = rope_table(32, d, 1e4, DEV)
    qkv = torch.randn(2, (hq + 2 * hkv) * d, device=DEV).half()
    q_out = torch.full((2, hq * d), 7.0, dtype=torch.float16, device=DEV)
    before = pool.k_layer_view(0).cpu().clone()
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    qkv_rope_append(qkv, rope, torch.tensor([32, 3], device=DEV), q_out, pool.k_layer_view(0),
                    pool.v_layer_view(0), torch.tensor([[1, 2], [3, 4]], dtype=torch.int32, device=DEV), hq, hkv,
                    err=err)
    assert int(err.item()) == 2
    assert float(q_out[0].abs().max()) == 0.0
    k_after = pool.k_layer_view(0).cpu()
    assert torch.equal(k_after[1], before[1])  # row 0 wrote nothing
    assert not torch.equal(k_after[3, :, 3], before[3, :, 3])  # row 1 did


def test_rope_table_matches_transformers():
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    from runtime_amd.phase2.decode_glue import rope_table

    cfg = Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2, rope_theta=1e6)
    pos = torch.arange(0, 4096, 37)
    cos, sin = Qwen2RotaryEmbedding(cfg)(torch.zeros(1, dtype=torch.float32), pos.view(1, -1))
    tab = rope_table(4096, 64, 1e6, DEV).cpu()[pos]
    torch.testing.assert_close(tab[..., 0], cos[0, :, :32], atol=1e-6, rtol=0)
    torch.testing.assert_close(tab[..., 1], sin[0, :, :32], atol=1e-6, rtol=0)


@pytest.mark.parametrize("m,h", [(1, 4096), (32, 4096), (16, 896), (100, 1024)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_add_rmsnorm(m, h, with_residual):
    from runtime_amd.phase2.decode_glue import add_rmsnorm

    g = torch.Generator().manual_seed(m + h)
    x = (3 * torch.randn(m, h, generator=g)).half()
    res = torch.randn(m, h, generator=g).half() if with_residual else None
    w = (1 + 0.2 * torch.randn(h, generator=g)).half()
    ref_out, ref_h = og.add_rmsnorm(x, w, 1e-5, residual=res)
    res_out = torch.empty(m, h, dtype=torch.float16, device=DEV) if with_residual else None
    out = add_rmsnorm(x.to(DEV), w.to(DEV), 1e-5, residual=res.to(DEV) if res is not None else None,
                      residual_out=res_out)
    _close(out, ref_out, max_ulps=2)
    if with_residual:
        assert torch.equal(res_out.cpu().float(), ref_h)


def test_add_rmsnorm_in_place_aliases():
    from runtime_amd.phase2.decode_glue import add_rmsnorm

    g = torch.Generator().manual_seed(9)
    x = torch.randn(32, 4096, generator=g).half()
    res = torch.randn(32, 4096, generator=g).half()
    w = (1 + 0.2 * torch.randn(4096, generator=g)).half()
    ref_out, ref_h = og.add_rmsnorm(x, w, 1e-6, residual=res)
    xd, rd = x.to(DEV), res.to(DEV)
    add_rmsnorm(xd, w.to(DEV), 1e-6, residual=rd, out=xd, residual_out=rd)
    _close(xd, ref_out, max_ulps=2)
    assert torch.equal(rd.cpu().float(), ref_h)


@pytest.mark.parametrize("m,i", [(1, 14336), (32, 14336), (16, 4864), (3, 8)])
def test_silu_mul(m, i):
    from runtime_amd.phase2.decode_glue import silu_mul

    g = torch.Generator().manual_seed(i)
    gu = (4 * torch.randn(m, 2 * i, generator=g)).half()
    _close(silu_mul(gu.to(DEV)), og.silu_mul(gu), max_ulps=2)


def test_glue_rejects_bad_arguments():
    from runtime_amd.phase2.decode_glue import add_rmsnorm, silu_mul

    with pytest.raises(ValueError):
        add_rmsnorm(torch.randn(2, 12, device=DEV).half(), torch.ones(12, device=DEV).half(), 1e-6)  # H % 8
    with pytest.raises(ValueError):
        silu_mul(torch.randn(2, 12, device=DEV).half())  # I = 6, not a multiple of 8
    with pytest.raises(ValueError):
        add_rmsnorm(torch.randn(2, 8), torch.ones(8), 1e-6)  # CPU tensors


def test_split_consumers_equal_fp16_consumers():
    """mx_qkv_rope_append_splits / mx_add_rmsnorm_splits on a projection's split partials give
    bit-for-bit what the fp16 kernels give on mx_w8a16_linear's output of the same projection."""
    from runtime_amd.phase2.decode_glue import (add_rmsnorm, add_rmsnorm_splits, qkv_rope_append,
                                                qkv_rope_append_splits, rope_table)
    from runtime_amd.phase2.int8_linear import (int8_linear, int8_linear_partials, linear_splits, pack_weight,
                                                quantize_weight)

    b, hq, hkv, d, hidden = 32, 32, 8, 128, 4096
    g = torch.Generator(device=DEV).manual_seed(77)
    x = torch.randn(b, hidden, generator=g, device=DEV).half()

    # qkv projection with bias -> RoPE + append
    n_qkv = (hq + 2 * hkv) * d
    q8, s8 = quantize_weight(torch.randn(n_qkv, hidden, generator=g, device=DEV) * 0.02)
    pk = pack_weight(q8)
    bias = (torch.randn(n_qkv, generator=g, device=DEV) * 0.1).half()
    splits = linear_splits(b, n_qkv, hidden)
    assert splits > 1
    part = torch.empty(splits * b * n_qkv, dtype=torch.float32, device=DEV)
    int8_linear_partials(x, pk, s8, n_qkv, part)
    qkv = int8_linear(x, pk, s8, bias, n_qkv)
    rope = rope_table(4096, d, 5e5, DEV)
    pos = torch.randint(0, 1000, (b,), generator=torch.Generator().manual_seed(1), dtype=torch.int32).to(DEV)
    tables = torch.arange(b * 64, dtype=torch.int32, device=DEV).view(b, 64)
    outs = []
    for use_splits in (False, True):
        pool = _pool(b * 64, hkv, 16, d, layers=1, seed=3)
        q_out = torch.empty(b, hq * d, dtype=torch.float16, device=DEV)
        if use_splits:
            qkv_rope_append_splits(part, splits, bias, rope, pos, q_out, pool.k_layer_view(0), pool.v_layer_view(0),
                                   tables, hq, hkv)
        else:
            qkv_rope_append(qkv, rope, pos, q_out, pool.k_layer_view(0), pool.v_layer_view(0), tables, hq, hkv)
        outs.append((q_out.clone(), pool.k_layer_view(0).clone(), pool.v_layer_view(0).clone()))
    for a, c in zip(*outs):
        assert torch.equal(a, c)

    # o projection (no bias) -> residual add + RMSNorm
    o8, os8 = quantize_weight(torch.randn(hidden, hidden, generator=g, device=DEV) * 0.02)
    po = pack_weight(o8)
    so = linear_splits(b, hidden, hidden)
    part_o = torch.empty(so * b * hidden, dtype=torch.float32, device=DEV)
    int8_linear_partials(x, po, os8, hidden, part_o)
    y = int8_linear(x, po, os8, None, hidden)
    res = torch.randn(b, hidden, generator=g, device=DEV).half()
    w = (1 + 0.1 * torch.randn(hidden, generator=g, device=DEV)).half()
    ra, rb = res.clone(), res.clone()
    out_a = add_rmsnorm(y, w, 1e-5, residual=ra, residual_out=ra)
    out_b = torch.empty_like(out_a)
    add_rmsnorm_splits(part_o, so, None, w, 1e-5, out_b, residual=rb, residual_out=rb)
    assert torch.equal(out_a, out_b) and torch.equal(ra, rb)


def test_qkv_rope_append_writes_lengths():
    """``lens_out`` receives ``positions + 1`` (the attention lengths after the append), also when a row's
    slot lies outside its table."""
    from runtime_amd.phase2.decode_glue import qkv_rope_append, rope_table

    hq, hkv, d = 4, 2, 64
    pool = _pool(8, hkv, 16, d)
    rope = rope_table(64, d, 1e4, DEV)
    qkv = torch.randn(3, (hq + 2 * hkv) * d, device=DEV).half()
    q_out = torch.empty(3, hq * d, dtype=torch.float16, device=DEV)
    positions = torch.tensor([0, 17, 40], dtype=torch.int32, device=DEV)
    lens = torch.full((3,), -5, dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    qkv_rope_append(qkv, rope, positions, q_out, pool.k_layer_view(0), pool.v_layer_view(0),
                    torch.tensor([[1, 2], [3, 4], [5, 6]], dtype=torch.int32, device=DEV), hq, hkv, err=err,
                    lens_out=lens)
    assert lens.cpu().tolist() == [1, 18, 41]
    assert int(err.item()) == 1  # position 40 lies past row 2's two blocks (bit 1: slot outside the table)


def test_add_rmsnorm_gathers_rows():
    """``rows`` reads row ``rows[m]`` of x (the embedding lookup); an out-of-range index reads a zero row."""
    from runtime_amd.phase2.decode_glue import add_rmsnorm

    vocab, h = 1000, 896
    g = torch.Generator().manual_seed(11)
    emb = (torch.randn(vocab, h, generator=g) * 0.5).half()
    w = (1.0 + 0.05 * torch.randn(h, generator=g)).half()
    rows = torch.tensor([0, 999, 5, 5, 123, 998, 1000, -1], dtype=torch.int64)
    valid = (rows >= 0) & (rows < vocab)
    out = torch.empty(8, h, dtype=torch.float16, device=DEV)
    h_out = torch.full((8, h), 3.0, dtype=torch.float16, device=DEV)
    add_rmsnorm(emb.to(DEV), w.to(DEV), 1e-6, out=out, residual_out=h_out, rows=rows.to(DEV))
    x = emb[rows.clamp(0, vocab - 1)] * valid[:, None].half()
    ref_out, ref_h = og.add_rmsnorm(x, w, 1e-6)
    assert torch.equal(h_out.cpu(), x)
    _close(out[valid.to(DEV)], ref_out[valid], max_ulps=2)
    assert float(out[~valid.to(DEV)].abs().max()) == 0.0


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("m,n", [(1, 8), (3, 128256), (32, 151936), (5, 1000), (2, 4096), (2, 4097), (128, 128256)])
def test_argmax_rows_matches_torch(m, n, split):
    from runtime_amd.phase2.decode_glue import argmax_rows

    g = torch.Generator().manual_seed(m * 1000 + n)
    logits = torch.randn(m, n, generator=g).half()
    got = argmax_rows(logits.to(DEV), split=split).cpu()
    assert got.dtype == torch.int64
    assert torch.equal(got, logits.float().argmax(dim=-1))


def test_argmax_split_ties_across_chunks_and_signed_zero():
    """The chunked argmax keys: equal maxima in different 4096-logit chunks give the first index;
    -0 and +0 tie (the first wins, as torch compares values); the smallest negative numbers order
    below -0 and above -inf; a NaN in a later chunk still wins over +inf in an earlier one."""
    from runtime_amd.phase2.decode_glue import argmax_rows

    n = 3 * 4096 + 5
    lg = torch.full((6, n), -1.0, dtype=torch.float16)
    lg[0, [9000, 4100, 12000]] = 3.0                     # first of three equal maxima: 4100
    lg[1, :] = 0.0; lg[1, :5000] = -0.0                  # -0 before +0: index 0
    lg[2, :] = float("-inf"); lg[2, 7000] = -65504.0     # the only finite value
    lg[2, 8000] = -2.0**-24                              # smallest-magnitude negative beats -65504
    lg[3, 100] = float("inf"); lg[3, 8200] = float("nan")
    lg[4, n - 1] = 0.5; lg[4, n - 5] = 0.5               # ties in the partial last chunk
    lg[5, :] = float("nan")                              # all NaN: index 0
    want = [4100, 0, 8000, 8200, n - 5, 0]
    for split in (True, False):
        got = argmax_rows(lg.to(DEV), split=split).cpu().tolist()
        assert got == want, f"split={split}: {got}"
    assert lg.float().argmax(dim=-1).tolist() == want


@pytest.mark.parametrize("split", [True, False])
def test_argmax_rows_ties_nan_inf_and_lengths(split):
    """First index on ties; NaN counts above every number (torch's convention, first NaN wins); -inf rows;
    ``seq_lens`` advances by one per row; a strided logits view reads only its N columns."""
    from runtime_amd.phase2.decode_glue import argmax_rows

    n = 5001  # not a multiple of 8: the tail loop
    base = torch.zeros(6, n + 7, dtype=torch.float16)
    base[:, n:] = 100.0  # padding outside the view must not count
    lg = base[:, :n]
    lg[0, [17, 4000, 4999]] = 2.0                 # tie: first index
    lg[1, :] = float("-inf")                      # all -inf: index 0
    lg[2, 300] = float("nan"); lg[2, 10] = 65504  # NaN wins over the largest finite value
    lg[3, [2500, 2501]] = float("nan")            # two NaNs: the first
    lg[4, n - 1] = 1.0                            # last column
    lg[5, :] = -1.0; lg[5, 1234] = float("inf")   # +inf
    dev = base.to(DEV)[:, :n]
    lens = torch.tensor([3, 0, 9, 1, 1, 2047], dtype=torch.int32, device=DEV)
    out = torch.full((6,), -1, dtype=torch.int64, device=DEV)
    argmax_rows(dev, out=out, seq_lens=lens, split=split)
    assert out.cpu().tolist() == [17, 0, 300, 2500, n - 1, 1234]
    assert out.cpu().tolist() == lg.float().argmax(dim=-1).tolist()
    assert lens.cpu().tolist() == [4, 1, 10, 2, 2, 2048]
