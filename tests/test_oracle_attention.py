"""CPU checks that pin the paged-attention oracle before it judges the GPU kernel."""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kv_pool, paged_attention

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _case(seed: int, bsz: int, hkv: int, grp: int, d: int, bs: int, seq_lens, num_blocks: int | None = None,
          dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    nblk = [math.ceil(s / bs) for s in seq_lens]
    max_blocks = max(max(nblk), 1) + 1
    num_blocks = num_blocks or sum(nblk) + 4
    perm = torch.randperm(num_blocks, generator=g)
    tables = torch.zeros(bsz, max_blocks, dtype=torch.int32)
    used = 0
    for b, n in enumerate(nblk):
        tables[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    k = torch.randn(num_blocks, hkv, bs, d, generator=g).to(dtype)
    v = torch.randn(num_blocks, hkv, bs, d, generator=g).to(dtype)
    q = torch.randn(bsz, hkv * grp, 1, d, generator=g).to(dtype)
    return q, k, v, tables


def _sdpa_library(q, k_layer, v_layer, tables, seq_lens, scale, grp):
    """torch's own scaled_dot_product_attention per row on gathered, GQA-expanded K/V."""
    outs = []
    for b, s in enumerate(seq_lens):
        keys, vals = kv_pool.gather_layer_view(k_layer, v_layer, tables[b].tolist(), s)
        keys = keys.float().repeat_interleave(grp, dim=1)
        vals = vals.float().repeat_interleave(grp, dim=1)
        outs.append(F.scaled_dot_product_attention(q[b:b + 1].float(), keys, vals, scale=scale))
    return torch.cat(outs, 0)


@pytest.mark.parametrize("hkv,grp,d,bs,seq_lens", [(2, 2, 32, 4, [7]), (4, 4, 64, 16, [100]),
                                                   (2, 4, 64, 16, [7, 15, 31, 63]), (8, 4, 128, 16, [1, 16, 17, 300]),
                                                   (2, 7, 64, 16, [33, 512]), (1, 1, 64, 32, [65])])
def test_rows_fp32_matches_library_sdpa(hkv, grp, d, bs, seq_lens):
    q, k, v, tables = _case(1, len(seq_lens), hkv, grp, d, bs, seq_lens)
    scale = d**-0.5
    got = paged_attention.decode_rows_fp32(q, k, v, tables, seq_lens, scale, grp)
    want = _sdpa_library(q, k, v, tables, seq_lens, scale, grp)
    assert torch.allclose(got, want, atol=2e-6, rtol=1e-5)


@pytest.mark.parametrize("hkv,grp,d,bs,s", [(2, 2, 32, 4, 7), (4, 4, 64, 16, 100)])
def test_reference_cpu_test_shapes(hkv, grp, d, bs, s):
    """The reference's CPU parity cases (tests/test_paged_attention_kernel_parity.py:81-101), restated:
    seed 42, write via the pool, SDPA on the gathered K/V vs the block-loop online softmax."""
    num_blocks = math.ceil(s / bs) + 1
    k_pool, v_pool = kv_pool.empty_pool(num_blocks, 1, hkv, bs, d)
    ids = list(range(num_blocks))
    torch.manual_seed(42)
    k = torch.randn(1, hkv, s, d)
    v = torch.randn(1, hkv, s, d)
    kv_pool.write_tokens(k_pool, v_pool, 0, ids, 0, k, v)
    query = torch.randn(1, hkv * grp, 1, d)
    scale = d**-0.5
    keys, values = kv_pool.gather_layer(k_pool, v_pool, 0, ids, s)
    expected = paged_attention.reference_sdpa_attention(query, keys, values, scale, grp)
    table = torch.tensor(ids[: math.ceil(s / bs)], dtype=torch.int32)
    actual = paged_attention.decode_blockloop(query, k_pool[:, 0], v_pool[:, 0], table, s, scale, grp)
    assert (expected - actual).abs().max().item() < 1e-5
    rows = paged_attention.decode_rows_fp32(query, k_pool[:, 0], v_pool[:, 0], table.view(1, -1), [s], scale, grp)
    assert (rows - expected).abs().max().item() < 1e-5


def test_closed_forms():
    d, bs, hkv, grp = 64, 16, 2, 3
    q, k, v, tables = _case(3, 3, hkv, grp, d, bs, [1, 40, 40])
    scale = d**-0.5
    # seq_len 1: output is V of token 0 for every head of the group.
    out = paged_attention.decode_rows_fp32(q, k, v, tables, [1, 40, 40], scale, grp)
    first = v[int(tables[0, 0]), :, 0, :]
    assert torch.allclose(out[0, :, 0, :], first.repeat_interleave(grp, 0), atol=1e-6)
    # identical keys: softmax is uniform, output is the mean of V.
    k2 = k.clone()
    for blk in tables[1, :3].tolist():
        k2[blk] = 0.5
    out2 = paged_attention.decode_rows_fp32(q, k2, v, tables, [1, 40, 40], scale, grp)
    kk, vv = kv_pool.gather_layer_view(k2, v, tables[1].tolist(), 40)
    assert torch.allclose(out2[1, :, 0, :], vv[0].mean(1).repeat_interleave(grp, 0), atol=1e-5)
    # one dominant key: output is that token's V.
    k3 = k.clone()
    blk = int(tables[2, 1])
    k3[blk, :, 5, :] = q[2, ::grp, 0, :] * 1e3
    out3 = paged_attention.decode_rows_fp32(q, k3, v, tables, [1, 40, 40], scale, grp)
    assert torch.allclose(out3[2, ::grp, 0, :], v[blk, :, 5, :], atol=1e-4)


def test_block_permutation_invariance_and_padding_never_read():
    d, bs, hkv, grp = 64, 16, 2, 4
    lens = [5, 33, 130]
    q, k, v, tables = _case(4, 3, hkv, grp, d, bs, lens, num_blocks=40)
    scale = d**-0.5
    base = paged_attention.decode_rows_fp32(q, k, v, tables, lens, scale, grp)
    perm = torch.randperm(k.shape[0], generator=torch.Generator().manual_seed(5))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    k_p, v_p = k[perm], v[perm]  # new block i holds old block perm[i]
    tables_p = inv[tables.long()].to(torch.int32)
    assert torch.allclose(paged_attention.decode_rows_fp32(q, k_p, v_p, tables_p, lens, scale, grp), base, atol=1e-6)
    # Poison every block not referenced by a valid table entry, and the table padding.
    used = set()
    for b, s in enumerate(lens):
        used.update(tables[b, :math.ceil(s / bs)].tolist())
    k_n, v_n = k.clone(), v.clone()
    for blk in range(k.shape[0]):
        if blk not in used:
            k_n[blk] = float("nan")
            v_n[blk] = float("nan")
    t_n = tables.clone()
    for b, s in enumerate(lens):
        t_n[b, math.ceil(s / bs):] = 0 if b else 7
    out = paged_attention.decode_rows_fp32(q, k_n, v_n, t_n, lens, scale, grp)
    assert torch.allclose(out, base, atol=1e-6)


@pytest.mark.parametrize("chunk", [16, 48, 64, 256])
def test_split_merge_invariance(chunk):
    d, bs, hkv, grp = 64, 16, 2, 4
    lens = [1, 17, 100, 257, 600]
    q, k, v, tables = _case(6, 5, hkv, grp, d, bs, lens)
    scale = d**-0.5
    base = paged_attention.decode_rows_fp32(q, k, v, tables, lens, scale, grp)
    split = paged_attention.decode_rows_split(q, k, v, tables, lens, scale, grp, chunk)
    assert torch.allclose(split, base, atol=2e-6, rtol=1e-5)


def test_gqa_equal_queries_equal_outputs_and_zero_length():
    d, bs, hkv, grp = 64, 16, 2, 4
    lens = [50, 0]
    q, k, v, tables = _case(8, 2, hkv, grp, d, bs, [50, 1])
    q[:, 4:8] = q[:, 4:5]
    out = paged_attention.decode_rows_fp32(q, k, v, tables, lens, d**-0.5, grp)
    assert torch.equal(out[0, 4], out[0, 7])
    assert torch.count_nonzero(out[1]) == 0


def test_max_blocks_clamp():
    """seq_len beyond the table width reads only max_blocks blocks (paged_attention_triton.py:194-196)."""
    d, bs, hkv, grp = 64, 16, 1, 2
    q, k, v, tables = _case(9, 1, hkv, grp, d, bs, [64])
    narrow = tables[:, :2]
    clamped = paged_attention.decode_rows_fp32(q, k, v, narrow, [64], d**-0.5, grp)
    exact = paged_attention.decode_rows_fp32(q, k, v, tables, [32], d**-0.5, grp)
    assert torch.allclose(clamped, exact, atol=1e-6)


def test_golden_attention_fixture_reproduces():
    f = np.load(os.path.join(GOLDEN, "attn_small.npz"))
    out = paged_attention.decode_rows_fp32(torch.from_numpy(f["q"]), torch.from_numpy(f["k_layer"]),
                                           torch.from_numpy(f["v_layer"]), torch.from_numpy(f["tables"]),
                                           f["seq_lens"].tolist(), float(f["scale"]), int(f["group"]))
    assert np.array_equal(out.numpy(), f["out"])


def test_attention_bytes():
    from runtime_amd.phase2.roofline import attention_hbm_bytes

    assert attention_hbm_bytes([16, 17], 8, 128, 32, 16) == (33 * 8 * 128 * 4 + 2 * 2 * 32 * 128 * 2
                                                                         + 3 * 4 + 2 * 4)


def test_checks_catch_planted_mistakes():
    """A wrong GQA mapping or a merge without rescaling (planted on the CPU) fails the checks."""
    d, bs, hkv, grp = 64, 16, 2, 4
    lens = [70, 200]
    q, k, v, tables = _case(10, 2, hkv, grp, d, bs, lens)
    scale = d**-0.5
    want = _sdpa_library(q, k, v, tables, lens, scale, grp)
    # h % Hkv instead of h // G.
    bad = []
    for b, s in enumerate(lens):
        keys, vals = kv_pool.gather_layer_view(k, v, tables[b].tolist(), s)
        idx = torch.arange(hkv * grp) % hkv
        sc = torch.einsum("hd,htd->ht", q[b, :, 0].float(), keys[0, idx].float()) * scale
        bad.append(torch.einsum("ht,htd->hd", sc.softmax(-1), vals[0, idx].float()))
    assert not torch.allclose(torch.stack(bad).unsqueeze(2), want, atol=1e-3)
    # Merging split partials without the exp(m_s - m*) factor.
    m = torch.tensor([[0.0, 3.0]])
    l = torch.tensor([[2.0, 1.0]])
    acc = torch.tensor([[[1.0], [5.0]]])
    good = paged_attention.merge_partials(m, l, acc)
    naive = acc.sum(-2) / l.sum(-1, keepdim=True)
    assert not torch.allclose(good, naive)


def test_valid_block_variant_pins():
    """decode_rows_fp32_valid: every id in the pool -> decode_rows_fp32; the trailing blocks of a
    row outside the pool -> the row truncated to its in-pool prefix; no block in the pool -> zeros;
    a block in the middle outside the pool -> SDPA over the remaining tokens (library routine)."""
    bs, d, hkv, grp = 8, 32, 2, 3
    lens = [40, 40, 40, 40]
    q, k, v, tables = _case(9, 4, hkv, grp, d, bs, lens, num_blocks=64)
    scale = d**-0.5
    full = paged_attention.decode_rows_fp32(q, k, v, tables, lens, scale, grp)
    assert torch.equal(paged_attention.decode_rows_fp32_valid(q, k, v, tables, lens, scale, grp, 64), full)
    t = tables.clone()
    t[0, 3:5] = 99         # row 0: blocks 3, 4 outside -> the first 24 tokens
    t[1, :5] = -1          # row 1: nothing left -> zeros
    t[2, 2] = 64           # row 2: middle block outside
    got = paged_attention.decode_rows_fp32_valid(q, k, v, t, lens, scale, grp, 64)
    trunc = paged_attention.decode_rows_fp32(q[:1], k, v, tables[:1], [24], scale, grp)
    assert torch.allclose(got[0], trunc[0], atol=1e-6)
    assert torch.count_nonzero(got[1]) == 0
    keep = [j for j in range(5) if j != 2]
    keys = torch.cat([k[int(tables[2, j])] for j in keep], dim=1).repeat_interleave(grp, dim=0).unsqueeze(0)
    vals = torch.cat([v[int(tables[2, j])] for j in keep], dim=1).repeat_interleave(grp, dim=0).unsqueeze(0)
    want2 = F.scaled_dot_product_attention(q[2:3].float(), keys.float(), vals.float(), scale=scale)
    assert torch.allclose(got[2], want2[0], atol=2e-6, rtol=1e-5)
    assert torch.equal(got[3], full[3])
