"""Oracle: paged decode attention. TEST INFRASTRUCTURE ONLY.

CPU torch restatements of the reference's attention math
(``runtime/phase2/paged_attention_triton.py``):

* :func:`reference_sdpa_attention` - ``:805-817``: K/V repeated per GQA group
  with ``repeat_interleave`` (``:812-814``), ``Q K^T * scale`` in the input
  dtype (``:815``), softmax in fp32 then cast to the query dtype (``:816``),
  ``P V`` in the input dtype (``:817``).
* :func:`decode_blockloop` - ``:663-704``: block-by-block online softmax in fp32
  with GQA by index ``kv = h // G`` (``:679``), per-block ``take`` of the last
  partial block (``:687-691``), output cast to the query dtype (``:703``).
* :func:`decode_rows_fp32` - the parity target of the HIP kernel: for every
  row, gather its ``ceil(S/bs)`` logical blocks (``paged_kv_kernel.py:252-283``)
  and evaluate softmax attention entirely in fp32. This is the per-row oracle
  the reference's batched test uses (``tests/test_paged_attention_kernel_parity.py:177-185``),
  without the unmasked zero-padding quirk of the batched torch fallback
  (``paged_attention_triton.py:720-722``), which is deliberately not a target.
* :func:`merge_partials` - ``:437-457``: log-sum-exp merge of split partials.
* :func:`decode_rows_split` - the split-K decomposition (``:245-336`` then
  ``:414-457``) at an arbitrary chunk size, used to pin the merge: its result
  must equal :func:`decode_rows_fp32` for every chunk size.

Metadata semantics (``paged_attention_triton.py:43-50``): ``seq_lens`` counts
the current token; ``block_tables`` rows are zero-padded past their valid
blocks and id 0 is a real block, so a reader bounds by ``ceil(S / bs)``, and
never by the table width alone. Like the reference's batched kernel
(``:194-196``) the number of blocks read is ``min(ceil(S/bs), max_blocks)``.

* :func:`decode_rows_fp32_valid` - the same with table entries outside the pool
  skipped (the build's contract for such ids; the reference has no check).

Parity pinning (tests/test_oracle_attention.py): torch's own
``scaled_dot_product_attention`` on gathered, GQA-expanded K/V (a library
routine); closed forms (S = 1 -> V[0]; identical keys -> mean of V;
one-hot dominant score -> that V row); invariance under physical block
permutation and under the split chunk size; GQA group members with equal
queries give equal outputs; and the reference's seeded test shapes.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def reference_sdpa_attention(query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scaling: float,
                             num_kv_groups: int) -> torch.Tensor:
    """Restatement of ``reference_sdpa_attention`` (``paged_attention_triton.py:805-817``)."""
    if num_kv_groups > 1:
        keys = keys.repeat_interleave(num_kv_groups, dim=1)
        values = values.repeat_interleave(num_kv_groups, dim=1)
    attn = torch.matmul(query, keys.transpose(2, 3)) * scaling
    attn = F.softmax(attn, dim=-1, dtype=torch.float32).to(query.dtype)
    return torch.matmul(attn, values)


def decode_blockloop(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table,
                     seq_len: int, scaling: float, num_kv_groups: int) -> torch.Tensor:
    """Restatement of ``_paged_attention_decode_torch`` (``paged_attention_triton.py:663-704``).

    ``query [1, Hq, 1, D]``, ``k_cache/v_cache [num_blocks, Hkv, bs, D]``.
    """
    _, num_heads, q_len, head_dim = query.shape
    if q_len != 1:
        raise ValueError("paged decode expects q_len=1")
    block_size = k_cache.shape[2]
    q = query[0, :, 0, :].float()
    kv_idx = torch.arange(num_heads) // num_kv_groups
    m = torch.full((num_heads,), float("-inf"))
    l = torch.zeros(num_heads)
    acc = torch.zeros(num_heads, head_dim)
    for blk in range(math.ceil(seq_len / block_size)):
        phys = int(block_table[blk])
        take = min(block_size, seq_len - blk * block_size)
        if take <= 0:
            continue
        kb = k_cache[phys, :, :take, :].float()[kv_idx]
        vb = v_cache[phys, :, :take, :].float()[kv_idx]
        scores = torch.einsum("hd,htd->ht", q, kb) * scaling
        m_new = torch.maximum(m, scores.max(dim=-1).values)
        p = torch.exp(scores - m_new.unsqueeze(-1))
        alpha = torch.exp(m - m_new)
        l = l * alpha + p.sum(dim=-1)
        acc = acc * alpha.unsqueeze(-1) + torch.einsum("ht,htd->hd", p, vb)
        m = m_new
    out = (acc / l.unsqueeze(-1)).to(query.dtype)
    return out.unsqueeze(0).unsqueeze(2)


def _row_kv(k_layer: torch.Tensor, v_layer: torch.Tensor, table_row: torch.Tensor, seq_len: int, max_blocks: int):
    block_size = k_layer.shape[2]
    nblk = min(math.ceil(seq_len / block_size), max_blocks)
    s_eff = min(seq_len, nblk * block_size)
    ids = table_row[:nblk].long()
    k = k_layer.index_select(0, ids).permute(1, 0, 2, 3).reshape(k_layer.shape[1], -1, k_layer.shape[3])[:, :s_eff]
    v = v_layer.index_select(0, ids).permute(1, 0, 2, 3).reshape(v_layer.shape[1], -1, v_layer.shape[3])[:, :s_eff]
    return k.float(), v.float()


def decode_rows_fp32(query: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor, block_tables: torch.Tensor,
                     seq_lens, scaling: float, num_kv_groups: int) -> torch.Tensor:
    """fp32 per-row paged decode attention; returns fp32 ``[B, Hq, 1, D]``.

    A row with ``seq_len <= 0`` yields zeros (the reference divides by zero
    there, ``paged_attention_triton.py:238``; this build defines it as zero).
    """
    bsz, hq, _, d = query.shape
    max_blocks = int(block_tables.shape[1])
    out = torch.zeros(bsz, hq, 1, d, dtype=torch.float32)
    kv_idx = torch.arange(hq) // num_kv_groups
    for b in range(bsz):
        s = int(seq_lens[b])
        if s <= 0:
            continue
        k, v = _row_kv(k_layer, v_layer, block_tables[b], s, max_blocks)
        q = query[b, :, 0, :].float()
        scores = torch.einsum("hd,htd->ht", q, k[kv_idx]) * scaling
        p = torch.softmax(scores, dim=-1)
        out[b, :, 0, :] = torch.einsum("ht,htd->hd", p, v[kv_idx])
    return out


def decode_rows_fp32_valid(query: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                           block_tables: torch.Tensor, seq_lens, scaling: float, num_kv_groups: int,
                           num_pool_blocks: int) -> torch.Tensor:
    """:func:`decode_rows_fp32` over the tokens whose physical block lies in ``[0, num_pool_blocks)``.

    The build's contract for a table entry outside the pool (the reference would index out of
    its slab, ``paged_kv_kernel.py:217-227``): that block's tokens are skipped, the softmax runs
    over the remaining tokens, and a row with none left is zeros. ``k_layer``/``v_layer`` only
    need to hold the in-pool blocks' rows (ids outside the pool are never indexed).
    """
    bsz, hq, _, d = query.shape
    max_blocks = int(block_tables.shape[1])
    bs = k_layer.shape[2]
    out = torch.zeros(bsz, hq, 1, d, dtype=torch.float32)
    kv_idx = torch.arange(hq) // num_kv_groups
    for b in range(bsz):
        s = int(seq_lens[b])
        nblk = min(math.ceil(max(s, 0) / bs), max_blocks)
        keys, vals = [], []
        for j in range(nblk):
            phys = int(block_tables[b, j])
            take = min(bs, s - j * bs)
            if 0 <= phys < num_pool_blocks:
                keys.append(k_layer[phys, :, :take].float())
                vals.append(v_layer[phys, :, :take].float())
        if not keys:
            continue
        k, v = torch.cat(keys, dim=1), torch.cat(vals, dim=1)
        q = query[b, :, 0, :].float()
        p = torch.softmax(torch.einsum("hd,htd->ht", q, k[kv_idx]) * scaling, dim=-1)
        out[b, :, 0, :] = torch.einsum("ht,htd->hd", p, v[kv_idx])
    return out


def merge_partials(m: torch.Tensor, l: torch.Tensor, acc: torch.Tensor) -> torch.Tensor:
    """Log-sum-exp merge (``paged_attention_triton.py:437-457``).

    ``m, l: [..., S]`` (natural-log domain), ``acc: [..., S, D]`` -> ``[..., D]``.
    """
    m_glob = m.max(dim=-1, keepdim=True).values
    w = torch.exp(m - m_glob)
    l_glob = (l * w).sum(dim=-1, keepdim=True)
    return (acc * w.unsqueeze(-1)).sum(dim=-2) / l_glob


def decode_rows_split(query: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor, block_tables: torch.Tensor,
                      seq_lens, scaling: float, num_kv_groups: int, chunk_tokens: int) -> torch.Tensor:
    """Split-K evaluation: per-chunk ``(m, l, acc)`` partials, then :func:`merge_partials`."""
    bsz, hq, _, d = query.shape
    max_blocks = int(block_tables.shape[1])
    out = torch.zeros(bsz, hq, 1, d, dtype=torch.float32)
    kv_idx = torch.arange(hq) // num_kv_groups
    for b in range(bsz):
        s = int(seq_lens[b])
        if s <= 0:
            continue
        k, v = _row_kv(k_layer, v_layer, block_tables[b], s, max_blocks)
        q = query[b, :, 0, :].float()
        ms, ls, accs = [], [], []
        for c0 in range(0, k.shape[1], chunk_tokens):
            kc = k[kv_idx, c0:c0 + chunk_tokens]
            vc = v[kv_idx, c0:c0 + chunk_tokens]
            sc = torch.einsum("hd,htd->ht", q, kc) * scaling
            mc = sc.max(dim=-1).values
            p = torch.exp(sc - mc.unsqueeze(-1))
            ms.append(mc)
            ls.append(p.sum(dim=-1))
            accs.append(torch.einsum("ht,htd->hd", p, vc))
        out[b, :, 0, :] = merge_partials(torch.stack(ms, -1), torch.stack(ls, -1), torch.stack(accs, -2))
    return out
