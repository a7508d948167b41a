"""Algorithmic byte counts used for roofline fractions (runtime_amd.phase2.roofline), checked
against hand counts and against the bytes of the tensors the kernels read and write."""

from __future__ import annotations

import math

import torch

from runtime_amd.phase2.roofline import attention_hbm_bytes, linear_hbm_bytes


def test_attention_bytes_hand_count():
    # Two rows of 16 and 17 tokens, Hkv 8, D 128, Hq 32, block 16: K and V of 33 tokens per
    # kv-head, q and out rows, 1 + 2 block ids and 2 lengths.
    assert attention_hbm_bytes([16, 17], 8, 128, 32, 16) == 33 * 8 * 128 * 2 * 2 + 2 * 2 * 32 * 128 * 2 + 3 * 4 + 2 * 4
    assert attention_hbm_bytes([0], 2, 64, 14, 16) == 2 * 14 * 64 * 2 + 4  # empty row: q, out, its length
    # bf16 and fp16 move the same bytes; 1-byte elements halve the K/V/q/out terms.
    assert attention_hbm_bytes([5], 1, 64, 1, 4, elem_bytes=1) == 5 * 64 * 2 + 2 * 64 + 2 * 4 + 4


def test_attention_bytes_equal_tensor_bytes():
    """Against the nbytes of the tensors one call touches (a pool with exactly the used blocks)."""
    lens, hkv, d, hq, bs = [3, 40, 129], 2, 64, 8, 16
    nblk = [math.ceil(s / bs) for s in lens]
    k = torch.zeros(sum(nblk), hkv, bs, d, dtype=torch.float16)
    q = torch.zeros(len(lens), hq, 1, d, dtype=torch.float16)
    touched_kv = sum(s * hkv * d * 2 for s in lens) * 2  # only the valid token rows
    tables = torch.zeros(sum(nblk), dtype=torch.int32)
    want = touched_kv + 2 * q.nbytes + tables.nbytes + 4 * len(lens)
    assert attention_hbm_bytes(lens, hkv, d, hq, bs) == want
    assert k.nbytes * 2 >= touched_kv  # whole blocks bound the valid rows


def test_linear_bytes():
    m, n, k = 32, 6144, 4096
    w = torch.zeros(n, k, dtype=torch.int8)
    s = torch.zeros(n, dtype=torch.float16)
    x = torch.zeros(m, k, dtype=torch.float16)
    y = torch.zeros(m, n, dtype=torch.float16)
    assert linear_hbm_bytes(m, n, k) == w.nbytes + s.nbytes + x.nbytes + y.nbytes
    assert linear_hbm_bytes(m, n, k, bias=True) == w.nbytes + 2 * s.nbytes + x.nbytes + y.nbytes
    # gate||up with the SwiGLU epilogue writes N / 2 columns.
    assert linear_hbm_bytes(m, 2 * 14336, 4096, out_cols=14336) == 2 * 14336 * 4096 + 2 * 2 * 14336 + 2 * m * 4096 + 2 * m * 14336
