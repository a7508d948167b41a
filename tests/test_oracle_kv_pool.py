"""CPU checks of the paged KV pool layout: the oracle and the product pool's host logic."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import kv_pool
from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool


def test_reference_roundtrip_kat_oracle():
    """tests/test_paged_kv_kernel.py:11-28 of the reference: K=1s, V=2s, bs=2, Hkv=2, D=4."""
    k_pool, v_pool = kv_pool.empty_pool(4, 1, 2, 2, 4)
    k = torch.ones((1, 2, 2, 4))
    v = torch.ones((1, 2, 2, 4)) * 2
    kv_pool.write_tokens(k_pool, v_pool, 0, [0, 1], 0, k, v)
    keys, values = kv_pool.gather_layer(k_pool, v_pool, 0, [0, 1], 2)
    assert keys.shape == (1, 2, 2, 4)
    assert torch.equal(keys, k) and torch.equal(values, v)


def test_reference_roundtrip_kat_product_pool():
    pool = GpuKVBlockPool(num_blocks=4, block_size_tokens=2, num_layers=1, num_kv_heads=2, head_dim=4,
                          dtype=torch.float32, device="cpu")
    k = torch.ones((1, 2, 2, 4))
    v = torch.ones((1, 2, 2, 4)) * 2
    pool.write_tokens(0, [0, 1], 0, k, v)
    keys, values = pool.gather_layer(0, [0, 1], 2)
    assert keys.shape == (1, 2, 2, 4)
    assert torch.equal(keys, k) and torch.equal(values, v)
    assert pool.allocated_block_count() == 1  # both tokens land in block 0 (bs=2)


@pytest.mark.parametrize("layout", ["split", "interleaved"])
def test_product_pool_matches_oracle_layout(layout):
    g = torch.Generator().manual_seed(0)
    nb, layers, hkv, bs, d = 12, 3, 2, 4, 8
    pool = GpuKVBlockPool(num_blocks=nb, block_size_tokens=bs, num_layers=layers, num_kv_heads=hkv, head_dim=d,
                          dtype=torch.float32, device="cpu", kv_layout=layout)
    ok, ov = kv_pool.empty_pool(nb, layers, hkv, bs, d)
    tables = torch.tensor([[3, 7, 1, 0], [9, 2, 11, 5]], dtype=torch.int32)
    starts = torch.tensor([0, 5])
    for layer in range(layers):
        k = torch.randn(2, hkv, 6, d, generator=g)
        v = torch.randn(2, hkv, 6, d, generator=g)
        pool.write_tokens_batch(layer, tables, starts, k, v)
        for b in range(2):
            kv_pool.write_tokens(ok, ov, layer, tables[b].tolist(), int(starts[b]), k[b:b + 1], v[b:b + 1])
    for layer in range(layers):  # same per-layer contents; layer-major storage
        assert torch.equal(pool.k_layer_view(layer), ok[:, layer])
        assert torch.equal(pool.v_layer_view(layer), ov[:, layer])
    k1v, v1v = pool.k_layer_view(1), pool.v_layer_view(1)
    if layout == "split":
        assert k1v.stride() == (hkv * bs * d, bs * d, d, 1) and k1v.is_contiguous()
    else:  # one (block, kv-head) holds its K run, then its V run
        assert k1v.stride() == v1v.stride() == (hkv * 2 * bs * d, 2 * bs * d, d, 1)
        assert v1v.data_ptr() - k1v.data_ptr() == bs * d * k1v.element_size()
        assert k1v[5, 1].data_ptr() - k1v.data_ptr() == (5 * hkv * 2 + 2) * bs * d * k1v.element_size()
    keys, vals = pool.gather_layer(2, tables[1].tolist(), 11)
    ok_k, ok_v = kv_pool.gather_layer(ok, ov, 2, tables[1].tolist(), 11)
    assert torch.equal(keys, ok_k) and torch.equal(vals, ok_v)
    # decode-style single-token append
    k1 = torch.randn(2, hkv, 1, d, generator=g)
    pool.write_tokens_batch(0, tables, torch.tensor([11, 15]), k1, k1)
    assert torch.equal(pool.k_layer_view(0)[int(tables[0, 2]), :, 3], k1[0, :, 0])
    assert torch.equal(pool.k_layer_view(0)[int(tables[1, 3]), :, 3], k1[1, :, 0])


def test_pool_errors_and_accounting():
    pool = GpuKVBlockPool(num_blocks=4, block_size_tokens=2, num_layers=1, num_kv_heads=1, head_dim=2,
                          dtype=torch.float32, device="cpu")
    with pytest.raises(IndexError):
        pool.write_tokens(0, [0], 0, torch.zeros(1, 1, 3, 2), torch.zeros(1, 1, 3, 2))
    with pytest.raises(IndexError):
        pool.gather_layer(0, [0], 5)
    with pytest.raises(ValueError):
        GpuKVBlockPool(num_blocks=0, block_size_tokens=2, num_layers=1, num_kv_heads=1, head_dim=2,
                       dtype=torch.float32, device="cpu")
    with pytest.raises(ValueError):
        pool.copy_blocks([0], [1, 2])
    pool.write_tokens(0, [2, 3], 0, torch.ones(1, 1, 4, 2), torch.ones(1, 1, 4, 2))
    assert pool.allocated_block_count() == 2 and pool.peak_allocated_block_count() == 2
    pool.copy_blocks([2], [0])
    k, _ = pool.gather_layer(0, [0], 2)
    assert torch.equal(k, torch.ones(1, 1, 2, 2))
    assert pool.bytes_per_block() == 1 * 1 * 2 * 2 * 2 * 4
    batch_k, _ = pool.gather_layer_batch(0, torch.tensor([[2, 3], [0, 1]]), torch.tensor([3, 1]))
    assert batch_k.shape == (2, 1, 3, 2) and torch.count_nonzero(batch_k[1, :, 1:]) == 0
    assert math.isclose(pool.peak_allocated_bytes(), pool.bytes_for_blocks(pool.peak_allocated_block_count()))
