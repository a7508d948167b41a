"""``GpuKVBlockPool.gather_layer`` / ``gather_layer_batch`` on the GPU against the oracle's gather
(``oracle/kv_pool.py``, the reference's ``paged_kv_kernel.py:252-309``), for both pool layouts.

Bar: bit-identical keys and values (a gather is a copy), zero padding past each row's length in the
batched form, and the reference's errors: ValueError for a non-positive length, IndexError when the
table holds fewer blocks than the length needs.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import kv_pool as okv

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _filled_pool(layout: str, nb: int, hkv: int, bs: int, d: int, layers: int, seed: int):
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    pool = GpuKVBlockPool(num_blocks=nb, block_size_tokens=bs, num_layers=layers, num_kv_heads=hkv, head_dim=d,
                          dtype=torch.float16, device=DEV, kv_layout=layout)
    pool._ensure_pools()
    g = torch.Generator(device=DEV).manual_seed(seed)
    for li in range(layers):
        pool.k_layer_view(li).copy_(torch.randn(pool.k_layer_view(li).shape, generator=g, device=DEV).half())
        pool.v_layer_view(li).copy_(torch.randn(pool.v_layer_view(li).shape, generator=g, device=DEV).half())
    return pool


@pytest.mark.parametrize("layout", ["interleaved", "split"])
@pytest.mark.parametrize("hkv,bs,d", [(8, 16, 128), (2, 16, 64), (1, 32, 128), (4, 8, 64)])
def test_gather_layer_and_batch_match_oracle(layout, hkv, bs, d):
    nb, layers = 96, 3
    pool = _filled_pool(layout, nb, hkv, bs, d, layers, seed=hkv * 100 + bs)
    gen = torch.Generator().manual_seed(bs + d)
    lens = [1, bs - 1, bs, bs + 1, 5 * bs + 3, 3]
    need = [math.ceil(n / bs) for n in lens]
    width = max(need) + 2  # tables longer than needed: the tail ids are never read
    perm = torch.randperm(nb, generator=gen)
    tables = torch.full((len(lens), width), -1, dtype=torch.int32)
    used = 0
    for r, n in enumerate(need):
        tables[r, : n + 1] = perm[used: used + n + 1].to(torch.int32)
        used += n + 1
    for li in range(layers):
        k_layer, v_layer = pool.k_layer_view(li).cpu(), pool.v_layer_view(li).cpu()
        want_k = torch.zeros(len(lens), hkv, max(lens), d, dtype=torch.float16)
        want_v = torch.zeros_like(want_k)
        for r, n in enumerate(lens):
            ids = tables[r, : need[r] + 1].tolist()
            k, v = pool.gather_layer(li, ids, n)
            rk, rv = okv.gather_layer_view(k_layer, v_layer, ids, n)
            assert k.shape == (1, hkv, n, d)
            assert torch.equal(k.cpu(), rk) and torch.equal(v.cpu(), rv)
            want_k[r, :, :n], want_v[r, :, :n] = rk[0], rv[0]
        print(f"gather_layer_batch layout={layout} hkv={hkv} bs={bs} d={d} layer {li}", flush=True)
        bk, bv = pool.gather_layer_batch(li, tables.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV))
        assert bk.shape == (len(lens), hkv, max(lens), d)
        assert torch.equal(bk.cpu(), want_k) and torch.equal(bv.cpu(), want_v)


def test_gather_errors_follow_the_reference():
    pool = _filled_pool("interleaved", 16, 2, 16, 64, 1, seed=3)
    with pytest.raises(ValueError):
        pool.gather_layer(0, [1, 2], 0)
    with pytest.raises(IndexError):
        pool.gather_layer(0, [1, 2], 33)  # 3 blocks needed, 2 in the table
    with pytest.raises(ValueError):
        pool.gather_layer_batch(0, torch.tensor([[1], [2]], device=DEV), torch.tensor([0, 0], device=DEV))
    with pytest.raises(IndexError):
        pool.gather_layer_batch(0, torch.tensor([[1], [2]], device=DEV), torch.tensor([16, 17], device=DEV))
