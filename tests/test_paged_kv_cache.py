"""CPU tests of the transformers cache adapters over the block pool.

Decode attention itself needs the GPU (the hook only takes the HIP path for
device queries, as the reference's does); here the pool writes, length
bookkeeping, published metadata, slot management and the prefill path
(eager attention over gathered K/V) are checked against DynamicCache and the
pool oracle.
"""

from __future__ import annotations

import pytest
import torch

from oracle import kv_pool as okv
from oracle import model as om
from runtime_amd.phase2.hf_decode import enable_block_paged_attention, prefill_request
from runtime_amd.phase2.paged_attention_hip import get_paged_decode_batch_metadata, set_paged_decode_batch_metadata
from runtime_amd.phase2.paged_kv_cache import BlockPagedBatchCache, BlockPagedCache
from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

TINY = dict(hidden_size=128, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
            intermediate_size=256, vocab_size=512, max_position_embeddings=256)
HKV, D, BS = 2, 32, 4


def _pool(num_blocks=64, layers=2):
    return GpuKVBlockPool(num_blocks=num_blocks, block_size_tokens=BS, num_layers=layers, num_kv_heads=HKV,
                          head_dim=D, dtype=torch.float32, device="cpu")


class _Cfg:
    num_hidden_layers = 2


@pytest.fixture(autouse=True)
def _clear_metadata():
    set_paged_decode_batch_metadata(None)
    yield
    set_paged_decode_batch_metadata(None)


def test_prefill_through_block_paged_cache_matches_dynamic_cache():
    model = om.random_qwen2(seed=11, **TINY)
    enable_block_paged_attention(model)
    pool = _pool()
    prompt = torch.randint(0, TINY["vocab_size"], (1, 13), generator=torch.Generator().manual_seed(1))
    blocks = [9, 3, 40, 17]
    cache, logits = prefill_request(model, pool, blocks, prompt)
    assert cache.get_seq_length() == 13 and cache.layers[1].get_seq_length() == 13
    assert get_paged_decode_batch_metadata() is None

    model.config._attn_implementation = "eager"
    ref = model(input_ids=prompt, use_cache=True)
    torch.testing.assert_close(logits, ref.logits[:, -1], atol=1e-5, rtol=1e-5)
    # The pool holds exactly the keys/values HF cached, at the table's blocks.
    for layer in range(2):
        k, v = okv.gather_layer_view(pool.k_layer_view(layer), pool.v_layer_view(layer), blocks, 13)
        torch.testing.assert_close(k, ref.past_key_values.layers[layer].keys, atol=0, rtol=0)
        torch.testing.assert_close(v, ref.past_key_values.layers[layer].values, atol=0, rtol=0)


def test_request_cache_decode_update_publishes_metadata():
    pool = _pool()
    cache = BlockPagedCache(_Cfg(), pool)
    cache.set_block_ids([5, 6])
    layer = cache.layers[1]
    k = torch.randn(1, HKV, 6, D)
    layer.update(k, k + 1)
    assert get_paged_decode_batch_metadata() is None
    k1 = torch.randn(1, HKV, 1, D)
    out_k, _ = layer.update(k1, k1 - 1)
    assert out_k is k1
    meta = get_paged_decode_batch_metadata()
    assert meta.layer_idx == 1 and meta.block_tables.tolist() == [[5, 6]] and meta.seq_lens.tolist() == [7]
    got_k, got_v = okv.gather_layer_view(pool.k_layer_view(1), pool.v_layer_view(1), [5, 6], 7)
    torch.testing.assert_close(got_k[:, :, 6:], k1, atol=0, rtol=0)
    torch.testing.assert_close(got_v[:, :, :6], k + 1, atol=0, rtol=0)
    with pytest.raises(IndexError):
        layer.update(torch.randn(1, HKV, 2, D), torch.randn(1, HKV, 2, D))
    assert cache.layers[0].get_seq_length() == 0


def _two_request_caches(pool):
    caches = []
    for blocks, n in (([1, 2, 3], 9), ([7], 2)):
        c = BlockPagedCache(_Cfg(), pool)
        c.set_block_ids(blocks)
        for layer in c.layers:
            layer.update(torch.randn(1, HKV, n, D), torch.randn(1, HKV, n, D))
        caches.append(c)
    return caches


@pytest.mark.parametrize("graph_safe", [False, True])
def test_batch_cache_decode_writes_rows_at_their_lengths(graph_safe):
    pool = _pool()
    batch = BlockPagedBatchCache.from_caches(_two_request_caches(pool), pool)
    batch._graph_safe = graph_safe
    batch._cached_seq_len_py = 9 if graph_safe else None
    assert batch.block_tables.tolist() == [[1, 2, 3], [7, 0, 0]]
    assert batch.seq_lens.tolist() == [9, 2] and batch.get_seq_length() == 9
    seq_lens_obj = batch.seq_lens
    new_k = torch.randn(2, HKV, 1, D)
    new_v = torch.randn(2, HKV, 1, D)
    for layer in batch.layers:
        layer.update(new_k + layer.layer_idx, new_v - layer.layer_idx)
        meta = get_paged_decode_batch_metadata()
        assert meta.layer_idx == layer.layer_idx
        assert meta.block_tables is batch.block_tables and meta.seq_lens is batch.seq_lens
        assert meta.seq_lens.tolist() == [10, 3]
    assert (batch.seq_lens is seq_lens_obj) == graph_safe
    for layer_idx in range(2):
        for row, (blocks, n) in enumerate((([1, 2, 3], 10), ([7], 3))):
            k, v = okv.gather_layer_view(pool.k_layer_view(layer_idx), pool.v_layer_view(layer_idx), blocks, n)
            torch.testing.assert_close(k[0, :, n - 1], new_k[row, :, 0] + layer_idx, atol=0, rtol=0)
            torch.testing.assert_close(v[0, :, n - 1], new_v[row, :, 0] - layer_idx, atol=0, rtol=0)
    expect = 9 if graph_safe else 10
    assert batch.layers[0].get_seq_length() == expect
    assert batch.layers[0].get_mask_sizes(1) == (expect + 1, 0)


def test_batch_cache_prefill_update_gathers_and_clears_metadata():
    pool = _pool()
    batch = BlockPagedBatchCache.from_caches(_two_request_caches(pool), pool)
    set_paged_decode_batch_metadata(object())
    k, v = batch.layers[0].update(torch.randn(2, HKV, 2, D), torch.randn(2, HKV, 2, D))
    assert get_paged_decode_batch_metadata() is None
    assert k.shape == (2, HKV, 11, D) and batch.seq_lens.tolist() == [11, 4]
    assert float(k[1, :, 4:].abs().max()) == 0.0  # zero padding past the short row


def test_persistent_slots_bind_dense_write_back_extract():
    pool = _pool()
    a, b = _two_request_caches(pool)
    persistent = BlockPagedBatchCache.empty(_Cfg(), pool, max_batch_size=3, max_blocks=2)
    assert persistent.bind_cache("a", a) == 0
    assert persistent.bind_cache("b", b) == 1
    assert persistent.bind_cache("a", a) == 0 and persistent.slot_of("b") == 1 and persistent.slot_of("zz") is None
    assert persistent.block_tables.shape == (3, 3)  # grown to a's three blocks
    assert persistent.block_tables.tolist() == [[1, 2, 3], [7, 0, 0], [0, 0, 0]]
    assert persistent.seq_lens.tolist() == [9, 2, 0]
    assert persistent.layers[1]._row_seq_lens.tolist() == [9, 2, 0]

    dense, slots = persistent.dense_active_cache(["b", "a"])
    assert slots == [1, 0] and dense.block_tables.tolist() == [[7, 0, 0], [1, 2, 3]]
    for layer in dense.layers:
        layer.update(torch.randn(2, HKV, 1, D), torch.randn(2, HKV, 1, D))
    dense.block_ids_rows[0] = [7, 8]
    persistent.write_back_dense(dense, slots)
    assert persistent.seq_lens.tolist() == [10, 3, 0]
    assert persistent.block_tables[1].tolist() == [7, 8, 0]
    assert persistent.layers[0]._row_seq_lens.tolist() == [10, 3, 0]

    ex = persistent.extract_cache(1)
    assert ex.block_table_ids == [7, 8] and ex.get_seq_length() == 3 and ex.layers[1].get_seq_length() == 3

    persistent.release_slot("b")
    assert persistent.seq_lens.tolist() == [10, 0, 0] and persistent.block_tables[1].tolist() == [0, 0, 0]
    assert persistent.allocate_slot("c") == 1
    assert persistent.allocate_slot("d") == 2
    with pytest.raises(RuntimeError):
        persistent.allocate_slot("e")
    with pytest.raises(KeyError):
        persistent.dense_active_cache(["b"])
    with pytest.raises(ValueError):
        BlockPagedBatchCache.empty(_Cfg(), pool, max_batch_size=0, max_blocks=1)
    with pytest.raises(ValueError):
        BlockPagedBatchCache.from_caches([], pool)


def test_greedy_decode_plumbing_with_oracle_attention():
    """The whole driver (prefill, bind, ragged batched decode at per-row positions)
    on the CPU, with the oracle's paged attention standing in for the HIP kernel,
    reproduces per-row greedy decode with DynamicCache."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    from oracle.paged_attention import decode_rows_fp32
    from runtime_amd.phase2 import block_paged_attention as bpa
    from runtime_amd.phase2.hf_decode import greedy_decode

    def cpu_hook(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
        meta = get_paged_decode_batch_metadata()
        if meta is not None and query.shape[-2] == 1:
            out = decode_rows_fp32(query, meta.pool.k_layer_view(meta.layer_idx), meta.pool.v_layer_view(meta.layer_idx),
                                   meta.block_tables, meta.seq_lens, scaling, module.num_key_value_groups)
            return out.to(query.dtype).transpose(1, 2).contiguous(), None
        return bpa.block_paged_attention_forward(module, query, key, value, attention_mask, scaling, dropout, **kwargs)

    model = om.random_qwen2(seed=21, **TINY)
    g = torch.Generator().manual_seed(4)
    prompts = [torch.randint(0, TINY["vocab_size"], (n,), generator=g) for n in (5, 11, 8)]
    steps = 6
    rows = [[30, 2, 17, 9], [4, 44, 12, 50, 8], [61, 0, 33, 6]]
    pool = _pool()
    ALL_ATTENTION_FUNCTIONS.register("block_paged", cpu_hook)
    model.config._attn_implementation = "block_paged"
    try:
        tokens, logits = greedy_decode(model, pool, prompts, rows, steps, keep_logits=True)
    finally:
        bpa.register_block_paged_attention()
    model.config._attn_implementation = "eager"
    for b, prompt in enumerate(prompts):
        ref_tokens, ref_logits = om.greedy_reference(model, prompt, steps)
        torch.testing.assert_close(logits[b], ref_logits, atol=1e-4, rtol=1e-4)
        assert tokens[b].tolist() == ref_tokens.tolist()
    with pytest.raises(ValueError):
        greedy_decode(model, pool, prompts[:1], [[1]], steps)
