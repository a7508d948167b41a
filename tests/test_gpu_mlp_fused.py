"""The fused MLP launch (``mx_w8a16_mlp_fused_partials``) against the two launches it replaces
(``mx_w8a16_gateup_swiglu``, then ``mx_w8a16_linear_partials`` of its output).

Bar: bit-identical activations and partials (both phases run the standalone kernels' code in the
same k order), on calls in a row with fresh inputs and a smaller batch between them (the launch
clears its own counters), inside a replayed HIP graph, and through the native decode step, whose
tokens and logits must not change when the MLP is fused.
"""

from __future__ import annotations

import pytest
import torch

from runtime_amd.phase2.int8_linear import (MLP_SYNC_ERR, MLP_SYNC_WORDS, gateup_interleave, int8_gateup_swiglu,
                                            int8_linear_partials, int8_mlp_fused_partials, linear_splits,
                                            mlp_fusable, pack_weight, quantize_weight)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
K, I, N = 4096, 14336, 4096  # the Llama-3-8B MLP


def _require_fusable(m: int) -> None:
    if not mlp_fusable(m, K, I, N):
        pytest.skip("this device cannot hold every workgroup of the fused launch at once")


@pytest.fixture(scope="module")
def mlp():
    g = torch.Generator(device=DEV).manual_seed(11)
    gate = torch.randn(I, K, generator=g, device=DEV) * 0.02
    up = torch.randn(I, K, generator=g, device=DEV) * 0.02
    qgu, sgu = quantize_weight(gateup_interleave(gate, up))
    del gate, up
    qd, sd = quantize_weight(torch.randn(N, I, generator=g, device=DEV) * 0.02)
    return (pack_weight(qgu), sgu, 2 * I, None), (pack_weight(qd), sd, N, None)


def _apart(x, gu, dn):
    m = x.shape[0]
    act = int8_gateup_swiglu(x, gu[0], gu[1], gu[3], I)
    ks = linear_splits(m, N, I)
    part = torch.empty(ks * m * N, dtype=torch.float32, device=DEV)
    int8_linear_partials(act, dn[0], dn[1], N, part)
    return act, part, ks


def _x(m: int, seed: int) -> torch.Tensor:
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(m, K, generator=g, device=DEV) * 0.5).half()


def test_fused_mlp_bit_identical_on_calls_in_a_row(mlp):
    gu, dn = mlp
    _require_fusable(32)
    act = torch.full((32, I), float("nan"), dtype=torch.float16, device=DEV)
    part = torch.full((linear_splits(32, N, I) * 32 * N,), float("nan"), dtype=torch.float32, device=DEV)
    sync = torch.zeros(MLP_SYNC_WORDS, dtype=torch.int32, device=DEV)
    for seed, m in enumerate((32, 32, 8, 16, 32, 5)):
        if not mlp_fusable(m, K, I, N):
            continue
        print(f"fused MLP call {seed}: M={m}", flush=True)
        x = _x(m, seed)
        ks = int8_mlp_fused_partials(x, gu, dn, act[:m], part, sync)
        want_act, want_part, want_ks = _apart(x, gu, dn)
        torch.cuda.synchronize()
        assert ks == want_ks > 1
        assert torch.equal(act[:m], want_act)
        assert torch.equal(part[:ks * m * N], want_part)
        words = sync.tolist()
        assert words[MLP_SYNC_ERR] == 0
        assert words[:MLP_SYNC_ERR] == [0] * MLP_SYNC_ERR  # counters cleared for the next call


def test_fused_mlp_with_gate_up_bias(mlp):
    """A gate||up bias (interleaved like the weight rows) enters the fused launch's epilogue exactly as
    it enters mx_w8a16_gateup_swiglu's."""
    gu, dn = mlp
    _require_fusable(16)
    g = torch.Generator(device=DEV).manual_seed(7)
    bias = gateup_interleave(torch.randn(I, generator=g, device=DEV) * 0.1,
                             torch.randn(I, generator=g, device=DEV) * 0.1).half()
    gub = (gu[0], gu[1], gu[2], bias)
    m = 16
    x = _x(m, 55)
    act = torch.empty(m, I, dtype=torch.float16, device=DEV)
    ks = linear_splits(m, N, I)
    part = torch.empty(ks * m * N, dtype=torch.float32, device=DEV)
    sync = torch.zeros(MLP_SYNC_WORDS, dtype=torch.int32, device=DEV)
    assert int8_mlp_fused_partials(x, gub, dn, act, part, sync) == ks
    want_act, want_part, _ = _apart(x, gub, dn)
    torch.cuda.synchronize()
    assert torch.equal(act, want_act)
    assert torch.equal(part, want_part)
    assert sync.tolist() == [0] * MLP_SYNC_WORDS


def test_fused_mlp_graph_replays(mlp):
    """Captured once, replayed with new inputs copied in between and the two-launch reference run
    eagerly between the replays: every replay equals it."""
    gu, dn = mlp
    _require_fusable(32)
    m = 32
    x = _x(m, 100)
    act = torch.empty(m, I, dtype=torch.float16, device=DEV)
    ks = linear_splits(m, N, I)
    part = torch.empty(ks * m * N, dtype=torch.float32, device=DEV)
    sync = torch.zeros(MLP_SYNC_WORDS, dtype=torch.int32, device=DEV)
    int8_mlp_fused_partials(x, gu, dn, act, part, sync)  # eager first call
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        int8_mlp_fused_partials(x, gu, dn, act, part, sync)
    for rep in range(4):
        print(f"fused MLP graph replay {rep}", flush=True)
        x.copy_(_x(m, 101 + rep))
        graph.replay()
        torch.cuda.synchronize()
        got_act, got_part = act.clone(), part.clone()
        want_act, want_part, _ = _apart(x, gu, dn)
        assert torch.equal(got_act, want_act)
        assert torch.equal(got_part, want_part)
        assert sync.tolist() == [0] * MLP_SYNC_WORDS


@pytest.mark.timeout(300)
def test_native_step_same_bits_with_fused_mlp():
    """The Llama-3-8B-shaped native step (2 layers, batch 32, graph replays) with the MLP fused and
    with its two launches: identical logits, tokens, K/V and lengths after 6 steps."""
    from runtime_amd.phase2.decode_step import LLAMA3_8B, Int8DecodeModel, make_contexts
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    _require_fusable(32)
    native = Int8DecodeModel(LLAMA3_8B, device=DEV, seed=9, layers=2)
    s = native.shape
    bsz, bs, nblk = 32, 16, 4096
    lens, tables = make_contexts(bsz, 128, 1024, bs, nblk, headroom=7, seed=9)
    g = torch.Generator(device=DEV).manual_seed(10)
    pool = GpuKVBlockPool(num_blocks=nblk, block_size_tokens=bs, num_layers=2, num_kv_heads=s.kv_heads,
                          head_dim=s.head_dim, dtype=torch.float16, device=DEV)
    pool._ensure_pools()
    init_k = torch.randn(pool._k_pool.shape, generator=g, device=DEV).half()
    init_v = torch.randn(pool._v_pool.shape, generator=g, device=DEV).half()
    runs = {}
    for fused in (True, False):
        native.fuse_mlp = fused
        pool._k_pool.copy_(init_k)
        pool._v_pool.copy_(init_v)
        seq = lens.to(DEV).clone()
        tok = torch.arange(bsz, device=DEV, dtype=torch.int64) * 997
        tdev = tables.to(DEV)
        native.step(tok, pool, tdev, seq, out=tok)  # eager: sizes the buffers
        assert native.buffers(bsz).mlp_fused
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            _, logits = native.step(tok, pool, tdev, seq, return_logits=True, out=tok)
        seen = []
        for rep in range(6):
            print(f"native step fused_mlp={fused} replay {rep}", flush=True)
            graph.replay()
            seen.append((logits.clone(), tok.clone()))
        torch.cuda.synchronize()
        runs[fused] = (seen, pool._k_pool.clone(), pool._v_pool.clone(), seq.clone())
        del graph
    assert native.error_flag() == 0
    (a, ka, va, sa), (b, kb, vb, sb) = runs[True], runs[False]
    assert torch.equal(sa, sb)
    for (la, ta), (lb, tb) in zip(a, b):
        assert torch.equal(la, lb) and torch.equal(ta, tb)
    assert torch.equal(ka, kb) and torch.equal(va, vb)
