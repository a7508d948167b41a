"""The worker's paged decode sequence on the GPU (``TransformersBackend``,
``runtime/phase2/worker_server.py``), through ``hf_decode.PagedDecoder``:

* persistent slots: ``_bind_states_to_persistent`` -> ``dense_active_cache`` -> the HF
  forward through the ``block_paged`` hook -> ``write_back_dense`` -> ``extract_cache``
  (``:619-641,740-782``), with a request finishing and a new one joining its slot;
* the batch-1 ``BlockPagedLayer`` decode (``kv_len == 1``, one request alone, ``:746-756``);
* the HIP-graph replay of the step (``hip_graph_decode``, the reference's
  ``cuda_graph_decode.py``) against eager decode, token for token (the reference's
  contract, ``tests/test_cuda_graph_decode.py:88-109``);
* the pool's deferred KV-write checks: no host sync per layer, an overrun raised as
  ``IndexError`` by ``check_write_errors``, block usage counted from the device map.

Model: the Qwen2-0.5B widths (hidden 896, 14/2 heads, head_dim 64, SwiGLU 4864) with 2
layers and a 32768-token vocabulary, int8 projections (``quantize_model_``), fp16. The
oracle and the rules are those of the greedy-decode tests: the fp32 HF model with the
same weights, teacher-forced on each request's tokens; logits within
``max(1e-2, 1.25 x torch fp16's error)``, token mismatches only at near ties.
"""

from __future__ import annotations

import copy
import math

import pytest
import torch

from conftest import report
from oracle import model as om

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
BS = 16
LOGIT_ATOL = 1e-2
YARDSTICK_SLACK = 1.25


def _model(seed: int):
    from runtime_amd.phase2.hf_decode import enable_block_paged_attention
    from runtime_amd.phase2.int8_linear import quantize_model_

    model = om.random_qwen2(seed=seed, num_hidden_layers=2, vocab_size=32768)
    ref = om.quantized_reference(model)
    torch16 = om.to_device_dtype(copy.deepcopy(ref), DEV, torch.float16).eval()
    quantize_model_(model, device=DEV)
    om.to_device_dtype(model, DEV, torch.float16)
    enable_block_paged_attention(model)
    return model, ref, torch16


def _pool(num_blocks: int):
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    return GpuKVBlockPool(num_blocks=num_blocks, block_size_tokens=BS, num_layers=2, num_kv_heads=2, head_dim=64,
                          dtype=torch.float16, device=DEV)


def _admit(model, pool, rid: str, prompt: torch.Tensor, blocks: list[int]):
    from runtime_amd.phase2.hf_decode import DecodeRequest, DecodeState, prefill_request

    cache, logits = prefill_request(model, pool, blocks, prompt.view(1, -1).to(DEV))
    tok = int(logits.argmax())
    state = DecodeState(DecodeRequest(rid), cache, tok, [tok])
    state.prompt, state.blocks, state.logits = prompt, blocks, [logits[0].float().cpu()]
    return state


def _compare(ref, torch16, state) -> tuple[float, float, dict]:
    gen = torch.tensor(state.generated_token_ids)
    ref_logits = om.teacher_forced_logits(ref, state.prompt, gen)
    ids = torch.cat([state.prompt, gen[:-1]]).view(1, -1).to(DEV)
    with torch.no_grad():
        t16 = torch16(input_ids=ids, use_cache=False, logits_to_keep=len(gen)).logits[0].float().cpu()
    mine = torch.stack(state.logits)
    err = float((mine - ref_logits).abs().max())
    err16 = float((t16 - ref_logits).abs().max())
    allowed = max(LOGIT_ATOL, YARDSTICK_SLACK * err16)
    return err, allowed, om.greedy_agreement(ref_logits, gen, tie_tol=2 * allowed)


@pytest.mark.timeout(600)
def test_worker_persistent_slots_and_single_row_decode():
    from runtime_amd.phase2.hf_decode import PagedDecoder

    model, ref, torch16 = _model(seed=21)
    g = torch.Generator().manual_seed(21)
    lens = [int(x) for x in torch.randint(20, 200, (7,), generator=g)]
    steps_max = 12
    need = [math.ceil((n + steps_max + 1) / BS) for n in lens]
    nb = 2 * sum(need)
    perm = torch.randperm(nb, generator=g).tolist()
    rows, at = [], 0
    for n in need:
        rows.append(perm[at:at + n])
        at += n
    pool = _pool(nb)
    prompts = [torch.randint(0, 32768, (n,), generator=g) for n in lens]
    states = [_admit(model, pool, f"r{i}", prompts[i], rows[i]) for i in range(6)]
    dec = PagedDecoder(model, pool, max_active=8)

    def step(active):
        dec.decode_step(active)
        logits = dec.last_logits.float().cpu()
        for i, s in enumerate(active):
            s.logits.append(logits[i])

    for _ in range(4):           # six rows: dense_active_cache -> forward -> write_back_dense
        step(states)
    finished = states.pop(2)     # a request finishes; a new one takes its slot
    slot = dec._paged_persistent.slot_of("r2")
    dec.release("r2")
    states.append(_admit(model, pool, "r6", prompts[6], rows[6]))
    for _ in range(4):
        step(states)
    assert dec._paged_persistent.slot_of("r6") == slot
    for _ in range(3):           # one request alone: the batch-1 BlockPagedLayer decode
        step(states[:1])
    pool.check_write_errors()

    results = []
    for s in states + [finished]:
        err, allowed, agree = _compare(ref, torch16, s)
        results.append((s.req.request_id, len(s.generated_token_ids), err, allowed, agree))
    summary = ", ".join(f"{r[0]}: {r[1]} tokens, err {r[2]:.2e}, mism {r[4]['mismatches']}" for r in results)
    for rid, n, err, allowed, agree in results:
        assert err <= allowed, f"{rid}: logits off by {err:.3e} (allowed {allowed:.3e}); {summary}"
        assert agree["ties_ok"], f"{rid}: mismatch outside the near-tie band {agree}; {summary}"
    # Lengths and block usage, from the device: every token written went to its row's blocks.
    persistent = dec._paged_persistent
    for s in states:
        n = len(s.prompt) + len(s.generated_token_ids) - 1
        assert s.past_key_values.get_seq_length() == n
        assert int(persistent.seq_lens[persistent.slot_of(s.req.request_id)]) == n
    used = set()
    for s in states + [finished]:
        n = len(s.prompt) + len(s.generated_token_ids) - 1
        used.update(s.blocks[:math.ceil(n / BS)])
    assert pool.allocated_block_count() == len(used)
    report(f"[worker path] {summary}")


@pytest.mark.timeout(600)
def test_hip_graph_decode_matches_eager():
    """Five rows for ``steps`` steps, then row 2 finishes and four rows decode ``tail`` more steps:
    one graph per (rows, table width), each warming up eagerly, then captured and replayed. Tokens
    and logits equal eager decoding over the same sequence, and every request's batch-1 cache ends
    at its own length."""
    from runtime_amd.phase2.hf_decode import PagedDecoder
    from runtime_amd.phase2.hip_graph_decode import CudaGraphDecodeManager

    model, _, _ = _model(seed=22)
    g = torch.Generator().manual_seed(22)
    # The longest row needs 16 blocks: the persistent cache's table width, which both the eager
    # dense step and the graph (keyed by that width) hand to attention.
    lens = [30, 100, 235, 57, 180]
    prompts = [torch.randint(0, 32768, (n,), generator=g) for n in lens]
    steps, tail = 10, 5
    need = [math.ceil((n + steps + tail + 1) / BS) for n in lens]
    assert max(need) == 16
    rows, at = [], 0
    for n in need:
        rows.append(list(range(at, at + n))[::-1])
        at += n
    runs = {}
    for mode in ("eager", "graph"):
        pool = _pool(at)
        states = [_admit(model, pool, f"r{i}", prompts[i], rows[i]) for i in range(len(lens))]
        mgr = CudaGraphDecodeManager(model=model, device=DEV, warmup_steps=2, enabled=True) if mode == "graph" else None
        dec = PagedDecoder(model, pool, max_active=8, graph_mgr=mgr)
        logits = []
        for _ in range(steps):
            dec.decode_step(states)
            logits.append(dec.last_logits.float().cpu().clone())
        done = states.pop(2)
        dec.release(done.req.request_id)
        for _ in range(tail):
            dec.decode_step(states)
            logits.append(dec.last_logits.float().cpu().clone().view(-1))
        lengths = [s.past_key_values.get_seq_length() for s in states]
        assert lengths == [lens[i] + steps + tail for i in (0, 1, 3, 4)], lengths
        runs[mode] = ([s.generated_token_ids for s in states + [done]], logits, mgr)
    mgr = runs["graph"][2]
    stats = mgr.stats()
    assert not stats["off_reason"], stats
    five, four = stats["graphs"]
    # Two eager warm-up steps each, then one capture + replay and a replay per later step.
    assert (five["rows"], five["width"], four["rows"], four["width"]) == (5, 16, 4, 16), stats
    assert five["state"] == "captured" and five["eager_steps"] == 2 and five["replays"] == steps - 2, stats
    assert four["state"] == "captured" and four["eager_steps"] == 2 and four["replays"] == tail - 2, stats
    assert runs["graph"][0] == runs["eager"][0], "graph replay tokens differ from eager decode"
    diff = max(float((a.view(-1) - b.view(-1)).abs().max()) for a, b in zip(runs["graph"][1], runs["eager"][1]))
    assert diff <= 1e-3, f"graph vs eager logits differ by {diff:.3e}"
    report(f"[hip graph] 5 rows x {steps} steps then 4 rows x {tail}: tokens identical to eager, max |dlogits| "
           f"{diff:.2e}, {five['replays']} + {four['replays']} replays of two captured steps")


def test_hip_graph_manager_keeps_max_graphs_and_declines_when_off():
    """``max_graphs=1``: five rows, then four after one finishes, then three: each row count gets its
    own graph and the older one is dropped (least recently used), tokens equal eager decoding over the
    same sequence. A manager that is not enabled (and not opted in by the environment) declines every
    step, so the decoder runs eagerly and no graph is built."""
    import os

    from runtime_amd.phase2.hf_decode import PagedDecoder
    from runtime_amd.phase2.hip_graph_decode import CudaGraphDecodeManager

    model, _, _ = _model(seed=23)
    g = torch.Generator().manual_seed(23)
    lens = [40, 75, 120, 33, 90]
    prompts = [torch.randint(0, 32768, (n,), generator=g) for n in lens]
    phase = 4
    need = [math.ceil((n + 3 * phase + 1) / BS) for n in lens]
    rows, at = [], 0
    for n in need:
        rows.append(list(range(at, at + n))[::-1])
        at += n
    runs = {}
    for mode in ("eager", "lru", "off"):
        pool = _pool(at)
        states = [_admit(model, pool, f"r{i}", prompts[i], rows[i]) for i in range(len(lens))]
        if mode == "lru":
            mgr = CudaGraphDecodeManager(model=model, device=DEV, warmup_steps=1, enabled=True, max_graphs=1)
        elif mode == "off":
            assert os.environ.get("PHASE2_CUDA_GRAPH", "0").strip() != "1", "the environment opts graphs in"
            mgr = CudaGraphDecodeManager(model=model, device=DEV, warmup_steps=1, enabled=False)
        else:
            mgr = None
        dec = PagedDecoder(model, pool, max_active=8, graph_mgr=mgr)
        seen = []
        for finish in (None, 1, 3):
            if finish is not None:
                done = states.pop(finish)
                dec.release(done.req.request_id)
                seen.append(done.generated_token_ids)
            for _ in range(phase):
                dec.decode_step(states)
            if mode == "lru":
                print(f"[hip graph lru] {len(states)} rows: {mgr.stats()['graphs']}", flush=True)
                graphs = mgr.stats()["graphs"]
                assert len(graphs) == 1 and graphs[0]["rows"] == len(states), graphs
                assert graphs[0]["state"] == "captured" and graphs[0]["replays"] == phase - 1, graphs
        seen += [s.generated_token_ids for s in states]
        runs[mode] = seen
        if mode == "off":
            assert mgr.stats()["graphs"] == [] and not mgr.stats()["enabled"], mgr.stats()
    assert runs["lru"] == runs["eager"], "graph replay tokens differ from eager decode"
    assert runs["off"] == runs["eager"]

def test_kv_write_overrun_raises_at_check():
    """write_tokens_batch queues the write without a host sync; a slot past the table is skipped
    and ``check_write_errors`` raises the reference's IndexError, once; with ``sync_write_checks`` the
    write itself raises, as in the reference."""
    pool = _pool(8)
    table = torch.tensor([[3, 5]], dtype=torch.int32, device=DEV)
    k = torch.randn(1, 2, 4, 64, device=DEV).half()
    pool.write_tokens_batch(0, table, torch.tensor([30], device=DEV), k, k)  # positions 30..33: 32, 33 overrun
    with pytest.raises(IndexError):
        pool.check_write_errors()
    pool.check_write_errors()  # cleared
    assert pool.allocated_block_count() == 1  # block 5 holds positions 30, 31
    torch.testing.assert_close(pool.k_layer_view(0)[5, :, 14:16], k[0, :, :2])
    # Opt-in: the reference's raise at the write itself (one host sync per call).
    pool.sync_write_checks = True
    with pytest.raises(IndexError):
        pool.write_tokens_batch(0, table, torch.tensor([31], device=DEV), k, k)
    pool.write_tokens_batch(0, table, torch.tensor([0], device=DEV), k, k)  # in range: no raise
    assert pool.allocated_block_count() == 2
