"""Shared-prefix (aliased) block tables and join/finish on the GPU path.

* Alias safety of the attention kernel: rows whose tables alias their group's prefix
  blocks give bit-identical output to the same rows with the prefix copied into private
  blocks (the reference's copy-on-hit, ``runtime/phase2/worker_server.py:1372-1375``),
  under either K/V cache policy, and match the fp32 oracle within atol/rtol 1e-2.
* The native decode step over a :class:`PrefixBatch`: rows of a group share a prompt
  prefix and its K/V blocks; half-way through, two requests finish and two new ones join
  their slots (freed blocks reused, tables and lengths rewritten in place while the step
  keeps replaying one captured HIP graph). Every request's logits and greedy tokens are
  compared with the fp32 HF oracle teacher-forced on its own tokens, with the rules of the
  native-step test (``max|dL| <= max(1e-2, 1.25 * torch-fp16 error)``, mismatches only at
  near ties).
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from conftest import report
from oracle import model as om
from oracle import paged_attention as oracle_pa

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
BS = 16


def test_aliased_prefix_blocks_equal_copied_blocks():
    from runtime_amd.phase2.paged_attention_hip import _decode
    from runtime_amd.phase2.prefix_batch import PrefixBatch

    hkv, grp, d = 4, 4, 128
    pb = PrefixBatch(batch=16, groups=2, prefix_tokens=256, lo=200, hi=900, block_size=BS, num_blocks=1400,
                     headroom=1, seed=3)
    assert sum(r.shared > 0 for r in pb.rows) >= 12
    g = torch.Generator(device=DEV).manual_seed(4)
    nb = 1400
    k = torch.randn(nb, hkv, BS, d, generator=g, device=DEV).half()
    v = torch.randn(nb, hkv, BS, d, generator=g, device=DEV).half()
    q = torch.randn(16, hkv * grp, 1, d, generator=g, device=DEV).half()
    tables = pb.tables
    lens = pb.lens + 1
    # Copy: every sharing row gets private copies of its group's prefix blocks.
    copied = tables.clone()
    spare = [i for i in range(nb) if pb.alloc.refcount(i) == 0]
    for b, r in enumerate(pb.rows):
        for j in range(r.shared):
            dst = spare.pop()
            k[dst] = k[r.blocks[j]]
            v[dst] = v[r.blocks[j]]
            copied[b, j] = dst
    scale = d**-0.5
    out_alias = _decode(q, k, v, tables.to(DEV), lens.to(DEV), scale, grp, shared_blocks=True)
    out_copy = _decode(q, k, v, copied.to(DEV), lens.to(DEV), scale, grp)
    assert torch.equal(out_alias, out_copy)
    # The streaming cache policy reads the aliased blocks to the same result.
    assert torch.equal(_decode(q, k, v, tables.to(DEV), lens.to(DEV), scale, grp), out_alias)
    want = oracle_pa.decode_rows_fp32(q.cpu(), k.cpu(), v.cpu(), tables, lens.tolist(), scale, grp)
    np.testing.assert_allclose(out_alias.float().cpu().numpy(), want.numpy(), atol=1e-2, rtol=1e-2)


LOGIT_ATOL = 1e-2
YARDSTICK_SLACK = 1.25
MAX_TIE_FRACTION = 0.02
STEPS = 16
JOIN_AT = 8


@pytest.mark.timeout(600)
def test_native_step_shared_prefix_join_finish():
    from runtime_amd.phase2.decode_glue import kv_append
    from runtime_amd.phase2.decode_step import Int8DecodeModel
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool
    from runtime_amd.phase2.prefix_batch import PrefixBatch

    hf = om.random_llama(seed=5, num_hidden_layers=2, vocab_size=32768)
    cfg = hf.config
    ref = om.quantized_reference(hf, targets=om.PROJECTIONS + ("lm_head",))
    torch16 = om.to_device_dtype(copy.deepcopy(ref), DEV, torch.float16).eval()
    native = Int8DecodeModel.from_hf(hf, device=DEV, max_positions=1024)
    native.shared_kv_blocks = True
    s = native.shape
    batch, groups, prefix = 16, 2, 64
    g = torch.Generator().manual_seed(6)
    group_prefix = [torch.randint(0, cfg.vocab_size, (prefix,), generator=g) for _ in range(groups)]

    def prompt_for(group: int, length: int) -> torch.Tensor:
        if length <= prefix:  # too short to share: its own tokens
            return torch.randint(0, cfg.vocab_size, (length,), generator=g)
        return torch.cat([group_prefix[group], torch.randint(0, cfg.vocab_size, (length - prefix,), generator=g)])

    lengths = [int(x) for x in torch.randint(40, 160, (batch,), generator=g)]
    lengths[0] = 50  # one row that does not share
    pb = PrefixBatch(batch=batch, groups=groups, prefix_tokens=prefix, lo=40, hi=160, block_size=BS,
                     num_blocks=600, headroom=STEPS + 1, seed=7, lengths=lengths)
    pool = GpuKVBlockPool(num_blocks=600, block_size_tokens=BS, num_layers=s.layers, num_kv_heads=s.kv_heads,
                          head_dim=s.head_dim, dtype=torch.float16, device=DEV)
    pool._ensure_pools()
    tables_d = torch.zeros(batch, pb.max_blocks, dtype=torch.int32, device=DEV)
    seq_lens = torch.zeros(batch, dtype=torch.int32, device=DEV)
    tokens = torch.zeros(batch, dtype=torch.int64, device=DEV)

    def admit(rows: list[int]) -> list[dict]:
        """Prefill the requests now in ``rows`` with the oracle and write their K/V into the pool."""
        reqs = []
        tbl = pb.tables.to(DEV)
        for b in rows:
            r = pb.rows[b]
            prompt = prompt_for(r.group, r.length)
            kv, logits = om.prefill_kv(ref, prompt)
            for li, (kk, vv) in enumerate(kv):
                kv_append(pool.k_layer_view(li), pool.v_layer_view(li), tbl[b:b + 1],
                          torch.zeros(1, dtype=torch.int32, device=DEV), kk.unsqueeze(0).half().to(DEV),
                          vv.unsqueeze(0).half().to(DEV))
            reqs.append(dict(slot=b, prompt=prompt, first=int(logits.argmax()), tokens=[], logits=[]))
        return reqs

    live = admit(list(range(batch)))
    pb.upload(tables_d, seq_lens)
    tokens.copy_(torch.tensor([q["first"] for q in live]))
    done = []
    step_graph = None
    print(f"[prefix] rows {batch}, groups {groups}, prefix {prefix}, lengths {lengths}", flush=True)
    for k in range(STEPS):
        if k == JOIN_AT:  # two requests finish, two join their slots
            finishing = [live[3], live[12]]
            done += finishing
            pb.rotate([3, 12], lengths=[130, 30])
            new = admit([3, 12])
            live[3], live[12] = new
            pb.upload(tables_d, seq_lens)
            tokens[3] = new[0]["first"]
            tokens[12] = new[1]["first"]
        if k == 1:
            step_graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(step_graph):
                nxt_g, logits_g = native.step(tokens, pool, tables_d, seq_lens, return_logits=True)
        if step_graph is not None:
            step_graph.replay()
            nxt, logits = nxt_g, logits_g
        else:
            nxt, logits = native.step(tokens, pool, tables_d, seq_lens, return_logits=True)
        nxt_h, logits_h = nxt.cpu(), logits.float().cpu()
        for q in live:
            q["tokens"].append(int(nxt_h[q["slot"]]))
            q["logits"].append(logits_h[q["slot"]])
        tokens.copy_(nxt)
        pb.advance(1)
    assert native.error_flag() == 0
    assert seq_lens.cpu().tolist() == pb.lens.tolist()

    results, ties, steps = [], 0, 0
    for q in done + live:
        gen = torch.tensor([q["first"]] + q["tokens"])
        n = len(q["tokens"])
        ref_logits = om.teacher_forced_logits(ref, q["prompt"], gen)[1:]
        ids = torch.cat([q["prompt"], gen[:-1]]).view(1, -1).to(DEV)
        with torch.no_grad():
            t16 = torch16(input_ids=ids, use_cache=False, logits_to_keep=n + 1).logits[0, 1:].float().cpu()
        mine = torch.stack(q["logits"])
        err = float((mine - ref_logits).abs().max())
        err16 = float((t16 - ref_logits).abs().max())
        allowed = max(LOGIT_ATOL, YARDSTICK_SLACK * err16)
        agree = om.greedy_agreement(ref_logits, torch.tensor(q["tokens"]), tie_tol=2 * allowed)
        print(f"[prefix] slot {q['slot']} prompt {len(q['prompt'])} steps {n}: native {err:.3e} "
              f"torch16 {err16:.3e} mismatches {agree['mismatches']}", flush=True)
        results.append((q["slot"], err, allowed, agree))
        ties += agree["mismatches"]
        steps += n
    for slot, err, allowed, agree in results:
        assert err <= allowed, f"slot {slot}: logits off by {err:.3e} (allowed {allowed:.3e})"
        assert agree["ties_ok"], f"slot {slot}: mismatch outside the near-tie band {agree}"
    assert ties <= MAX_TIE_FRACTION * steps


C5_ROWS, C5_GROUPS, C5_PREFIX = 128, 16, 1024


@pytest.mark.timeout(900)
def test_native_step_config5_rows_join_finish():
    """Config 5's batch on the native step (Llama-3-8B dims, 2 layers, 32768-token vocabulary):
    128 rows in 16 groups of 8. In every group six rows hold the group's 1024-token prefix in
    aliased blocks plus a private suffix (contexts 1025..1400), and two rows are shorter than
    the prefix and own all their blocks (contexts 1..1024). At step 8 the 16 rows b with
    b % 8 == 0 finish and 16 new requests of the same groups join their slots (freed blocks
    reused, tables and lengths rewritten in place while one captured HIP graph keeps
    replaying). Every request is teacher-forced against the fp32 oracle (the prefix run once
    per group, om.prefix_cache) with the rules of the other native-step tests."""
    from runtime_amd.phase2.decode_glue import kv_append
    from runtime_amd.phase2.decode_step import Int8DecodeModel
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool
    from runtime_amd.phase2.prefix_batch import PrefixBatch

    hf = om.random_llama(seed=9, num_hidden_layers=2, vocab_size=32768)
    cfg = hf.config
    ref = om.quantized_reference(hf, targets=om.PROJECTIONS + ("lm_head",))
    torch16 = om.to_device_dtype(copy.deepcopy(ref), DEV, torch.float16).eval()
    native = Int8DecodeModel.from_hf(hf, device=DEV, max_positions=2048)
    native.shared_kv_blocks = True
    s = native.shape
    g = torch.Generator().manual_seed(10)
    group_prefix = [torch.randint(0, cfg.vocab_size, (C5_PREFIX,), generator=g) for _ in range(C5_GROUPS)]
    past = [om.prefix_cache(ref, p) for p in group_prefix]

    def draw_length(slot: int) -> int:
        if slot % 8 in (3, 7):  # shorter than the prefix: own blocks only
            return int(torch.randint(1, C5_PREFIX + 1, (1,), generator=g))
        return int(torch.randint(C5_PREFIX + 1, 1401, (1,), generator=g))

    lengths = [draw_length(b) for b in range(C5_ROWS)]
    num_blocks = 16384
    pb = PrefixBatch(batch=C5_ROWS, groups=C5_GROUPS, prefix_tokens=C5_PREFIX, lo=1, hi=1400, block_size=BS,
                     num_blocks=num_blocks, headroom=STEPS + 1, seed=11, lengths=lengths)
    assert sum(r.shared > 0 for r in pb.rows) == 96
    pool = GpuKVBlockPool(num_blocks=num_blocks, block_size_tokens=BS, num_layers=s.layers, num_kv_heads=s.kv_heads,
                          head_dim=s.head_dim, dtype=torch.float16, device=DEV)
    pool._ensure_pools()
    tables_d = torch.zeros(C5_ROWS, pb.max_blocks, dtype=torch.int32, device=DEV)
    seq_lens = torch.zeros(C5_ROWS, dtype=torch.int32, device=DEV)
    tokens = torch.zeros(C5_ROWS, dtype=torch.int64, device=DEV)

    def admit(rows: list[int]) -> list[dict]:
        """Prefill the requests now in ``rows`` with the oracle and write their K/V into the pool."""
        reqs = []
        tbl = pb.tables.to(DEV)
        for b in rows:
            r = pb.rows[b]
            if r.shared:
                prompt = torch.cat([group_prefix[r.group],
                                    torch.randint(0, cfg.vocab_size, (r.length - C5_PREFIX,), generator=g)])
                pre = past[r.group]
            else:
                prompt, pre = torch.randint(0, cfg.vocab_size, (r.length,), generator=g), None
            kv, logits = om.prefill_kv(ref, prompt, past=pre)
            for li, (kk, vv) in enumerate(kv):
                kv_append(pool.k_layer_view(li), pool.v_layer_view(li), tbl[b:b + 1],
                          torch.zeros(1, dtype=torch.int32, device=DEV), kk.unsqueeze(0).half().to(DEV),
                          vv.unsqueeze(0).half().to(DEV))
            reqs.append(dict(slot=b, prompt=prompt, past=pre, first=int(logits.argmax()), tokens=[], logits=[]))
        return reqs

    live = admit(list(range(C5_ROWS)))
    pb.upload(tables_d, seq_lens)
    tokens.copy_(torch.tensor([q["first"] for q in live]))
    done = []
    step_graph = None
    finish = [b for b in range(C5_ROWS) if b % 8 == 0]
    print(f"[config5] rows {C5_ROWS}, groups {C5_GROUPS}, prefix {C5_PREFIX}, sharing "
          f"{sum(r.shared > 0 for r in pb.rows)}, unique K/V tokens {pb.unique_tokens()} of "
          f"{pb.logical_tokens()}", flush=True)
    for k in range(STEPS):
        if k == JOIN_AT:  # 16 requests finish, 16 join their slots
            done += [live[b] for b in finish]
            pb.rotate(finish, lengths=[draw_length(b) for b in finish])
            for q in admit(finish):
                live[q["slot"]] = q
            pb.upload_rows(finish, tables_d, seq_lens)
            for b in finish:
                tokens[b] = live[b]["first"]
        if k == 1:
            step_graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(step_graph):
                nxt_g, logits_g = native.step(tokens, pool, tables_d, seq_lens, return_logits=True)
        if step_graph is not None:
            step_graph.replay()
            nxt, logits = nxt_g, logits_g
        else:
            nxt, logits = native.step(tokens, pool, tables_d, seq_lens, return_logits=True)
        nxt_h, logits_h = nxt.cpu(), logits.float().cpu()
        for q in live:
            q["tokens"].append(int(nxt_h[q["slot"]]))
            q["logits"].append(logits_h[q["slot"]])
        tokens.copy_(nxt)
        pb.advance(1)
    assert native.error_flag() == 0
    assert seq_lens.cpu().tolist() == pb.lens.tolist()

    results, ties, steps, identical = [], 0, 0, 0
    for q in done + live:
        gen = torch.tensor([q["first"]] + q["tokens"])
        n = len(q["tokens"])
        ref_logits = om.teacher_forced_logits(ref, q["prompt"], gen, past=q["past"])[1:]
        ids = torch.cat([q["prompt"], gen[:-1]]).view(1, -1).to(DEV)
        with torch.no_grad():
            t16 = torch16(input_ids=ids, use_cache=False, logits_to_keep=n + 1).logits[0, 1:].float().cpu()
        mine = torch.stack(q["logits"])
        err = float((mine - ref_logits).abs().max())
        err16 = float((t16 - ref_logits).abs().max())
        allowed = max(LOGIT_ATOL, YARDSTICK_SLACK * err16)
        agree = om.greedy_agreement(ref_logits, torch.tensor(q["tokens"]), tie_tol=2 * allowed)
        results.append((q["slot"], len(q["prompt"]), err, allowed, agree))
        ties += agree["mismatches"]
        steps += n
        identical += agree["mismatches"] == 0
    worst = max(results, key=lambda r: r[2] / r[3])
    summary = (f"{len(results)} requests, {steps} steps: {identical} with every token identical, {ties} near-tie "
               f"mismatches; worst logit error {worst[2]:.3e} (allowed {worst[3]:.3e}, slot {worst[0]}, prompt "
               f"{worst[1]})")
    for slot, plen, err, allowed, agree in results:
        assert err <= allowed, f"slot {slot} (prompt {plen}): logits off by {err:.3e} (allowed {allowed:.3e}); {summary}"
        assert agree["ties_ok"], f"slot {slot}: mismatch outside the near-tie band {agree}; {summary}"
    assert ties <= MAX_TIE_FRACTION * steps, summary
    report(f"[config5 native step] {summary}")
