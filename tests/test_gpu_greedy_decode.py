"""Greedy decode of a Qwen2-shaped int8 model through HF + the HIP decode path.

Config 3: hidden 896, 24 layers, 14 Q / 2 KV heads (head_dim 64, GQA 7),
SwiGLU 4864, vocab 151936, RoPE theta 1e6, random init (seed 0); batch 16,
prompts of random token ids with lengths uniform in [512, 2048], paged fp16 KV
with block_size 16 and block tables drawn from a shuffled pool, 64 greedy
decode steps after the prefill token.

Device path: ``quantize_model_`` (q/k/v/o/gate/up/down -> Int8Linear on the
HIP GEMV/GEMM), ``block_paged`` attention hook (HIP paged decode), the
``BlockPagedCache`` / ``BlockPagedBatchCache`` adapters, fp16 everything else.

Oracle: the same HF model in fp32 on the CPU holding exactly the device
weights (``oracle.model.quantized_reference``), teacher-forced on the device's
tokens, so every one of the 65 steps of every row is compared on the same
prefix. Yardstick: that weight set in plain torch fp16 on the GPU (eager
attention, dequantized ``nn.Linear``), teacher-forced the same way; its
distance from the oracle is what fp16 activations alone cost on this model.

Checks, per row:

* logits: ``max|L_dev - L_ref| <= max(LOGIT_ATOL, 1.25 * max|L_torch16 - L_ref|)``,
  i.e. the HIP path is within the stated tolerance or no more than 25 % less
  accurate than torch's own fp16 path on identical weights. Both fp16 models keep
  HF's rotary frequencies in fp32 (``oracle.model.to_device_dtype``), as a model
  loaded in fp16 has them; cast with a plain ``.to(float16)`` they round, and that
  alone had put both paths near 2e-2 at these positions. Measured on the MI355X
  per row (24 layers, seed 0): HIP 7.8e-3 .. 1.06e-2, torch fp16 8.3e-3 .. 1.22e-2;
  2 layers: HIP 3.7e-3 .. 4.3e-3, torch fp16 4.2e-3 .. 5.0e-3. Logit std is ~0.6;
* tokens: the device token is the oracle's argmax at every step, except where
  the oracle prefers its argmax over the device token by less than twice the
  allowed logit error (a near tie that fp16 activations break either way;
  torch fp16 breaks as many). With random weights the median gap is ~0.1 and the smallest of ~1000
  steps ~1e-3, so such steps must stay rare: at most 2 % of all steps. Rows
  without one have all 65 greedy tokens identical to the oracle's own greedy
  decode (the count is printed).
"""

from __future__ import annotations

import copy
import math

import pytest
import torch

from conftest import report
from oracle import model as om
from oracle.int8_quant import pack_tiles, quantize_per_channel

pytestmark = pytest.mark.gpu

LOGIT_ATOL = 1e-2
YARDSTICK_SLACK = 1.25
MAX_TIE_FRACTION = 0.02
BLOCK_SIZE = 16
STEPS = 64


def _case(layers: int, batch: int, lo: int, hi: int, seed: int, margin: bool = False):
    from runtime_amd.phase2 import block_paged_attention as bpa
    from runtime_amd.phase2.hf_decode import enable_block_paged_attention, greedy_decode
    from runtime_amd.phase2.int8_linear import Int8Linear, quantize_model_
    from runtime_amd.phase2.paged_attention_hip import workspace_error_flag
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    device = torch.device("cuda:0")
    model = om.random_qwen2(seed=seed, num_hidden_layers=layers)
    if margin:
        om.margin_controlled_(model, seed=seed)
    cfg = model.config
    ref = om.quantized_reference(model)
    torch16 = om.to_device_dtype(copy.deepcopy(ref), device, torch.float16).eval()
    w0 = model.model.layers[0].mlp.down_proj.weight.detach().numpy().copy()
    quantize_model_(model, device=device)
    om.to_device_dtype(model, device, torch.float16)
    enable_block_paged_attention(model)
    assert sum(isinstance(m, Int8Linear) for m in model.modules()) == 7 * layers
    packed0 = model.model.layers[0].mlp.down_proj.packed_weight.cpu().numpy()
    assert (packed0 == pack_tiles(quantize_per_channel(w0)[0])).all()

    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g) for n in lens]
    need = [math.ceil((n + STEPS) / BLOCK_SIZE) for n in lens]
    pool_blocks = 2 * sum(need)
    perm = torch.randperm(pool_blocks, generator=g).tolist()
    rows, at = [], 0
    for n in need:
        rows.append(perm[at:at + n])
        at += n
    pool = GpuKVBlockPool(num_blocks=pool_blocks, block_size_tokens=BLOCK_SIZE, num_layers=layers,
                          num_kv_heads=cfg.num_key_value_heads, head_dim=cfg.hidden_size // cfg.num_attention_heads,
                          dtype=torch.float16, device=device)

    calls = {"n": 0}
    hip_decode = bpa.paged_attention_decode_batched

    def counting(*args, **kwargs):
        calls["n"] += 1
        return hip_decode(*args, **kwargs)

    bpa.paged_attention_decode_batched = counting
    try:
        print(f"[greedy] layers={layers} batch={batch} lens={lo}..{hi} seed={seed}", flush=True)
        tokens, logits = greedy_decode(model, pool, prompts, rows, STEPS, keep_logits=True)
        torch.cuda.synchronize()
    finally:
        bpa.paged_attention_decode_batched = hip_decode
    assert calls["n"] == STEPS * layers, "decode attention did not go through the HIP kernel"
    assert workspace_error_flag(device) == 0
    tokens = tokens.cpu()

    results = []
    for b in range(batch):
        ref_logits = om.teacher_forced_logits(ref, prompts[b], tokens[b])
        ids = torch.cat([prompts[b], tokens[b][:-1]]).view(1, -1).to(device)
        with torch.no_grad():
            t16 = torch16(input_ids=ids, use_cache=False, logits_to_keep=STEPS + 1).logits[0].float().cpu()
        err = float((logits[b].cpu() - ref_logits).abs().max())
        err16 = float((t16 - ref_logits).abs().max())
        allowed = max(LOGIT_ATOL, YARDSTICK_SLACK * err16)
        agree = om.greedy_agreement(ref_logits, tokens[b], tie_tol=2 * allowed)
        top2 = ref_logits.topk(2, dim=-1).values
        agree["min_margin"] = float((top2[:, 0] - top2[:, 1]).min())
        results.append((b, lens[b], err, err16, agree))
        print(f"[greedy] row {b} prompt {lens[b]}: max|dL| hip {err:.3e} torch16 {err16:.3e}, "
              f"mismatches {agree['mismatches']}/{agree['steps']} first {agree['first_mismatch']} "
              f"max gap {agree['max_gap_at_mismatch']:.3e} min oracle margin {agree['min_margin']:.3e}", flush=True)
    return results


def _check(results):
    total = sum(r[4]["steps"] for r in results)
    ties = sum(r[4]["mismatches"] for r in results)
    for b, n, err, err16, agree in results:
        assert err <= max(LOGIT_ATOL, YARDSTICK_SLACK * err16), \
            f"row {b} (prompt {n}): logits off by {err:.3e} (torch fp16: {err16:.3e})"
        assert agree["ties_ok"], f"row {b}: a mismatch outside the near-tie band {agree}"
    identical = sum(r[4]["mismatches"] == 0 for r in results)
    summary = (f"[greedy] {len(results)} rows: {identical} with all {STEPS + 1} tokens identical, {ties} near-tie "
               f"mismatches in {total} steps, largest logit error {max(r[2] for r in results):.3e}, smallest "
               f"oracle top-1 margin {min(r[4]['min_margin'] for r in results):.3e}")
    assert ties <= MAX_TIE_FRACTION * total, summary
    report(summary)


# The margin-controlled case must keep the oracle's top-1 margin at least this many times the
# largest device logit error at every step; then fp16 error cannot flip a token.
MARGIN_MULTIPLE = 10.0


def _check_identical(results):
    """Zero token mismatches: every row's 65 greedy tokens equal the oracle's."""
    steps = sum(r[4]["steps"] for r in results)
    flips = sum(r[4]["mismatches"] for r in results)
    identical = sum(r[4]["mismatches"] == 0 for r in results)
    max_err = max(r[2] for r in results)
    min_margin = min(r[4]["min_margin"] for r in results)
    summary = (f"{identical}/{len(results)} rows with all {STEPS + 1} tokens identical, {flips} mismatches in "
               f"{steps} steps; smallest oracle top-1 margin {min_margin:.3e}, largest logit error {max_err:.3e} "
               f"(ratio {min_margin / max_err:.1f})")
    for b, n, err, err16, agree in results:
        assert err <= max(LOGIT_ATOL, YARDSTICK_SLACK * err16), \
            f"row {b} (prompt {n}): logits off by {err:.3e} (torch fp16: {err16:.3e}); {summary}"
    assert min_margin >= MARGIN_MULTIPLE * max_err, f"margin premise broken: {summary}"
    assert flips == 0, summary
    report(f"[greedy, margin-controlled] {summary}")


def test_greedy_qwen2_two_layers_all_rows():
    _check(_case(layers=2, batch=16, lo=64, hi=256, seed=0))


@pytest.mark.timeout(900)
def test_greedy_qwen2_config3():
    _check(_case(layers=24, batch=16, lo=512, hi=2048, seed=0))


@pytest.mark.timeout(600)
def test_greedy_bf16_model_through_the_hook():
    """An unquantized HF Qwen2 (2 layers, config-3 widths, 32768-token vocabulary) in bf16: the
    block_paged hook, the cache adapters and a bf16 pool (MX_PA_BF16 decode, bf16 K/V append).
    Oracle: the same weights in fp32 on the CPU, teacher-forced on the device's tokens;
    yardstick: torch's own bf16 path (eager attention) on the GPU. Per row, the rules of the
    int8 cases (logits within max(1e-2, 1.25 x torch bf16's error), mismatches only at near
    ties). bf16 logits are ~8x coarser than fp16 ones (~4e-2 here), so near ties are too: the
    aggregate bound is the larger of 2 % of the steps and 2 x (torch bf16's own argmax
    disagreements with the oracle on the same prefixes) + 2, not the fp16 cases' 2 %."""
    from runtime_amd.phase2 import block_paged_attention as bpa
    from runtime_amd.phase2.hf_decode import enable_block_paged_attention, greedy_decode
    from runtime_amd.phase2.paged_attention_hip import workspace_error_flag
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    device = torch.device("cuda:0")
    steps, batch = 16, 6
    model = om.random_qwen2(seed=11, num_hidden_layers=2, vocab_size=32768)
    cfg = model.config
    ref = copy.deepcopy(model).eval()
    yard = om.to_device_dtype(copy.deepcopy(model), device, torch.bfloat16).eval()
    om.to_device_dtype(model, device, torch.bfloat16)
    enable_block_paged_attention(model)
    g = torch.Generator().manual_seed(11)
    lens = torch.randint(40, 160, (batch,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g) for n in lens]
    need = [math.ceil((n + steps) / BLOCK_SIZE) for n in lens]
    perm = torch.randperm(2 * sum(need), generator=g).tolist()
    rows, at = [], 0
    for n in need:
        rows.append(perm[at:at + n])
        at += n
    pool = GpuKVBlockPool(num_blocks=2 * sum(need), block_size_tokens=BLOCK_SIZE, num_layers=2,
                          num_kv_heads=cfg.num_key_value_heads, head_dim=cfg.hidden_size // cfg.num_attention_heads,
                          dtype=torch.bfloat16, device=device)
    calls = {"n": 0}
    hip_decode = bpa.paged_attention_decode_batched

    def counting(*args, **kwargs):
        calls["n"] += 1
        return hip_decode(*args, **kwargs)

    bpa.paged_attention_decode_batched = counting
    try:
        tokens, logits = greedy_decode(model, pool, prompts, rows, steps, keep_logits=True)
        torch.cuda.synchronize()
    finally:
        bpa.paged_attention_decode_batched = hip_decode
    assert calls["n"] == steps * 2, "decode attention did not go through the HIP kernel"
    assert workspace_error_flag(device) == 0
    tokens = tokens.cpu()
    results = []
    for b in range(batch):
        ref_logits = om.teacher_forced_logits(ref, prompts[b], tokens[b])
        ids = torch.cat([prompts[b], tokens[b][:-1]]).view(1, -1).to(device)
        with torch.no_grad():
            tb = yard(input_ids=ids, use_cache=False, logits_to_keep=steps + 1).logits[0].float().cpu()
        err = float((logits[b].float().cpu() - ref_logits).abs().max())
        errb = float((tb - ref_logits).abs().max())
        allowed = max(LOGIT_ATOL, YARDSTICK_SLACK * errb)
        agree = om.greedy_agreement(ref_logits, tokens[b], tie_tol=2 * allowed)
        yard_miss = int((tb.argmax(dim=-1) != ref_logits.argmax(dim=-1)).sum())
        print(f"[bf16] row {b} prompt {lens[b]}: max|dL| hip {err:.3e} torch bf16 {errb:.3e}, "
              f"mismatches {agree['mismatches']}/{agree['steps']} (torch bf16 {yard_miss})", flush=True)
        assert err <= allowed, f"row {b}: logits off by {err:.3e} (torch bf16: {errb:.3e})"
        assert agree["ties_ok"], f"row {b}: a mismatch outside the near-tie band {agree}"
        results.append((agree["mismatches"], agree["steps"], yard_miss))
    ties, total, yard = (sum(r[i] for r in results) for i in range(3))
    assert ties <= max(MAX_TIE_FRACTION * total, 2 * yard + 2), f"{ties} near ties in {total} steps (torch bf16 {yard})"


@pytest.mark.timeout(900)
def test_greedy_qwen2_config3_margin_controlled_identical_tokens():
    """Config 3 (24 layers, batch 16, prompts U[512, 2048], 64 greedy steps) with the
    margin-controlled init (oracle.model.margin_controlled_: embedding scaled 200x, a successor
    term of 0.2 in lm_head): the north star's bar, greedy tokens identical to the oracle's at
    every step of every row, with the oracle's top-1 margin at least MARGIN_MULTIPLE times the
    largest logit error, both measured in the run and printed. The plain-init case above keeps
    the tolerance rule, because there near ties below fp16 error occur."""
    _check_identical(_case(layers=24, batch=16, lo=512, hi=2048, seed=0, margin=True))
