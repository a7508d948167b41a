"""Seeded randomized parity sweep of the native decode step (``Int8DecodeModel.step``).

Each case draws a small decoder and a batch from a fixed seed, so a failure names a reproducible
case: Qwen2 (qkv biases) or Llama (none), head_dim 64 or 128, 1-4 kv-heads with GQA groups 1-16
(above 8 the attention splits a pool head into virtual heads), 1-3 layers, SwiGLU widths
512-1536, a 4096- or 8192-token vocabulary, RoPE theta 1e4 or 1e6; 1-100 rows (the VALU GEMV at
<= 4 rows, the MFMA kernel's one- to four-m-tile shapes, the fused qkv + RoPE launch up to 32 rows
and the two-launch path above, the M-split shape past 48), pool block size 8, 16 or 32 (the tile
plan at >= 16), prompts of 1-300 tokens, eager steps or a captured step graph.

Oracle and rules as in ``test_gpu_decode_step.py``: the fp32 HF model with the device's weights
(``oracle.model.quantized_reference``) computes each prompt's K/V, which the pool receives in
fp16; after the native steps it continues from those K/V over the native tokens
(``oracle.model.continue_logits``). Per row ``max|dL| <= max(1e-2, 1.25 x torch fp16's error)``
(torch fp16 continuing from the same K/V on the GPU), mismatching tokens only at near ties, at
most 2 % of all steps or as many as torch fp16 makes plus one.
"""

from __future__ import annotations

import copy
import math

import numpy as np
import pytest
import torch

from oracle import glue as og
from oracle import model as om

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
LOGIT_ATOL = 1e-2
YARDSTICK_SLACK = 1.25
MAX_TIE_FRACTION = 0.02
STEPS = 6
BATCHES = [1, 2, 4, 5, 16, 17, 32, 33, 48, 64, 100]


def _case(seed: int) -> dict:
    rng = np.random.default_rng(9000 + seed)
    d = int(rng.choice([64, 128]))
    hkv = int(rng.choice([1, 2, 4]))
    grp = int(rng.choice([g for g in (1, 2, 3, 4, 7, 8, 16) if hkv * g * d <= 2048]))
    return dict(
        arch=str(rng.choice(["qwen2", "llama"])), d=d, hkv=hkv, grp=grp, heads=hkv * grp,
        layers=int(rng.integers(1, 4)), inter=int(rng.choice([512, 1024, 1536])),
        vocab=int(rng.choice([4096, 8192])), theta=float(rng.choice([1e4, 1e6])),
        batch=BATCHES[seed % len(BATCHES)], bs=int(rng.choice([8, 16, 16, 32])),
        hi=int(rng.integers(20, 301)), graph=bool(rng.random() < 0.6), seed=seed)


def _model(c: dict):
    kw = dict(hidden_size=c["heads"] * c["d"], num_hidden_layers=c["layers"], num_attention_heads=c["heads"],
              num_key_value_heads=c["hkv"], intermediate_size=c["inter"], vocab_size=c["vocab"],
              max_position_embeddings=1024)
    if c["arch"] == "qwen2":
        return om.random_qwen2(seed=c["seed"], rope_theta=c["theta"], **kw)
    return om.random_llama(seed=c["seed"], rope_theta=c["theta"], head_dim=c["d"], **kw)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("seed", range(40))
def test_native_step_random_case(seed):
    from runtime_amd.phase2.decode_step import Int8DecodeModel
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    c = _case(seed)
    print(f"[random step] {c}", flush=True)
    hf = _model(c)
    ref = om.quantized_reference(hf, targets=om.PROJECTIONS + ("lm_head",))
    torch16 = om.to_device_dtype(copy.deepcopy(ref), DEV, torch.float16).eval()
    native = Int8DecodeModel.from_hf(hf, device=DEV, max_positions=1024)
    s = native.shape
    assert (s.head_dim, s.kv_heads, s.group, s.qkv_bias) == (c["d"], c["hkv"], c["grp"], c["arch"] == "qwen2")
    bs, batch = c["bs"], c["batch"]
    g = torch.Generator().manual_seed(c["seed"])
    lens = torch.randint(1, c["hi"] + 1, (batch,), generator=g).tolist()
    prompts = [torch.randint(0, c["vocab"], (n,), generator=g) for n in lens]
    need = [math.ceil((n + STEPS + 1) / bs) for n in lens]
    nb = sum(need) + 5
    perm = torch.randperm(nb, generator=g)
    tables = torch.zeros(batch, max(need), dtype=torch.int32)
    at = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[at:at + n].to(torch.int32)
        at += n
    pool_k = torch.zeros(nb, s.layers, s.kv_heads, bs, s.head_dim, dtype=torch.float16)
    pool_v = torch.zeros_like(pool_k)
    kv_rows, first = [], []
    for b, prompt in enumerate(prompts):
        kv, last = om.prefill_kv(ref, prompt)
        first.append(int(last.argmax()))
        kv16 = [(k.half(), v.half()) for k, v in kv]
        kv_rows.append([(k.float(), v.float()) for k, v in kv16])
        for li, (k, v) in enumerate(kv16):
            assert og.append_tokens(pool_k[:, li], pool_v[:, li], tables[b:b + 1], [0], k.unsqueeze(0),
                                    v.unsqueeze(0)) == []
    pool = GpuKVBlockPool(num_blocks=nb, block_size_tokens=bs, num_layers=s.layers, num_kv_heads=s.kv_heads,
                          head_dim=s.head_dim, dtype=torch.float16, device=DEV)
    pool._ensure_pools()
    for li in range(s.layers):
        pool.k_layer_view(li).copy_(pool_k[:, li])
        pool.v_layer_view(li).copy_(pool_v[:, li])
    tables_d = tables.to(DEV)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    tokens = torch.tensor(first, dtype=torch.int64, device=DEV)
    inputs, outputs, logits = [tokens.cpu()], [], []
    graph = None
    for k in range(STEPS):
        if c["graph"] and k == 1:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                _, logits_g = native.step(tokens, pool, tables_d, seq_lens, return_logits=True, out=tokens)
        if graph is not None:
            graph.replay()
            step_logits = logits_g
        else:
            _, step_logits = native.step(tokens, pool, tables_d, seq_lens, return_logits=True, out=tokens)
        logits.append(step_logits.float().cpu())
        outputs.append(tokens.cpu())
        inputs.append(tokens.cpu())
    assert native.error_flag() == 0
    assert seq_lens.cpu().tolist() == [n + STEPS for n in lens]
    inputs = torch.stack(inputs[:-1], dim=1)
    outputs = torch.stack(outputs, dim=1)
    logits = torch.stack(logits, dim=1)
    flips = yard = 0
    worst = 0.0
    for b in range(batch):
        ref_logits = om.continue_logits(ref, kv_rows[b], inputs[b])
        t16 = om.continue_logits(torch16, kv_rows[b], inputs[b])
        err = float((logits[b] - ref_logits).abs().max())
        err16 = float((t16 - ref_logits).abs().max())
        allowed = max(LOGIT_ATOL, YARDSTICK_SLACK * err16)
        agree = om.greedy_agreement(ref_logits, outputs[b], tie_tol=2 * allowed)
        assert err <= allowed, f"{c}: row {b} logits off by {err:.3e} (allowed {allowed:.3e})"
        assert agree["ties_ok"], f"{c}: row {b} mismatch outside the near-tie band {agree}"
        flips += agree["mismatches"]
        yard += int((t16.argmax(dim=-1) != ref_logits.argmax(dim=-1)).sum())
        worst = max(worst, err)
    assert flips <= max(MAX_TIE_FRACTION * batch * STEPS, yard + 1), f"{c}: {flips} near-tie flips (torch16 {yard})"
    print(f"[random step] seed {seed}: worst logit error {worst:.3e}, {flips} flips (torch16 {yard})", flush=True)
