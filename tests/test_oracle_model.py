"""Pins of the greedy-decode model oracle (CPU).

The model math is transformers' own; what these tests pin is what the oracle
adds on top: the teacher-forcing window, the weight substitution and the
agreement rule used by the GPU greedy-decode tests.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle.int8_quant import dequantize, quantize_per_channel

TINY = dict(hidden_size=128, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
            intermediate_size=256, vocab_size=512, max_position_embeddings=256)


@pytest.fixture(scope="module")
def tiny_pair():
    model = om.random_qwen2(seed=3, **TINY)
    return model, om.quantized_reference(model)


def test_random_qwen2_is_seeded_and_has_biases():
    a = om.random_qwen2(seed=5, **TINY)
    b = om.random_qwen2(seed=5, **TINY)
    c = om.random_qwen2(seed=6, **TINY)
    for (na, pa), (_, pb), (_, pc) in zip(a.named_parameters(), b.named_parameters(), c.named_parameters()):
        assert torch.equal(pa, pb), na
        assert not torch.equal(pa, pc), na
    bias = a.model.layers[0].self_attn.q_proj.bias
    assert bias is not None and float(bias.detach().abs().max()) > 0


def test_quantized_reference_holds_device_weights(tiny_pair):
    model, ref = tiny_pair
    named = dict(ref.named_parameters())
    for name, p in model.named_parameters():
        r = named[name]
        leaf = name.split(".")[-2]
        if leaf in om.PROJECTIONS and name.endswith("weight"):
            q, s = quantize_per_channel(p.detach().numpy())
            assert torch.equal(r, torch.from_numpy(dequantize(q, s))), name
            # A plausible slip, storing the projection as fp16 instead of q*s, differs.
            assert not torch.equal(r, p.detach().half().float()), name
        else:
            assert torch.equal(r, p.detach().half().float()), name
    # The source model is untouched.
    assert not torch.equal(model.model.layers[0].mlp.down_proj.weight, ref.model.layers[0].mlp.down_proj.weight)


def test_teacher_forcing_equals_stepwise_decode(tiny_pair):
    _, ref = tiny_pair
    prompt = torch.randint(0, TINY["vocab_size"], (37,), generator=torch.Generator().manual_seed(0))
    tokens, logits = om.greedy_reference(ref, prompt, steps=12)
    tf = om.teacher_forced_logits(ref, prompt, tokens)
    assert tf.shape == logits.shape == (13, TINY["vocab_size"])
    torch.testing.assert_close(tf, logits, atol=1e-4, rtol=1e-4)
    assert torch.equal(tf.argmax(dim=-1), tokens)
    # Planted off-by-one: a window shifted by one token no longer matches.
    shifted = om.teacher_forced_logits(ref, prompt[:-1], tokens)
    assert (shifted - logits).abs().max() > 1e-2


def test_greedy_agreement_rule():
    logits = torch.tensor([[0.0, 1.0, 0.5], [2.0, 1.99, 0.0], [0.0, 0.0, 3.0]])
    exact = om.greedy_agreement(logits, torch.tensor([1, 0, 2]), tie_tol=0.05)
    assert exact == {"steps": 3, "mismatches": 0, "first_mismatch": -1, "max_gap_at_mismatch": 0.0, "ties_ok": True}
    tie = om.greedy_agreement(logits, torch.tensor([1, 1, 2]), tie_tol=0.05)
    assert tie["mismatches"] == 1 and tie["first_mismatch"] == 1 and tie["ties_ok"]
    assert abs(tie["max_gap_at_mismatch"] - 0.01) < 1e-6
    wrong = om.greedy_agreement(logits, torch.tensor([2, 0, 2]), tie_tol=0.05)
    assert wrong["first_mismatch"] == 0 and not wrong["ties_ok"]


def test_config3_shape_constants():
    cfg = om.QWEN2_05B
    assert (cfg["hidden_size"], cfg["num_hidden_layers"], cfg["num_attention_heads"], cfg["num_key_value_heads"],
            cfg["intermediate_size"], cfg["vocab_size"]) == (896, 24, 14, 2, 4864, 151936)
    assert cfg["hidden_size"] // cfg["num_attention_heads"] == 64
    assert np.isclose(cfg["rope_theta"], 1e6)


def test_prefix_cache_continuation_equals_full_forward(tiny_pair):
    """Continuing from prefix_cache gives the full forward's teacher-forced logits and prompt K/V; the
    cache itself is not consumed (a second continuation from it agrees too)."""
    _, ref = tiny_pair
    g = torch.Generator().manual_seed(1)
    prefix = torch.randint(0, TINY["vocab_size"], (32,), generator=g)
    past = om.prefix_cache(ref, prefix)
    assert past[1] == 32
    for n_suffix in (1, 9):
        prompt = torch.cat([prefix, torch.randint(0, TINY["vocab_size"], (n_suffix,), generator=g)])
        tokens, _ = om.greedy_reference(ref, prompt, steps=6)
        full = om.teacher_forced_logits(ref, prompt, tokens)
        cont = om.teacher_forced_logits(ref, prompt, tokens, past=past)
        torch.testing.assert_close(cont, full, atol=1e-4, rtol=1e-4)
        kv_full, last_full = om.prefill_kv(ref, prompt)
        kv_cont, last_cont = om.prefill_kv(ref, prompt, past=past)
        torch.testing.assert_close(last_cont, last_full, atol=1e-4, rtol=1e-4)
        for (kf, vf), (kc, vc) in zip(kv_full, kv_cont):
            assert kc.shape == kf.shape == (TINY["num_key_value_heads"], prompt.numel(), 32)
            torch.testing.assert_close(kc, kf, atol=1e-5, rtol=1e-5)
            torch.testing.assert_close(vc, vf, atol=1e-5, rtol=1e-5)
    # A wrong prefix length (the cache continued one token too early) is caught.
    prompt = torch.cat([prefix, torch.randint(0, TINY["vocab_size"], (4,), generator=g)])
    tokens, _ = om.greedy_reference(ref, prompt, steps=3)
    bad = om.teacher_forced_logits(ref, prompt, tokens, past=(past[0], 31))
    assert (bad - om.teacher_forced_logits(ref, prompt, tokens)).abs().max() > 1e-2


def test_margin_controlled_init_pins():
    """margin_controlled_: the greedy successor of token u is perm[u] with a wide margin, on a small
    model whose plain-init margins include near ties; the permutation is seeded."""
    plain = om.random_qwen2(seed=4, **dict(TINY, num_hidden_layers=3, vocab_size=4096))
    sharp = om.random_qwen2(seed=4, **dict(TINY, num_hidden_layers=3, vocab_size=4096))
    perm = om.margin_controlled_(sharp, seed=1)
    assert torch.equal(perm, om.margin_controlled_(om.random_qwen2(seed=4, **dict(TINY, vocab_size=4096)), seed=1))
    prompt = torch.randint(0, 4096, (50,), generator=torch.Generator().manual_seed(2))
    tokens, logits = om.greedy_reference(sharp, prompt, steps=24)
    prev = torch.cat([prompt[-1:], tokens[:-1]])
    assert torch.equal(tokens, perm[prev])
    top2 = logits.topk(2, dim=-1).values
    _, plain_logits = om.greedy_reference(plain, prompt, steps=24)
    plain_top2 = plain_logits.topk(2, dim=-1).values
    assert float((top2[:, 0] - top2[:, 1]).min()) > 10 * float((plain_top2[:, 0] - plain_top2[:, 1]).min())


def test_continue_logits_from_given_kv(tiny_pair):
    """continue_logits over a context's K/V equals teacher forcing over the whole sequence; K/V one
    token short (positions shifted) or from the wrong layers are caught."""
    _, ref = tiny_pair
    g = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, TINY["vocab_size"], (41,), generator=g)
    tokens, _ = om.greedy_reference(ref, prompt, steps=8)
    full = om.teacher_forced_logits(ref, prompt, tokens)
    kv, last = om.prefill_kv(ref, prompt)
    torch.testing.assert_close(last, full[0], atol=1e-4, rtol=1e-4)
    cont = om.continue_logits(ref, kv, tokens[:-1])
    assert cont.shape == (8, TINY["vocab_size"])
    torch.testing.assert_close(cont, full[1:], atol=1e-4, rtol=1e-4)
    short = [(k[:, :-1], v[:, :-1]) for k, v in kv]
    assert (om.continue_logits(ref, short, tokens[:-1]) - full[1:]).abs().max() > 1e-2
    # The layers' K/V handed over in the wrong order (a layer-index slip in a layer-major pool).
    swapped = [kv[1], kv[0]]
    assert (om.continue_logits(ref, swapped, tokens[:-1]) - full[1:]).abs().max() > 1e-2
    # The given tensors are not modified.
    kv2, _ = om.prefill_kv(ref, prompt)
    for (k, v), (k2, v2) in zip(kv, kv2):
        assert torch.equal(k, k2) and torch.equal(v, v2)


def test_parallel_init_is_seeded_and_distributed():
    """random_llama(parallel=True): the same seed gives the same weights, another seed other ones,
    and the draws have the stated distributions (matrices N(0, 0.02), norms 1 + N(0, 0.05))."""
    small = dict(hidden_size=256, num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
                 intermediate_size=512, vocab_size=70000)  # embedding of 17.9 M elements: two streams
    a = om.random_llama(seed=7, parallel=True, **small)
    b = om.random_llama(seed=7, parallel=True, **small)
    c = om.random_llama(seed=8, parallel=True, **small)
    for (name, pa), (_, pb), (_, pc) in zip(a.named_parameters(), b.named_parameters(), c.named_parameters()):
        assert torch.equal(pa, pb), name
        assert not torch.equal(pa, pc), name
    emb = a.model.embed_tokens.weight.detach()
    assert abs(float(emb.std()) - 0.02) < 2e-4 and abs(float(emb.mean())) < 1e-4
    # The two streams of the embedding are independent draws, not one stream repeated.
    flat = emb.reshape(-1)
    assert not torch.equal(flat[:1000], flat[1 << 24:(1 << 24) + 1000])
    norm = a.model.layers[0].input_layernorm.weight.detach()
    assert abs(float(norm.mean()) - 1.0) < 0.02 and abs(float(norm.std()) - 0.05) < 0.01


def test_to_device_dtype_keeps_rotary_frequencies_fp32():
    """A model converted to a 16-bit dtype keeps HF's rotary frequencies in fp32 (as a model loaded in
    that dtype has them): its (cos, sin) at long positions are the fp32 ones rounded once. Converted
    with a plain ``.to(dtype)`` the frequencies round and the angles drift by up to radians."""
    cfg = dict(hidden_size=128, num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
               intermediate_size=256, vocab_size=512, max_position_embeddings=8192)
    ref = om.random_llama(seed=9, **cfg)
    fixed = om.to_device_dtype(copy.deepcopy(ref), "cpu", torch.bfloat16)
    naive = copy.deepcopy(ref).to(dtype=torch.bfloat16)
    rot = fixed.model.rotary_emb
    assert rot.inv_freq.dtype == rot.original_inv_freq.dtype == torch.float32
    assert torch.equal(rot.inv_freq, ref.model.rotary_emb.inv_freq)
    assert naive.model.rotary_emb.inv_freq.dtype == torch.bfloat16
    assert fixed.model.layers[0].mlp.down_proj.weight.dtype == torch.bfloat16
    pos = torch.arange(2000, 4096, 7).view(1, -1)
    x = torch.zeros(1, pos.shape[1], 128)
    with torch.no_grad():
        cos_ref, sin_ref = ref.model.rotary_emb(x, pos)
        cos_f, sin_f = rot(x.to(torch.bfloat16), pos)
        cos_n, sin_n = naive.model.rotary_emb(x.to(torch.bfloat16), pos)
    err_fixed = max(float((cos_f.float() - cos_ref).abs().max()), float((sin_f.float() - sin_ref).abs().max()))
    err_naive = max(float((cos_n.float() - cos_ref).abs().max()), float((sin_n.float() - sin_ref).abs().max()))
    assert err_fixed <= 2.0 ** -8, err_fixed   # one bf16 rounding of a value in [-1, 1]
    assert err_naive > 0.5, err_naive
