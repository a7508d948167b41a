"""fp32 CPU oracle for greedy decode of an HF decoder with int8 projections.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

What it restates: the greedy decode loop of ``TransformersBackend``
(``runtime/phase2/worker_server.py:733-794``: one token per row per step,
``argmax`` over the last logits, ``:786``) on a model whose quantized-linear
slot (``:194-205``) holds the build's int8 format. The model math itself is the
transformers library's Qwen2 / Llama modelling code (third-party: 5.15.0
installed, the reference pins 5.8.1 in ``runtime/requirements-transformers.txt:4``),
run in fp32 on the CPU with eager attention.

Weights are made identical to the device model's:

* every projection the device path quantizes (``q/k/v/o/gate/up/down_proj``)
  becomes ``q * s`` from :func:`oracle.int8_quant.quantize_per_channel`, which
  is bit-exact with the device quantizer;
* every other parameter (embeddings, norms, biases, ``lm_head``) is rounded
  through fp16, the dtype the device model stores it in.

What remains different is activation precision only (fp16 on the device,
fp32 here), which is what the greedy-decode tolerance covers.

Teacher forcing: :func:`teacher_forced_logits` runs one causal forward over
``prompt + generated[:-1]`` and returns the logits every generated token was
chosen from. If the device's tokens are the argmax of these logits at every
step, the oracle's own free-running greedy decode produces the same tokens.

Parity pins (``tests/test_oracle_model.py``): teacher-forced logits equal a
step-by-step ``DynamicCache`` decode of the same model (an off-by-one in the
window fails it); continuing from a :func:`prefix_cache` gives the logits and
keys/values of the full forward; projection weights equal
``dequantize(quantize_per_channel(W))`` exactly; a planted fp16 rounding of a
projection weight is detected.
"""

from __future__ import annotations

import copy
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch
from torch import nn

from .int8_quant import dequantize, quantize_per_channel

PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

# Config 3: Qwen2-0.5B-shaped decoder (hidden 896, 24 layers, 14 Q / 2 KV heads,
# head_dim 64, SwiGLU 4864, vocab 151936, RMSNorm, RoPE theta 1e6).
QWEN2_05B = dict(hidden_size=896, num_hidden_layers=24, num_attention_heads=14, num_key_value_heads=2,
                 intermediate_size=4864, vocab_size=151936, rope_theta=1000000.0, rms_norm_eps=1e-6,
                 max_position_embeddings=32768, tie_word_embeddings=False)


# Llama-3-8B-shaped decoder (the headline bench shape): 32 layers, hidden 4096,
# 32 Q / 8 KV heads, head_dim 128, SwiGLU 14336, vocab 128256, theta 5e5, no biases.
LLAMA3_8B = dict(hidden_size=4096, num_hidden_layers=32, num_attention_heads=32, num_key_value_heads=8,
                 intermediate_size=14336, vocab_size=128256, rope_theta=500000.0, rms_norm_eps=1e-5,
                 max_position_embeddings=32768, tie_word_embeddings=False)


def random_qwen2(seed: int = 0, **overrides):
    """A random-init ``Qwen2ForCausalLM`` in fp32 on the CPU (eager attention).

    Weights come from one numpy PCG64 stream in parameter order: matrices and
    embeddings ~ N(0, 0.02), biases ~ N(0, 0.02), norm weights ~ 1 + N(0, 0.05).
    (HF's own initializer is not used: it takes minutes at this size and zeroes
    the biases, which would leave the bias path untested.)
    """
    from transformers import Qwen2Config, Qwen2ForCausalLM

    kwargs = dict(QWEN2_05B)
    kwargs.update(overrides)
    return _random_model(Qwen2ForCausalLM, Qwen2Config(**kwargs), seed)


def random_llama(seed: int = 0, parallel: bool = False, **overrides):
    """A random-init ``LlamaForCausalLM`` (Llama-3-8B shape unless overridden), as :func:`random_qwen2`.

    ``parallel`` draws the weights from independent seeded streams on several threads (same
    distributions, other values): the Llama-3-8B widths hold ~2 G parameters at 4 layers, a minute
    of single-stream sampling.
    """
    from transformers import LlamaConfig, LlamaForCausalLM

    kwargs = dict(LLAMA3_8B)
    kwargs.update(overrides)
    return _random_model(LlamaForCausalLM, LlamaConfig(**kwargs), seed, parallel=parallel)


_CHUNK = 1 << 24  # elements per independent stream in the parallel fills


def _workers() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else 1))


def _normal_parallel(shape, seq: np.random.SeedSequence, pool) -> np.ndarray:
    """N(0, 1) float32 of ``shape`` from ``ceil(numel / _CHUNK)`` child streams of ``seq``, filled by ``pool``."""
    out = np.empty(int(np.prod(shape)), np.float32)
    n_chunks = max(1, -(-out.size // _CHUNK))
    seqs = seq.spawn(n_chunks)

    def fill(i):
        np.random.Generator(np.random.PCG64(seqs[i])).standard_normal(
            out=out[i * _CHUNK:(i + 1) * _CHUNK], dtype=np.float32)

    list(pool.map(fill, range(n_chunks)))
    return out.reshape(shape)


def _random_model(model_cls, config, seed: int, parallel: bool = False):
    from transformers.initialization import no_init_weights

    config._attn_implementation = "eager"
    with no_init_weights():
        model = model_cls(config)
    rng = np.random.default_rng(seed)
    params = list(model.named_parameters())
    seqs = np.random.SeedSequence(seed).spawn(len(params))
    with torch.no_grad(), ThreadPoolExecutor(_workers()) as pool:
        for (name, p), seq in zip(params, seqs):
            if parallel:
                noise = _normal_parallel(tuple(p.shape), seq, pool)
            else:
                noise = rng.standard_normal(p.shape, dtype=np.float32)
            if name.endswith("norm.weight"):
                p.copy_(torch.from_numpy(1.0 + 0.05 * noise))
            else:
                p.copy_(torch.from_numpy(0.02 * noise))
    return model.float().eval()


# Buffers of HF's rotary embedding that ``nn.Module.to(dtype)`` would cast along with the weights.
_ROPE_BUFFERS = ("inv_freq", "original_inv_freq")


def to_device_dtype(model: nn.Module, device, dtype: torch.dtype) -> nn.Module:
    """``model.to(device=device, dtype=dtype)`` with the rotary frequencies kept in fp32 (in place).

    ``Module.to(dtype)`` casts every floating buffer, HF's ``inv_freq`` included. In fp16 the
    frequencies carry a relative error of up to 2^-11, so the rotary angle ``pos * inv_freq`` is
    off by ~1 rad at position 2000 for the fastest frequency: an error of the conversion, not of
    fp16 arithmetic. A model loaded with ``from_pretrained(torch_dtype=fp16)`` (as the reference's
    worker loads it, ``worker_server.py:176-186``) computes ``inv_freq`` in fp32 and keeps it; this
    restores that for a model built in fp32 and converted afterwards. Used for the fp16/bf16
    yardsticks and the HF device models of the GPU tests.
    """
    saved = {(mod_name, b): buf.detach().clone() for mod_name, mod in model.named_modules()
             for b, buf in mod.named_buffers(recurse=False) if b in _ROPE_BUFFERS}
    model.to(device=device, dtype=dtype)
    modules = dict(model.named_modules())
    for (mod_name, b), buf in saved.items():
        setattr(modules[mod_name], b, buf.to(device=device, dtype=torch.float32))
    return model


def margin_controlled_(model: nn.Module, embed_scale: float = 200.0, successor: float = 0.2, seed: int = 0
                       ) -> torch.Tensor:
    """Give a random-init model a greedy top-1 margin far above fp16 activation error (in place).

    With N(0, 0.02) weights the logits over a 151936-token vocabulary are near-Gaussian, so over
    a thousand greedy steps the gap between the two best tokens falls below the ~1e-2 logit error
    of fp16 activations somewhere, and no decode in fp16 can promise identical tokens. Here:

    * the token embedding is scaled by ``embed_scale`` (std 0.02 -> 4), so the current token
      dominates the residual stream over the layers' outputs (the layers still move every logit,
      attention included; their RMSNorm inputs are normalised either way);
    * ``lm_head`` row ``perm[u]`` gets ``successor`` times the unit embedding of token ``u``, for one
      seeded permutation ``perm`` of the vocabulary, so the token after ``u`` is ``perm[u]`` with a
      margin of several logit units.

    Returns ``perm``. Measured on the Qwen2-0.5B shape (24 layers, seed 0): smallest top-1 margin
    2.09 over 17 steps against a 0.0057 fp16 logit error; the layers move logits by up to 1.05,
    attention alone by up to 0.10.
    """
    emb = model.get_input_embeddings().weight
    head = model.get_output_embeddings().weight
    perm = torch.randperm(emb.shape[0], generator=torch.Generator().manual_seed(seed))
    with torch.no_grad():
        emb.mul_(embed_scale)
        unit = emb / emb.norm(dim=1, keepdim=True)
        head[perm] += successor * unit
    return perm


def _dequantized(w: np.ndarray) -> np.ndarray:
    """``dequantize(quantize_per_channel(w))``, computed over row blocks on several threads (the
    format is per row, so the blocks give the whole matrix's values bit for bit)."""
    out = np.empty(w.shape, np.float32)
    step = max(16, -(-w.shape[0] // (4 * _workers())))

    def one(lo):
        q, s = quantize_per_channel(w[lo:lo + step])
        out[lo:lo + step] = dequantize(q, s)

    with ThreadPoolExecutor(_workers()) as pool:
        list(pool.map(one, range(0, w.shape[0], step)))
    return out


def _round_fp16_(t: torch.Tensor) -> None:
    t.copy_(t.to(torch.float16).to(torch.float32))


def quantized_reference(model: nn.Module, targets: tuple[str, ...] = PROJECTIONS) -> nn.Module:
    """Deep copy of ``model`` (fp32, CPU) holding exactly the device model's weights."""
    ref = copy.deepcopy(model).float().cpu().eval()
    projected: set[int] = set()
    with torch.no_grad():
        for parent in ref.modules():
            for name, child in parent.named_children():
                if isinstance(child, nn.Linear) and name in targets:
                    child.weight.copy_(torch.from_numpy(_dequantized(child.weight.detach().numpy())))
                    projected.add(id(child.weight))
        for p in ref.parameters():
            if id(p) not in projected:
                _round_fp16_(p)
    ref.config._attn_implementation = "eager"
    return ref


@torch.no_grad()
def prefix_cache(model: nn.Module, prefix: torch.Tensor):
    """``(cache, n)``: the ``DynamicCache`` after a forward over the ``n`` tokens of ``prefix``, for
    :func:`teacher_forced_logits` / :func:`prefill_kv` on prompts that start with it (rows that share
    a prompt prefix, as the reference's prefix cache serves them)."""
    ids = prefix.reshape(1, -1).to(torch.long).cpu()
    out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
    return out.past_key_values, int(ids.shape[1])


def _rest(prompt: torch.Tensor, past):
    """The cache to continue from (a deep copy of ``past``'s) and how many prompt tokens it holds."""
    if past is None:
        return None, 0
    cache, n = past
    if prompt.numel() <= n:
        raise ValueError("a prompt continued from a prefix cache must be longer than the prefix")
    return copy.deepcopy(cache), n


@torch.no_grad()
def teacher_forced_logits(model: nn.Module, prompt: torch.Tensor, generated: torch.Tensor, past=None) -> torch.Tensor:
    """Logits ``[len(generated), V]`` (fp32) that each of ``generated`` was chosen from.

    ``generated[0]`` follows ``prompt``; ``generated[i]`` follows
    ``prompt + generated[:i]``. One causal forward over
    ``prompt + generated[:-1]`` keeping the last ``len(generated)`` positions;
    with ``past`` (from :func:`prefix_cache`, holding the first ``n`` prompt
    tokens) the forward starts after them.
    """
    prompt = prompt.reshape(-1).to(torch.long).cpu()
    generated = generated.reshape(-1).to(torch.long).cpu()
    n = int(generated.numel())
    cache, skip = _rest(prompt, past)
    ids = torch.cat([prompt[skip:], generated[:-1]]).view(1, -1)
    out = model(input_ids=ids, past_key_values=cache, use_cache=cache is not None, logits_to_keep=n)
    return out.logits[0].float()


@torch.no_grad()
def prefill_kv(model: nn.Module, prompt: torch.Tensor, past=None
               ) -> tuple[list[tuple[torch.Tensor, torch.Tensor]], torch.Tensor]:
    """Prompt forward: per layer ``(keys, values)`` ``[Hkv, P, D]`` (after RoPE, fp32) and the last logits ``[V]``.

    With ``past`` (:func:`prefix_cache`) only the tokens after the prefix are run; the keys and
    values returned still cover the whole prompt.
    """
    prompt = prompt.reshape(-1).to(torch.long).cpu()
    cache, skip = _rest(prompt, past)
    out = model(input_ids=prompt[skip:].view(1, -1), past_key_values=cache, use_cache=True, logits_to_keep=1)
    kv = [(layer.keys[0], layer.values[0]) for layer in out.past_key_values.layers]
    return kv, out.logits[0, -1].float()


@torch.no_grad()
def continue_logits(model: nn.Module, kv: list[tuple[torch.Tensor, torch.Tensor]], tokens: torch.Tensor
                    ) -> torch.Tensor:
    """Logits ``[len(tokens), V]`` (fp32, on the CPU) of a forward over ``tokens`` continuing a context
    whose per-layer keys and values ``kv`` (``[Hkv, S, D]``, keys after RoPE, as :func:`prefill_kv`
    returns them or as a paged pool holds them) are given: ``tokens[i]`` sits at position ``S + i``
    and row ``i`` is the distribution of the token after it.

    This is the decode step's view of a context: the native step reads K/V from the pool whatever
    wrote them, so a context of random K/V (the bench's) is checked by handing those same values
    here. The cache is built in the model's own device and dtype, so an fp16 copy of the model on
    the GPU gives the fp16 yardstick of the same continuation.
    """
    from transformers import DynamicCache

    p = next(model.parameters())
    cache = DynamicCache(config=model.config)
    for li, (k, v) in enumerate(kv):
        cache.update(k.to(device=p.device, dtype=p.dtype).unsqueeze(0),
                     v.to(device=p.device, dtype=p.dtype).unsqueeze(0), li)
    ids = tokens.reshape(1, -1).to(device=p.device, dtype=torch.long)
    out = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=int(ids.shape[1]))
    return out.logits[0].float().cpu()


@torch.no_grad()
def greedy_reference(model: nn.Module, prompt: torch.Tensor, steps: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Free-running greedy decode with a ``DynamicCache``: ``steps + 1`` tokens and their logits."""
    ids = prompt.reshape(1, -1).to(torch.long).cpu()
    out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
    cache = out.past_key_values
    logits = [out.logits[0, -1].float()]
    tokens = [int(logits[-1].argmax())]
    for _ in range(steps):
        out = model(input_ids=torch.tensor([[tokens[-1]]]), past_key_values=cache, use_cache=True)
        cache = out.past_key_values
        logits.append(out.logits[0, -1].float())
        tokens.append(int(logits[-1].argmax()))
    return torch.tensor(tokens), torch.stack(logits)


def greedy_agreement(logits_ref: torch.Tensor, tokens: torch.Tensor, tie_tol: float) -> dict:
    """Compare device greedy ``tokens [T]`` with the teacher-forced oracle ``logits_ref [T, V]``.

    A step agrees when the token is the oracle's argmax. A step that does not
    agree is a near tie when the oracle prefers its argmax by at most
    ``tie_tol`` over the chosen token. Returns counts, the index of the first
    disagreement (or -1) and the largest gap seen at a disagreement.
    """
    tokens = tokens.reshape(-1).to(torch.long).cpu()
    best = logits_ref.argmax(dim=-1)
    gap = logits_ref.max(dim=-1).values - logits_ref.gather(1, tokens.view(-1, 1)).squeeze(1)
    miss = best != tokens
    idx = torch.nonzero(miss).flatten()
    return {
        "steps": int(tokens.numel()),
        "mismatches": int(miss.sum()),
        "first_mismatch": int(idx[0]) if idx.numel() else -1,
        "max_gap_at_mismatch": float(gap[miss].max()) if idx.numel() else 0.0,
        "ties_ok": bool((gap[miss] <= tie_tol).all()) if idx.numel() else True,
    }
