"""Generate the committed golden fixtures from the CPU oracle.

Run from the repo root: ``python tests/golden/make_golden.py``. The fixtures pin
the oracle's outputs (and through the GPU parity tests, the kernels') against
later edits. Inputs are seeded and constructed here; nothing is imported from
the reference.

* ``int8_edge.npz``     - quantizer / pack / linear on a 48x128 matrix whose
                          rows cover random, zero, exact half-way ties,
                          underflowing, clamped-scale, single-element and
                          negative-extreme cases.
* ``int8_config1.json`` - sha256 digests and slices of q / s / packed for the
                          4096x4096 weight of the single-linear benchmark
                          (seed 0), plus y for x [1, 4096].
* ``attn_small.npz``    - a ragged batched paged-decode case (B=3, Hkv=2,
                          G=4, D=64, bs=16, seq_lens 1/17/100, permuted block
                          ids) with its fp32 output.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import int8_quant, paged_attention  # noqa: E402


def edge_weight() -> np.ndarray:
    rng = np.random.default_rng(0)
    n, k = 48, 128
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[32] = 0.0
    # Row 33: exact ties. amax = 127*s so s is exactly recovered; other entries are (j + 0.5)*s.
    s = np.float32(np.float16(0.01))
    vals = (np.arange(k) % 120 - 60 + 0.5).astype(np.float32) * s
    vals[0] = np.float32(127) * s
    vals[1] = np.float32(-126.5) * s
    vals[2] = np.float32(0.5) * s
    vals[3] = np.float32(-0.5) * s
    vals[4] = np.float32(1.5) * s
    vals[5] = np.float32(2.5) * s
    w[33] = vals
    w[34] = (rng.standard_normal(k) * 1e-30).astype(np.float32)  # s underflows fp16 -> 2^-24
    w[35] = (rng.standard_normal(k) * 1e7).astype(np.float32)  # amax/127 > 65504 -> clamped
    w[36] = 0.0
    w[36, 77] = np.float32(-3.25)  # single element
    w[37] = -np.abs(w[37])
    w[37, 5] = np.float32(-0.5)  # negative extreme
    w[38:] = rng.standard_normal((10, k)).astype(np.float32)
    w[38, 0] = np.max(np.abs(w[38])) * -1.0
    return w


def make_int8_edge(out_dir: str) -> None:
    w = edge_weight()
    q, s = int8_quant.quantize_per_channel(w)
    packed = int8_quant.pack_tiles(q)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, w.shape[1])).astype(np.float16)
    bias = (rng.standard_normal(w.shape[0]) * 0.1).astype(np.float16)
    y = int8_quant.linear_ref_fp32(x, q, s, bias)
    np.savez_compressed(os.path.join(out_dir, "int8_edge.npz"), w=w, q=q, s=s, packed=packed, x=x, bias=bias, y=y)


def config1_inputs() -> tuple[np.ndarray, np.ndarray]:
    """Config 1: x [1,4096] fp16 ~ N(0,1), W [4096,4096] fp32 ~ N(0,0.02), torch seed 0 (x drawn first)."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 4096, generator=g).to(torch.float16).numpy()
    w = (torch.randn(4096, 4096, generator=g) * 0.02).numpy().astype(np.float32)
    return x, w


def make_int8_config1(out_dir: str) -> None:
    x, w = config1_inputs()
    q, s = int8_quant.quantize_per_channel(w)
    packed = int8_quant.pack_tiles(q)
    y = int8_quant.linear_ref_fp32(x, q, s)
    doc = {
        "inputs": "torch.Generator().manual_seed(0); x = randn(1,4096).half(); w = randn(4096,4096)*0.02",
        "q_sha256": hashlib.sha256(q.tobytes()).hexdigest(),
        "s_sha256": hashlib.sha256(s.tobytes()).hexdigest(),
        "packed_sha256": hashlib.sha256(packed.tobytes()).hexdigest(),
        "w_sha256": hashlib.sha256(w.tobytes()).hexdigest(),
        "q_head": q[:2, :16].tolist(),
        "s_head_bits": s[:8].view(np.uint16).tolist(),
        "y_head": [float(v) for v in y[0, :16]],
        "y_sum": float(np.sum(y.astype(np.float64))),
    }
    with open(os.path.join(out_dir, "int8_config1.json"), "w") as f:
        json.dump(doc, f, indent=1)


def make_attn_small(out_dir: str) -> None:
    g = torch.Generator().manual_seed(7)
    bsz, hkv, grp, d, bs = 3, 2, 4, 64, 16
    seq_lens = [1, 17, 100]
    num_blocks = 24
    perm = torch.randperm(num_blocks, generator=g)
    max_blocks = 8
    tables = torch.zeros(bsz, max_blocks, dtype=torch.int32)
    used = 0
    for b, s in enumerate(seq_lens):
        n = -(-s // bs)
        tables[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    k_layer = torch.randn(num_blocks, hkv, bs, d, generator=g).to(torch.float16)
    v_layer = torch.randn(num_blocks, hkv, bs, d, generator=g).to(torch.float16)
    q = torch.randn(bsz, hkv * grp, 1, d, generator=g).to(torch.float16)
    scale = d**-0.5
    out = paged_attention.decode_rows_fp32(q, k_layer, v_layer, tables, seq_lens, scale, grp)
    np.savez_compressed(os.path.join(out_dir, "attn_small.npz"), q=q.numpy(), k_layer=k_layer.numpy(),
                        v_layer=v_layer.numpy(), tables=tables.numpy(), seq_lens=np.array(seq_lens, np.int32),
                        scale=np.float32(scale), group=np.int32(grp), out=out.numpy())


def main() -> None:
    make_int8_edge(HERE)
    make_int8_config1(HERE)
    make_attn_small(HERE)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
