"""Algorithmic HBM bytes of the decode-step kernels, for roofline fractions.

These are the bytes a kernel must move at the least, not what a counter reads:

* paged attention: K and V of every attended token once per kv-head (the GQA query heads
  of a kv-head share them), the query and output rows, the block ids read and the lengths;
* an int8 linear ``[M, K] x [K, N]``: the int8 weights once, the fp16 scales (and bias),
  the fp16 input rows and the fp16 output rows (``out_cols`` when the epilogue writes fewer
  columns than N, as the gate||up SwiGLU epilogue writes N / 2).
"""

from __future__ import annotations

import math


def attention_hbm_bytes(seq_lens, num_kv_heads: int, head_dim: int, num_heads: int, block_size: int,
                        elem_bytes: int = 2) -> int:
    lens = [max(int(s), 0) for s in seq_lens]
    kv = sum(lens) * num_kv_heads * head_dim * 2 * elem_bytes
    qo = 2 * len(lens) * num_heads * head_dim * elem_bytes
    meta = sum(math.ceil(s / block_size) for s in lens) * 4 + len(lens) * 4
    return kv + qo + meta


def linear_hbm_bytes(m: int, n: int, k: int, bias: bool = False, out_cols: int | None = None) -> int:
    return n * k + 2 * n + 2 * m * k + 2 * m * (n if out_cols is None else out_cols) + (2 * n if bias else 0)
