"""Seeded randomized parity sweeps of the two hot-path kernels against the CPU oracle.

Each case draws its shape from a fixed seed, so a failure names a reproducible case:

* paged attention (through the C ABI): D 64/128, block 4/8/16/32, GQA 1..8, 1..24 rows of
  0..2048 tokens or 65..100 rows of 0..300 tokens, split granularity 0/16/64/256 tokens,
  tables narrower than some rows, rows that alias other rows' blocks (with and without
  ``MX_PA_SHARED_BLOCKS``),
  strided query/output views and bf16 (``MX_PA_BF16``); bar atol/rtol 1e-2 (2e-2 in bf16)
  against ``decode_rows_fp32``;
* int8 linear: N = 16..6400, K = 64..4096, M = 1..300 (chunks of 128 rows past that),
  strided x, with and without bias; bar atol/rtol 1e-2 against ``linear_ref_fp32``, and
  where K is split the partials summed bias-first in split order equal the output bit
  for bit.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import int8_quant
from oracle import paged_attention as oracle_pa
from runtime_amd.phase2 import _hip
from runtime_amd.phase2.int8_linear import int8_linear, int8_linear_partials, linear_splits, pack_weight

pytestmark = pytest.mark.gpu
ATOL = 1e-2
RTOL = 1e-2
MX_PA_SHARED_BLOCKS = 1
MX_PA_BF16 = 2
BF16_TOL = 2e-2  # 8 significant bits: output and probabilities rounded to bf16 (2^-9 relative each)


def _attention_case(seed: int):
    rng = np.random.default_rng(5000 + seed)
    d = int(rng.choice([64, 128]))
    bs = int(rng.choice([4, 8, 16, 16, 32]))
    grp = int(rng.integers(1, 9))
    hkv = int(rng.choice([1, 2, 4, 8]))
    if rng.random() < 0.2:  # more than 64 rows: the kernel's multi-pass row search
        bsz = int(rng.integers(65, 101))
        lens = rng.integers(0, 300, size=bsz)
    else:
        bsz = int(rng.integers(1, 25))
        lens = rng.integers(0, 2049, size=bsz)
    lens[rng.random(bsz) < 0.15] = 0
    lens[rng.random(bsz) < 0.15] = bs * rng.integers(1, 8)  # exact block multiples
    need = [math.ceil(int(s) / bs) for s in lens]
    width = max(max(need), 1)
    if rng.random() < 0.25:
        width = max(1, width - int(rng.integers(1, 4)))  # some rows run past the table
    chunk = int(rng.choice([0, 0, 16, 64, 256]))
    return dict(d=d, bs=bs, grp=grp, hkv=hkv, lens=[int(s) for s in lens], need=need, width=width, chunk=chunk,
                alias=bool(rng.random() < 0.4), strided=bool(rng.random() < 0.3), bf16=bool(rng.random() < 0.3),
                rng=rng)


@pytest.mark.parametrize("seed", range(48))
def test_attention_randomized(seed):
    c = _attention_case(seed)
    d, bs, grp, hkv, lens, width, rng = c["d"], c["bs"], c["grp"], c["hkv"], c["lens"], c["width"], c["rng"]
    bsz, hq = len(lens), hkv * grp
    total = sum(min(n, width) for n in c["need"])
    nb = total + 5
    perm = rng.permutation(nb)
    tables = np.zeros((bsz, width), dtype=np.int32)
    used = 0
    for b, n in enumerate(c["need"]):
        n = min(n, width)
        tables[b, :n] = perm[used:used + n]
        used += n
    if c["alias"] and bsz > 1:  # later rows reuse the first row's leading blocks
        share = min(c["need"][0], width, 3)
        for b in range(1, bsz, 2):
            m = min(share, c["need"][b], width)
            tables[b, :m] = tables[0, :m]
    g = torch.Generator().manual_seed(seed)
    dt = torch.bfloat16 if c["bf16"] else torch.float16
    k = torch.randn(nb, hkv, bs, d, generator=g).to(dt).cuda()
    v = torch.randn(nb, hkv, bs, d, generator=g).to(dt).cuda()
    if c["strided"]:
        qbig = torch.randn(bsz, hq + 3, 1, d + 8, generator=g).to(dt).cuda()
        q = qbig[:, 2:2 + hq, :, 8:]
        out_big = torch.full((bsz, hq + 1, 1, d + 16), float("nan"), dtype=dt, device="cuda")
        out = out_big[:, 1:, :, 16:]
    else:
        q = torch.randn(bsz, hq, 1, d, generator=g).to(dt).cuda()
        out = torch.empty_like(q)
    tables_d = torch.from_numpy(tables).cuda()
    lens_d = torch.tensor(lens, dtype=torch.int32, device="cuda")
    scale = d ** -0.5
    lib = _hip.load()
    nbytes = lib.mx_paged_attn_workspace_bytes(bsz, hq, hkv, d, width, bs, c["chunk"])
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    flags = (MX_PA_SHARED_BLOCKS if c["alias"] and seed % 2 == 0 else 0) | (MX_PA_BF16 if c["bf16"] else 0)
    print(f"[attn] seed {seed}: B {bsz} Hq {hq} Hkv {hkv} D {d} bs {bs} width {width} chunk {c['chunk']} "
          f"alias {c['alias']} strided {c['strided']} bf16 {c['bf16']} flags {flags} lens {lens}", flush=True)
    _hip.check(lib.mx_paged_attn_decode(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
        tables_d.data_ptr(), tables_d.stride(0), width, lens_d.data_ptr(), bsz, hq, hkv, d, bs, nb, scale,
        out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), nbytes, c["chunk"], flags,
        _hip.stream_handle(q.device)), "decode")
    torch.cuda.synchronize()
    err = int(ws[lib.mx_paged_attn_error_offset(bsz, hq, hkv, d, width, bs, c["chunk"]):][:4].view(torch.int32).item())
    assert err == 0
    want = oracle_pa.decode_rows_fp32(q.cpu(), k.cpu(), v.cpu(), tables_d.cpu(), lens, scale, grp)
    tol = BF16_TOL if c["bf16"] else ATOL
    np.testing.assert_allclose(out.float().cpu().numpy(), want.numpy(), atol=tol, rtol=tol)
    if c["strided"]:  # nothing outside the output view was written
        assert torch.isnan(out_big[:, :1]).all() and torch.isnan(out_big[:, 1:, :, :16]).all()


def _linear_case(seed: int):
    rng = np.random.default_rng(7000 + seed)
    n = 16 * int(rng.integers(1, 401))
    k = 64 * int(rng.integers(1, 65))
    m = int(rng.choice([1, 2, 3, 4, 5, 8, 16, 31, 32, 33, 48, 64, 65, 96, 100, 127, 128, 129, 200, 300]))
    return n, k, m, bool(rng.random() < 0.5), bool(rng.random() < 0.3)


@pytest.mark.parametrize("seed", range(48))
def test_linear_randomized(seed):
    n, k, m, with_bias, strided = _linear_case(seed)
    print(f"[linear] seed {seed}: M {m} N {n} K {k} bias {with_bias} strided {strided}", flush=True)
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 0.02).numpy().astype(np.float32)
    q, s = int8_quant.quantize_per_channel(w)
    xfull = (torch.randn(m, k + (72 if strided else 0), generator=g)).to(torch.float16)
    x = xfull[:, :k].cuda() if not strided else xfull.cuda()[:, :k]
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.float16) if with_bias else None
    packed = pack_weight(torch.from_numpy(q).cuda())
    sd = torch.from_numpy(s).cuda()
    bd = bias.cuda() if bias is not None else None
    y = int8_linear(x, packed, sd, bd, n)
    want = int8_quant.linear_ref_fp32(x.cpu().numpy(), q, s, None if bias is None else bias.numpy())
    np.testing.assert_allclose(y.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    if m <= 128:
        splits = linear_splits(m, n, k)
        if splits > 1:
            part = torch.full((splits * m * n,), float("nan"), dtype=torch.float32, device="cuda")
            assert int8_linear_partials(x, packed, sd, n, part) == splits
            acc = (bd.float() if bd is not None else torch.zeros(n, device="cuda")).unsqueeze(0).expand(m, n).clone()
            for sp in part.view(splits, m, n):
                acc = acc + sp
            assert torch.equal(acc.half(), y)
