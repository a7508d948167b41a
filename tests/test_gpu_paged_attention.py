"""GPU parity of the HIP paged-attention decode kernel against the CPU oracle.

Bar: fp16 outputs within atol 1e-2 and rtol 1e-2 of the fp32 per-row oracle
(oracle/paged_attention.py: decode_rows_fp32), on the reference's own test
shapes (tests/test_paged_attention_kernel_parity.py:103-198 of the reference),
the full config-2 shape, and the edge cases (ragged, zero-length, clamped,
GQA 1..8, D 64/128, block size 16/32, split granularities).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_attention as oracle_pa
from runtime_amd.phase2 import _hip
from runtime_amd.phase2.block_paged_attention import block_paged_attention_forward
from runtime_amd.phase2.paged_attention_hip import (
    PagedDecodeBatchMetadata,
    paged_attention_decode,
    paged_attention_decode_batched,
    reset_paged_decode_batch_metadata,
    set_paged_decode_batch_metadata,
    workspace_error_flag,
)
from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

pytestmark = pytest.mark.gpu
ATOL = 1e-2
RTOL = 1e-2


def oracle_out(q, k_layer, v_layer, tables, seq_lens, scale, grp):
    """Copy only the referenced blocks to the host and run the fp32 per-row oracle."""
    lens = [int(s) for s in torch.as_tensor(seq_lens).cpu().tolist()]
    t_cpu = tables.cpu()
    bs = k_layer.shape[2]
    max_blocks = t_cpu.shape[1]
    ids = sorted({int(x) for b, s in enumerate(lens) if s > 0
                  for x in t_cpu[b, :min(math.ceil(s / bs), max_blocks)].tolist()})
    if not ids:
        ids = [0]
    remap = {old: i for i, old in enumerate(ids)}
    idx = torch.tensor(ids, device=k_layer.device, dtype=torch.long)
    kc = k_layer.index_select(0, idx).cpu()
    vc = v_layer.index_select(0, idx).cpu()
    t2 = torch.zeros_like(t_cpu)
    for b, s in enumerate(lens):
        for j in range(min(math.ceil(max(s, 0) / bs), max_blocks)):
            t2[b, j] = remap[int(t_cpu[b, j])]
    return oracle_pa.decode_rows_fp32(q.cpu(), kc, vc, t2, lens, scale, grp)


def _check(got, want, msg=""):
    np.testing.assert_allclose(got.float().cpu().numpy(), want.numpy(), atol=ATOL, rtol=RTOL, err_msg=msg)


def _random_case(seed, bsz, hkv, grp, d, bs, seq_lens, num_blocks=None, pad_value=0):
    g = torch.Generator().manual_seed(seed)
    nblk = [math.ceil(max(s, 0) / bs) for s in seq_lens]
    max_blocks = max(max(nblk), 1)
    num_blocks = num_blocks or (sum(nblk) + 3)
    perm = torch.randperm(num_blocks, generator=g)
    tables = torch.full((bsz, max_blocks), pad_value, dtype=torch.int32)
    used = 0
    for b, n in enumerate(nblk):
        tables[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    k = torch.randn(num_blocks, hkv, bs, d, generator=g).to(torch.float16).cuda()
    v = torch.randn(num_blocks, hkv, bs, d, generator=g).to(torch.float16).cuda()
    q = torch.randn(bsz, hkv * grp, 1, d, generator=g).to(torch.float16).cuda()
    return q, k, v, tables.cuda(), torch.tensor(seq_lens, dtype=torch.int32, device="cuda")


class _Pool:
    """Minimal pool stand-in exposing the views the decode entry point reads."""

    def __init__(self, k, v):
        self.k, self.v = k, v

    def _ensure_pools(self):
        pass

    def k_layer_view(self, layer):
        return self.k

    def v_layer_view(self, layer):
        return self.v


def _decode(q, k, v, tables, lens, scale, grp):
    meta = PagedDecodeBatchMetadata(pool=_Pool(k, v), layer_idx=0, block_tables=tables, seq_lens=lens)
    return paged_attention_decode_batched(q, meta, grp, scale)


@pytest.mark.parametrize("seq_len", [128, 768])
def test_reference_single_row_cases(seq_len):
    """tests/test_paged_attention_kernel_parity.py:103-125 and :187-198 (Hkv=2, G=4, D=64, bs=16)."""
    hkv, grp, d, bs = 2, 4, 64, 16
    num_blocks = math.ceil(seq_len / bs) + 1
    pool = GpuKVBlockPool(num_blocks=num_blocks, block_size_tokens=bs, num_layers=1, num_kv_heads=hkv, head_dim=d,
                          dtype=torch.float16, device="cuda")
    ids = list(range(num_blocks))
    torch.manual_seed(42)
    k = torch.randn(1, hkv, seq_len, d, device="cuda", dtype=torch.float16)
    v = torch.randn(1, hkv, seq_len, d, device="cuda", dtype=torch.float16)
    pool.write_tokens(0, ids, 0, k, v)
    query = torch.randn(1, hkv * grp, 1, d, device="cuda", dtype=torch.float16)
    scale = d**-0.5
    got = paged_attention_decode(query=query, pool=pool, layer_idx=0, block_ids=ids, seq_len=seq_len,
                                 num_kv_groups=grp, scaling=scale)
    keys, values = pool.gather_layer(0, ids, seq_len)
    want = oracle_pa.reference_sdpa_attention(query.cpu().float(), keys.cpu().float(), values.cpu().float(), scale,
                                              grp)
    assert (got.float().cpu() - want).abs().max().item() < 1e-2
    table = torch.tensor(ids, dtype=torch.int32, device="cuda").view(1, -1)
    _check(got, oracle_out(query, pool.k_layer_view(0), pool.v_layer_view(0), table, [seq_len], scale, grp))


def test_reference_batched_ragged():
    """tests/test_paged_attention_kernel_parity.py:127-185: B=4, seq_lens 7/15/31/63, seed 99."""
    hkv, grp, d, bs, bsz = 2, 4, 64, 16, 4
    seq_lens = [7, 15, 31, 63]
    num_blocks = math.ceil(max(seq_lens) / bs) + 2
    pool = GpuKVBlockPool(num_blocks=num_blocks * bsz, block_size_tokens=bs, num_layers=1, num_kv_heads=hkv,
                          head_dim=d, dtype=torch.float16, device="cuda")
    torch.manual_seed(99)
    scale = d**-0.5
    tables = torch.zeros(bsz, num_blocks, device="cuda", dtype=torch.int32)
    for b in range(bsz):
        ids = list(range(b * num_blocks, (b + 1) * num_blocks))
        nlog = math.ceil(seq_lens[b] / bs)
        tables[b, :nlog] = torch.tensor(ids[:nlog], device="cuda", dtype=torch.int32)
        k = torch.randn(1, hkv, seq_lens[b], d, device="cuda", dtype=torch.float16)
        v = torch.randn(1, hkv, seq_lens[b], d, device="cuda", dtype=torch.float16)
        pool.write_tokens(0, ids, 0, k, v)
    query = torch.randn(bsz, hkv * grp, 1, d, device="cuda", dtype=torch.float16)
    meta = PagedDecodeBatchMetadata(pool=pool, layer_idx=0, block_tables=tables,
                                    seq_lens=torch.tensor(seq_lens, device="cuda", dtype=torch.int32))
    got = paged_attention_decode_batched(query, meta, grp, scale)
    _check(got, oracle_out(query, pool.k_layer_view(0), pool.v_layer_view(0), tables, seq_lens, scale, grp))


def _config2(seed=0):
    """Benchmark config 2: B=32, Hq=32, Hkv=8, D=128, bs=16, ctx ~ U[128, 4096], one randperm(16384) pool."""
    g = torch.Generator().manual_seed(seed)
    bsz, hkv, grp, d, bs, nb = 32, 8, 4, 128, 16, 16384
    lens = torch.randint(128, 4097, (bsz,), generator=g)
    perm = torch.randperm(nb, generator=g)
    max_blocks = 4096 // bs
    tables = torch.zeros(bsz, max_blocks, dtype=torch.int32)
    used = 0
    for b in range(bsz):
        n = math.ceil(int(lens[b]) / bs)
        tables[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    gd = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn(nb, hkv, bs, d, generator=gd, device="cuda", dtype=torch.float16)
    v = torch.randn(nb, hkv, bs, d, generator=gd, device="cuda", dtype=torch.float16)
    q = torch.randn(bsz, hkv * grp, 1, d, generator=gd, device="cuda", dtype=torch.float16)
    return q, k, v, tables.cuda(), lens.to(torch.int32).cuda(), grp, d**-0.5


@pytest.mark.parametrize("seq_len", [7, 100])
def test_reference_block_size_4_shapes(seq_len):
    """tests/test_paged_attention_kernel_parity.py:80-100 of the reference run its short case at block size 4
    (Hkv 2, G 2, 7 tokens; there D 32 in fp32 on the CPU path). The same shapes at D 64 in fp16 (the kernel's
    smallest head dim): a 16-token tile spans 4 blocks, each lane reads its own block."""
    hkv, grp, d, bs = 2, 2, 64, 4
    q, k, v, tables, sl = _random_case(40 + seq_len, 1, hkv, grp, d, bs, [seq_len])
    scale = d**-0.5
    _check(_decode(q, k, v, tables, sl, scale, grp), oracle_out(q, k, v, tables, sl, scale, grp))


# bf16 has 8 significant bits: rounding the output alone moves it by up to 2^-9 relative and the
# probabilities enter P.V rounded to bf16 (2^-9 relative each), so the bar is atol = rtol = 2e-2.
BF16_TOL = 2e-2


@pytest.mark.parametrize("hkv,grp,d,bs,lens", [(2, 4, 64, 16, [128, 768, 1, 0]), (8, 4, 128, 16, [300, 2049, 16]),
                                               (2, 7, 64, 32, [100, 513]), (4, 2, 128, 4, [7, 100, 37])])
def test_bf16_pool_and_query(hkv, grp, d, bs, lens):
    """bf16 q and pool (MX_PA_BF16): K/V written through GpuKVBlockPool.write_tokens (the bf16
    append), decoded through paged_attention_decode_batched, against the fp32 oracle on the same
    bf16 values."""
    bsz = len(lens)
    need = [math.ceil(max(s, 0) / bs) for s in lens]
    nb = sum(need) + 3
    g = torch.Generator().manual_seed(sum(lens) + d)
    perm = torch.randperm(nb, generator=g)
    pool = GpuKVBlockPool(num_blocks=nb, block_size_tokens=bs, num_layers=1, num_kv_heads=hkv, head_dim=d,
                          dtype=torch.bfloat16, device="cuda")
    tables = torch.zeros(bsz, max(max(need), 1), dtype=torch.int32)
    at = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[at:at + n].to(torch.int32)
        at += n
        if lens[b] > 0:
            kv = torch.randn(2, 1, hkv, lens[b], d, generator=g).to(torch.bfloat16).cuda()
            pool.write_tokens(0, tables[b, :n].tolist(), 0, kv[0], kv[1])
    q = torch.randn(bsz, hkv * grp, 1, d, generator=g).to(torch.bfloat16).cuda()
    meta = PagedDecodeBatchMetadata(pool=pool, layer_idx=0, block_tables=tables.cuda(),
                                    seq_lens=torch.tensor(lens, dtype=torch.int32, device="cuda"))
    scale = d**-0.5
    out = paged_attention_decode_batched(q, meta, grp, scale)
    assert out.dtype == torch.bfloat16
    want = oracle_out(q, pool.k_layer_view(0), pool.v_layer_view(0), tables, lens, scale, grp)
    np.testing.assert_allclose(out.float().cpu().numpy(), want.numpy(), atol=BF16_TOL, rtol=BF16_TOL)
    with pytest.raises(ValueError):  # mixed dtypes are refused
        paged_attention_decode_batched(q.half(), meta, grp, scale)


def test_config2_full_shape_and_repeatability():
    q, k, v, tables, lens, grp, scale = _config2()
    got = _decode(q, k, v, tables, lens, scale, grp)
    again = _decode(q, k, v, tables, lens, scale, grp)
    assert torch.equal(got, again), "decode must be deterministic and leave its workspace reusable"
    _check(got, oracle_out(q, k, v, tables, lens, scale, grp))
    assert workspace_error_flag() == 0



def test_config2_full_shape_bf16_plain_and_tile_plan():
    """Config 2's shape (B 32, Hq 32, Hkv 8, D 128, block 16, contexts U[128, 4096], 16384-block pool)
    with bf16 q and K/V (MX_PA_BF16): the plain call, the recording call and the plan-reading call give
    the same bits, and match the fp32 oracle on the same bf16 values within BF16_TOL."""
    from runtime_amd.phase2.paged_attention_hip import MX_PA_PLAN_READ, MX_PA_PLAN_WRITE

    q, k, v, tables, lens, grp, scale = _config2(seed=3)
    q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    dev = q.device
    before = workspace_error_flag(dev)
    plain = _decode(q, k, v, tables, lens, scale, grp)
    from runtime_amd.phase2.paged_attention_hip import _decode as hip_decode
    rec = hip_decode(q, k, v, tables, lens, scale, grp, plan=MX_PA_PLAN_WRITE)
    read = hip_decode(q, k, v, tables, lens, scale, grp, plan=MX_PA_PLAN_READ)
    torch.cuda.synchronize()
    assert plain.dtype == torch.bfloat16
    assert torch.equal(rec.view(torch.int16), plain.view(torch.int16))
    assert torch.equal(read.view(torch.int16), plain.view(torch.int16))
    assert (workspace_error_flag(dev) & ~before) == 0
    want = oracle_out(q, k, v, tables, lens, scale, grp)
    np.testing.assert_allclose(plain.float().cpu().numpy(), want.numpy(), atol=BF16_TOL, rtol=BF16_TOL)

def _abi_decode(q, k, v, tables, lens, scale, grp, chunk_tokens, num_pool_blocks=None, flags=0):
    lib = _hip.load()
    bsz, hq, _, d = q.shape
    nb, hkv, bs, _ = k.shape
    mb = tables.shape[1]
    nbytes = lib.mx_paged_attn_workspace_bytes(bsz, hq, hkv, d, mb, bs, chunk_tokens)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    _hip.check(lib.mx_paged_attn_decode(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
        tables.data_ptr(), tables.stride(0), mb, lens.data_ptr(), bsz, hq, hkv, d, bs,
        num_pool_blocks if num_pool_blocks is not None else nb, scale, out.data_ptr(), out.stride(0), out.stride(1),
        ws.data_ptr(), nbytes, chunk_tokens, flags, _hip.stream_handle(q.device)), "decode")
    torch.cuda.synchronize()
    err = int(ws[lib.mx_paged_attn_error_offset(bsz, hq, hkv, d, mb, bs, chunk_tokens):][:4].view(torch.int32).item())
    return out, err


def test_split_chunk_size_invariance():
    q, k, v, tables, lens = _random_case(3, 6, 2, 4, 128, 16, [1, 16, 17, 255, 1000, 2049])
    grp, scale = 4, 128**-0.5
    want = oracle_out(q, k, v, tables, lens, scale, grp)
    outs = []
    for ct in (16, 64, 256, 1024, 0):
        out, err = _abi_decode(q, k, v, tables, lens, scale, grp, ct)
        assert err == 0
        _check(out, want, f"chunk_tokens={ct}")
        outs.append(out.float())
    for o in outs[1:]:
        assert (o - outs[0]).abs().max().item() < 2e-3


@pytest.mark.parametrize("d,bs", [(128, 16), (128, 32), (64, 16), (64, 32), (128, 4), (64, 8)])
def test_shared_blocks_flag_is_bit_identical(d, bs):
    """MX_PA_SHARED_BLOCKS changes only the cache policy of the K/V loads: same bits, with
    rows that alias each other's blocks."""
    q, k, v, tables, lens = _random_case(31 + d + bs, 4, 2, 4, d, bs, [300, 700, 64, 1000])
    tables = tables.clone()
    tables[1, :4] = tables[0, :4]  # rows 0, 1 and 3 share their first blocks
    tables[3, :4] = tables[0, :4]
    scale = d**-0.5
    plain, err0 = _abi_decode(q, k, v, tables, lens, scale, 4, 0)
    shared, err1 = _abi_decode(q, k, v, tables, lens, scale, 4, 0, flags=1)
    assert err0 == 0 and err1 == 0
    assert torch.equal(plain, shared)
    _check(shared, oracle_out(q, k, v, tables, lens, scale, 4))


@pytest.mark.parametrize("hkv,grp,d,bs", [(2, 7, 64, 16), (4, 1, 128, 16), (2, 8, 128, 16), (3, 2, 64, 32),
                                          (8, 4, 128, 32), (1, 3, 64, 16), (2, 5, 128, 16), (1, 6, 64, 16),
                                          (2, 2, 64, 4), (4, 4, 128, 4), (2, 7, 64, 8), (8, 4, 128, 8)])
def test_gqa_dims_and_block_sizes(hkv, grp, d, bs):
    lens = [1, 15, 16, 17, 300, 1000]
    q, k, v, tables, sl = _random_case(11 + grp + d + bs, len(lens), hkv, grp, d, bs, lens)
    scale = d**-0.5
    _check(_decode(q, k, v, tables, sl, scale, grp), oracle_out(q, k, v, tables, sl, scale, grp))


@pytest.mark.parametrize("hkv,grp,d,bs,bf16", [(2, 12, 128, 16, False), (1, 16, 64, 16, False), (2, 11, 64, 16, False),
                                                (1, 24, 128, 32, True), (4, 9, 64, 8, False), (1, 14, 64, 16, True)])
def test_gqa_groups_above_eight(hkv, grp, d, bs, bf16):
    # Groups above 8 run as virtual kv-heads (12 -> 2 x 6, 16 -> 2 x 8, 11 -> 11 x 1, 24 -> 3 x 8, 9 -> 3 x 3,
    # 14 -> 2 x 7); the result is still the oracle's over the pool head's K/V.
    lens = [1, 17, 300, 1000, 64]
    q, k, v, tables, sl = _random_case(41 + grp + d + bs, len(lens), hkv, grp, d, bs, lens)
    if bf16:
        q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    scale = d**-0.5
    got = _decode(q, k, v, tables, sl, scale, grp).float()
    want = oracle_out(q.float(), k.float(), v.float(), tables, sl, scale, grp)
    tol = 2e-2 if bf16 else 1e-2
    torch.testing.assert_close(got.cpu(), want.float().cpu().view_as(got), atol=tol, rtol=tol)


def test_zero_length_rows_and_table_clamp():
    lens = [0, 40, 0, 100]
    q, k, v, tables, sl = _random_case(21, 4, 2, 4, 64, 16, lens)
    out = _decode(q, k, v, tables, sl, 0.125, 4)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0
    _check(out, oracle_out(q, k, v, tables, sl, 0.125, 4))
    # seq_len beyond the table width: only max_blocks blocks are read.
    narrow = tables[:, :2].contiguous()
    clamp = _decode(q, k, v, narrow, sl, 0.125, 4)
    _check(clamp, oracle_out(q, k, v, narrow, sl, 0.125, 4))


def test_padding_entries_and_unused_blocks_never_read():
    lens = [5, 33, 130]
    q, k, v, tables, sl = _random_case(31, 3, 2, 4, 128, 16, lens, num_blocks=40, pad_value=-7)
    base = oracle_out(q, k, v, tables.clamp(min=0), sl, 0.0883, 4)
    used = set()
    for b, s in enumerate(lens):
        used.update(tables[b, :math.ceil(s / 16)].tolist())
    k2, v2 = k.clone(), v.clone()
    for blk in range(k.shape[0]):
        if blk not in used:
            k2[blk] = float("nan")
            v2[blk] = float("nan")
    out, err = _abi_decode(q, k2, v2, tables, sl, 0.0883, 4, 0)
    assert err == 0
    assert torch.isfinite(out.float()).all()
    _check(out, base)


def test_hook_contract():
    lens = [9, 70]
    q, k, v, tables, sl = _random_case(41, 2, 2, 4, 64, 16, lens)

    class Mod:
        num_key_value_groups = 4
        training = False

    meta = PagedDecodeBatchMetadata(pool=_Pool(k, v), layer_idx=0, block_tables=tables, seq_lens=sl)
    tok = set_paged_decode_batch_metadata(meta)
    try:
        out, weights = block_paged_attention_forward(Mod(), q, None, None, None, 0.125)
    finally:
        reset_paged_decode_batch_metadata(tok)
    assert weights is None and out.shape == (2, 1, 8, 64)
    _check(out.transpose(1, 2), oracle_out(q, k, v, tables, sl, 0.125, 4))


@pytest.mark.parametrize("d", [64, 128])
def test_stale_nan_past_sequence_end(d):
    """Slots past seq_len in a row's last block may hold anything a freed sequence (or an uninitialised pool)
    left there, NaN and Inf included: they never reach the output (the reference loads them masked to 0,
    paged_attention_triton.py:225-226)."""
    lens = [5, 33, 130, 16, 1]
    q, k, v, tables, sl = _random_case(51 + d, len(lens), 2, 4, d, 16, lens)
    base = oracle_out(q, k, v, tables, sl, d**-0.5, 4)
    k2, v2 = k.clone(), v.clone()
    for b, s in enumerate(lens):
        last = int(tables[b, (s - 1) // 16])
        if s % 16:
            k2[last, :, s % 16:] = float("nan")
            v2[last, :, s % 16:] = float("inf") if b % 2 else float("nan")
    for ct in (0, 16):
        out, err = _abi_decode(q, k2, v2, tables, sl, d**-0.5, 4, ct)
        assert err == 0
        assert torch.isfinite(out.float()).all(), f"chunk_tokens={ct}"
        _check(out, base, f"chunk_tokens={ct}")


@pytest.mark.parametrize("d,bs", [(128, 16), (64, 8), (128, 4), (64, 32)])
def test_block_ids_outside_the_pool(d, bs):
    """Table entries outside [0, num_pool_blocks) are skipped, never dereferenced: the error word
    gets bit 1, the output stays finite, a row with no block left is zeros, and every other row is
    the oracle over its in-pool blocks (oracle.paged_attention.decode_rows_fp32_valid). Covers a
    row's first block(s) out (the running max is still -inf when the first in-pool tile arrives),
    a block in the middle, the last block, and at block sizes 4 and 8 a whole 16-token tile of out
    blocks at the start of a piece (chunk_tokens 16 cuts every row into one-tile pieces)."""
    lens = [40, 64, 100, 37, 300, 77]
    grp = 4
    q, k, v, tables, sl = _random_case(61 + d + bs, len(lens), 2, grp, d, bs, lens)
    n_valid = int(k.shape[0])
    t = tables.clone()
    nblk = [math.ceil(s / bs) for s in lens]
    t[0, :nblk[0]] = n_valid + 5                      # every block out: zeros
    t[1, :max(1, 16 // bs)] = -1                     # the first tile's blocks out
    t[2, nblk[2] // 2] = n_valid                     # a block in the middle
    t[3, nblk[3] - 1] = 1 << 30                      # the last (partial) block
    t[4, 1:1 + max(1, 32 // bs)] = n_valid + 1       # two tiles' worth in the second piece
    scale = d**-0.5
    want = oracle_pa.decode_rows_fp32_valid(q.cpu(), k.cpu(), v.cpu(), t.cpu(), lens, scale, grp, n_valid)
    for ct in (0, 16):
        out, err = _abi_decode(q, k, v, t, sl, scale, grp, ct, num_pool_blocks=n_valid)
        assert err & 1, f"chunk_tokens={ct}: out-of-pool ids not flagged"
        assert torch.isfinite(out.float()).all(), f"chunk_tokens={ct}: non-finite output"
        assert torch.count_nonzero(out[0]) == 0
        _check(out, want, f"chunk_tokens={ct}")


def _config5_attention_case(seed=0):
    """Benchmark config 5's attention shape: 128 rows in 16 groups of 8, each group's rows longer than
    1024 tokens aliasing the group's 1024-token prefix blocks; contexts U[1, 8192]; Llama-3-8B heads
    (Hq 32, Hkv 8, D 128), block 16, a 40960-block pool with seeded block ids."""
    from runtime_amd.phase2.prefix_batch import PrefixBatch

    nb, bs, hkv, grp, d = 40960, 16, 8, 4, 128
    pb = PrefixBatch(batch=128, groups=16, prefix_tokens=1024, lo=1, hi=8192, block_size=bs, num_blocks=nb,
                     headroom=1, seed=seed)
    lens = pb.lens + 1  # the attention length counts the current token
    gd = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn(nb, hkv, bs, d, generator=gd, device="cuda", dtype=torch.float16)
    v = torch.randn(nb, hkv, bs, d, generator=gd, device="cuda", dtype=torch.float16)
    q = torch.randn(128, hkv * grp, 1, d, generator=gd, device="cuda", dtype=torch.float16)
    return pb, q, k, v, pb.tables.cuda(), lens.to(torch.int32).cuda(), grp, d**-0.5


@pytest.mark.timeout(600)
def test_config5_shared_prefix_full_shape():
    """Config 5 at its stated size under both K/V cache policies (streaming loads, and the default
    policy that MX_PA_SHARED_BLOCKS selects for aliased blocks): bit-identical to each other and
    within atol/rtol 1e-2 of the fp32 per-row oracle."""
    pb, q, k, v, tables, lens, grp, scale = _config5_attention_case()
    shared_rows = sum(r.shared > 0 for r in pb.rows)
    lens_h = lens.cpu().tolist()
    print(f"[config5] rows 128, sharing {shared_rows}, contexts {min(lens_h)}..{max(lens_h)}, "
          f"logical tokens {sum(lens_h)}, unique {pb.unique_tokens(1)}", flush=True)
    assert shared_rows >= 100 and max(lens_h) > 7000 and min(lens_h) < 1024
    shared, err1 = _abi_decode(q, k, v, tables, lens, scale, grp, 0, flags=1)
    stream, err0 = _abi_decode(q, k, v, tables, lens, scale, grp, 0)
    assert err0 == 0 and err1 == 0
    assert torch.equal(shared, stream)
    _check(shared, oracle_out(q, k, v, tables, lens_h, scale, grp))


@pytest.mark.parametrize("bsz,hq,hkv,d,bs,dtype", [
    (16, 14, 2, 64, 16, torch.float16),    # config 3 heads
    (32, 32, 8, 128, 16, torch.float16),   # config 2 heads
    (8, 16, 4, 128, 32, torch.bfloat16),   # block size 32 (2 tiles per block), bf16
    (72, 8, 2, 64, 16, torch.float16),     # more than 64 rows (the lengths are not read in one pass)
    (4, 24, 2, 64, 16, torch.float16),     # G = 12: virtual kv-heads
])
def test_tile_plan_matches_plain_calls(bsz, hq, hkv, d, bs, dtype):
    """MX_PA_PLAN_WRITE then MX_PA_PLAN_READ, as a decode step uses them (layer 0 records, the later
    layers start from the record): with the same lengths and tables, both calls equal the plain
    call bit for bit, for another query and another layer's K/V too, and no error bit is set.
    Rows of length 0, 1 and ones that fill their last block exactly are included."""
    from runtime_amd.phase2.paged_attention_hip import MX_PA_PLAN_READ, MX_PA_PLAN_WRITE
    from runtime_amd.phase2.paged_attention_hip import _decode as hip_decode

    grp = hq // hkv
    g = torch.Generator().manual_seed(bsz * 7 + d)
    lens = torch.randint(1, 1500, (bsz,), generator=g)
    lens[0], lens[1 % bsz] = 0, 1
    lens[2 % bsz] = 4 * bs
    print(f"[plan] B={bsz} Hq={hq} Hkv={hkv} D={d} bs={bs} {dtype}", flush=True)
    q, k, v, tables, seq_lens = _random_case(11, bsz, hkv, grp, d, bs, lens.tolist())
    k2, v2 = torch.randn_like(k.float()).to(dtype), torch.randn_like(v.float()).to(dtype)
    k, v, q = k.to(dtype), v.to(dtype), q.to(dtype)
    q2 = torch.randn_like(q.float()).to(dtype)
    scale = d ** -0.5
    dev = q.device
    before = workspace_error_flag(dev)
    plain1 = hip_decode(q, k, v, tables, seq_lens, scale, grp)
    plain2 = hip_decode(q2, k2, v2, tables, seq_lens, scale, grp)
    rec = hip_decode(q, k, v, tables, seq_lens, scale, grp, plan=MX_PA_PLAN_WRITE)
    read2 = hip_decode(q2, k2, v2, tables, seq_lens, scale, grp, plan=MX_PA_PLAN_READ)
    read1 = hip_decode(q, k, v, tables, seq_lens, scale, grp, plan=MX_PA_PLAN_READ)
    torch.cuda.synchronize()
    assert torch.equal(rec.view(torch.int16), plain1.view(torch.int16))
    assert torch.equal(read1.view(torch.int16), plain1.view(torch.int16))
    assert torch.equal(read2.view(torch.int16), plain2.view(torch.int16))
    assert (workspace_error_flag(dev) & ~before & 8) == 0
    if dtype == torch.float16:
        _check(read2, oracle_out(q2, k2, v2, tables, seq_lens, scale, grp), "plan read vs oracle")


@pytest.mark.parametrize("bsz,hq,hkv,d", [(8, 16, 4, 128), (16, 14, 2, 64)])
def test_tile_plan_with_many_pieces_per_segment(monkeypatch, bsz, hq, hkv, d):
    """Ranges of one 16-token tile (chunk_tokens 16): segments are cut into far more pieces than
    a merge window holds, so workers' first pieces reach the overflow slots, with and without the
    tile plan. Plain, recording and reading calls agree bit for bit and match the oracle."""
    from runtime_amd.phase2 import paged_attention_hip as pah

    monkeypatch.setattr(pah, "_CHUNK_TOKENS", 16)
    grp = hq // hkv
    g = torch.Generator().manual_seed(bsz + d)
    lens = torch.randint(200, 1500, (bsz,), generator=g).tolist()
    print(f"[plan] many pieces B={bsz} Hq={hq} Hkv={hkv} D={d}", flush=True)
    q, k, v, tables, seq_lens = _random_case(17, bsz, hkv, grp, d, 16, lens)
    scale = d ** -0.5
    plain = pah._decode(q, k, v, tables, seq_lens, scale, grp)
    rec = pah._decode(q, k, v, tables, seq_lens, scale, grp, plan=pah.MX_PA_PLAN_WRITE)
    read = pah._decode(q, k, v, tables, seq_lens, scale, grp, plan=pah.MX_PA_PLAN_READ)
    torch.cuda.synchronize()
    assert torch.equal(rec.view(torch.int16), plain.view(torch.int16))
    assert torch.equal(read.view(torch.int16), plain.view(torch.int16))
    assert (workspace_error_flag(q.device) & 8) == 0
    _check(plain, oracle_out(q, k, v, tables, seq_lens, scale, grp), "one-tile ranges vs oracle")


def test_tile_plan_flags_changed_lengths():
    """A MX_PA_PLAN_READ call whose lengths differ from the recording call: the pieces of the rows
    that changed are dropped and error bit 8 is set; nothing is read outside the pool (every
    plan entry is checked), and a plain call afterwards is still exact."""
    from runtime_amd.phase2.paged_attention_hip import MX_PA_PLAN_READ, MX_PA_PLAN_WRITE
    from runtime_amd.phase2.paged_attention_hip import _decode as hip_decode

    bsz, hkv, grp, d, bs = 6, 2, 4, 128, 16
    lens = [700, 33, 64, 1000, 5, 300]
    print("[plan] changed lengths", flush=True)
    q, k, v, tables, seq_lens = _random_case(5, bsz, hkv, grp, d, bs, lens)
    scale = d ** -0.5
    dev = q.device
    hip_decode(q, k, v, tables, seq_lens, scale, grp, plan=MX_PA_PLAN_WRITE)
    torch.cuda.synchronize()
    assert (workspace_error_flag(dev) & 8) == 0
    shorter = seq_lens.clone()
    shorter[0] -= 20  # still within the row's blocks: only the length check can catch it
    hip_decode(q, k, v, tables, shorter, scale, grp, plan=MX_PA_PLAN_READ)
    torch.cuda.synchronize()
    assert workspace_error_flag(dev) & 8
    out = hip_decode(q, k, v, tables, shorter, scale, grp)
    _check(out, oracle_out(q, k, v, tables, shorter, scale, grp), "plain call after a mismatched plan")
    # Clear the bit this test set on purpose, so later checks of the cached workspaces start clean.
    from runtime_amd.phase2 import paged_attention_hip as pah
    for key, ws in list(pah._workspaces.items()):
        off = int(_hip.load().mx_paged_attn_error_offset(*key[1:]))
        ws[off:off + 4].zero_()
    torch.cuda.synchronize()
    assert workspace_error_flag(dev) == 0


@pytest.mark.parametrize("d,bs,grp", [(128, 16, 4), (64, 16, 7), (128, 4, 4), (64, 32, 2)])
def test_interleaved_pool_layout_is_bit_identical(d, bs, grp):
    """The pool's default layout keeps each (block, kv-head)'s K and V runs adjacent in one tensor
    ([nb, Hkv, 2, bs, D]); the kernel reads strided views of it. The same K/V in that layout and in two
    separate tensors give the same bits, and the oracle's answer."""
    q, k, v, tables, lens = _random_case(21, 5, 2, grp, d, bs, [1, 40, 300, 2049, 0])
    kv = torch.empty(k.shape[0], k.shape[1], 2, bs, d, dtype=k.dtype, device=k.device)
    kv[:, :, 0] = k
    kv[:, :, 1] = v
    ki, vi = kv[:, :, 0], kv[:, :, 1]
    assert ki.stride() == vi.stride() == (k.shape[1] * 2 * bs * d, 2 * bs * d, d, 1)
    scale = d ** -0.5
    split = _decode(q, k, v, tables, lens, scale, grp)
    inter = _decode(q, ki, vi, tables, lens, scale, grp)
    assert torch.equal(split, inter)
    _check(inter, oracle_out(q, ki, vi, tables, lens, scale, grp))
    assert workspace_error_flag() == 0
