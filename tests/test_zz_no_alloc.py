"""mx_paged_attn_decode_noalloc (the workspace-free attention entry point) against
mx_paged_attn_decode, through the C ABI: bit-identical outputs on two calls in a row, the
second smaller than the first (the shared scratch keeps the first call's contents), errors
OR-ed into the caller's word, and shapes beyond the scratch refused before any launch."""

from __future__ import annotations

import math

import pytest
import torch

from runtime_amd.phase2 import _hip

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SCRATCH_BYTES = 32 << 20  # MX_PA_NOALLOC_SCRATCH_BYTES


def _case(seed, lens, hkv, grp, d, bs, num_blocks=None):
    g = torch.Generator().manual_seed(seed)
    nblk = [math.ceil(s / bs) for s in lens]
    nb = num_blocks or sum(nblk) + 5
    perm = torch.randperm(nb, generator=g)
    tables = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
    at = 0
    for b, n in enumerate(nblk):
        tables[b, :n] = perm[at:at + n].to(torch.int32)
        at += n
    gd = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn(nb, hkv, bs, d, generator=gd, device="cuda").half()
    v = torch.randn(nb, hkv, bs, d, generator=gd, device="cuda").half()
    q = torch.randn(len(lens), hkv * grp, 1, d, generator=gd, device="cuda").half()
    return q, k, v, tables.cuda(), torch.tensor(lens, dtype=torch.int32, device="cuda")


def _args(q, k, v, tables, lens):
    bsz, hq, _, d = q.shape
    nb, hkv, bs, _ = k.shape
    return (q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
            tables.data_ptr(), tables.stride(0), tables.shape[1], lens.data_ptr(), bsz, hq, hkv, d, bs, nb,
            d**-0.5)


def _with_workspace(q, k, v, tables, lens, flags=0):
    lib = _hip.load()
    bsz, hq, _, d = q.shape
    nb, hkv, bs, _ = k.shape
    nbytes = lib.mx_paged_attn_workspace_bytes(bsz, hq, hkv, d, tables.shape[1], bs, 0)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)
    _hip.check(lib.mx_paged_attn_decode(*_args(q, k, v, tables, lens), out.data_ptr(), out.stride(0), out.stride(1),
                                        ws.data_ptr(), nbytes, 0, flags, _hip.stream_handle(DEV)), "decode")
    return out, nbytes


def _noalloc(q, k, v, tables, lens, err=None, flags=0):
    lib = _hip.load()
    out = torch.full_like(q, float("nan"))
    _hip.check(lib.mx_paged_attn_decode_noalloc(*_args(q, k, v, tables, lens), out.data_ptr(), out.stride(0),
                                                out.stride(1), 0, flags, err.data_ptr() if err is not None else None,
                                                _hip.stream_handle(DEV)), "decode_noalloc")
    return out


def test_noalloc_equals_workspace_entry_two_calls():
    # Call 1: benchmark config 2 (32 rows, GQA 4, D 128, contexts U[128, 4096], 16384-block pool).
    g = torch.Generator().manual_seed(0)
    lens1 = torch.randint(128, 4097, (32,), generator=g).tolist()
    big = _case(0, lens1, 8, 4, 128, 16, num_blocks=16384)
    want1, nbytes1 = _with_workspace(*big)
    got1 = _noalloc(*big)
    # Call 2, smaller: 3 rows, GQA 7, D 64, block 16, with a block id outside the pool.
    small = _case(1, [40, 1, 300], 2, 7, 64, 16)
    q, k, v, tables, lens = small
    tables = tables.clone()
    tables[2, 3] = k.shape[0] + 2
    want2, nbytes2 = _with_workspace(q, k, v, tables, lens)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    got2 = _noalloc(q, k, v, tables, lens, err=err)
    torch.cuda.synchronize()
    assert nbytes2 < nbytes1 <= SCRATCH_BYTES
    assert torch.equal(got1, want1)
    assert torch.equal(got2, want2)
    assert int(err.item()) & 1
    # The first shape again after the smaller one, shared-blocks flag: same bits as the workspace entry.
    assert torch.equal(_noalloc(*big, flags=1), _with_workspace(*big, flags=1)[0])


def test_noalloc_refuses_shapes_beyond_its_scratch():
    lib = _hip.load()
    q, k, v, tables, lens = _case(2, [16], 8, 4, 128, 16)
    wide = torch.zeros(512, 2048, dtype=torch.int32, device=DEV)
    rows = torch.ones(512, dtype=torch.int32, device=DEV)
    qq = torch.zeros(512, 32, 1, 128, dtype=torch.float16, device=DEV)
    assert lib.mx_paged_attn_workspace_bytes(512, 32, 8, 128, 2048, 16, 0) > SCRATCH_BYTES
    out = torch.zeros_like(qq)
    rc = lib.mx_paged_attn_decode_noalloc(*_args(qq, k, v, wide, rows), out.data_ptr(), out.stride(0), out.stride(1),
                                          0, 0, None, _hip.stream_handle(DEV))
    assert rc == _hip.MX_ERR_WORKSPACE
    assert b"scratch" in lib.mx_last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0  # nothing was launched
