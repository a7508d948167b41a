"""Host logic of the shared-prefix batch (block allocator, aliasing, join/finish, byte counts)."""

from __future__ import annotations

import pytest
import torch

from runtime_amd.phase2.prefix_batch import BlockAllocator, PrefixBatch


def test_allocator_refcounts_and_errors():
    a = BlockAllocator(8, seed=3)
    ids = a.alloc(3)
    assert len(set(ids)) == 3 and a.free_blocks == 5
    a.incref(ids[:1])
    a.decref(ids)
    assert a.free_blocks == 7 and a.refcount(ids[0]) == 1
    a.decref(ids[:1])
    assert a.free_blocks == 8
    with pytest.raises(RuntimeError):
        a.decref(ids[:1])  # freed twice
    with pytest.raises(RuntimeError):
        a.alloc(9)
    with pytest.raises(RuntimeError):
        a.incref([ids[1]])  # not allocated


def _batch(**kw):
    args = dict(batch=16, groups=2, prefix_tokens=64, lo=1, hi=200, block_size=16, num_blocks=400, headroom=20, seed=5)
    args.update(kw)
    return PrefixBatch(**args)


def test_rows_of_a_group_alias_the_prefix_blocks():
    pb = _batch()
    t, lens = pb.tables, pb.lens
    assert t.shape == (16, pb.max_blocks) and lens.dtype == torch.int32
    for b, r in enumerate(pb.rows):
        assert r.group == b // 8
        n = -(-(int(lens[b]) + pb.headroom) // 16)
        assert t[b, :n].tolist() == r.blocks and (t[b, n:] == 0).all()
        if r.length > 64:
            assert r.blocks[:4] == pb.prefix_blocks[r.group] and r.shared == 4
        else:
            assert r.shared == 0 and not set(r.blocks) & set(pb.prefix_blocks[r.group])
    # Private blocks are never shared between rows.
    private = [blk for r in pb.rows for blk in r.blocks[r.shared:]]
    assert len(private) == len(set(private))


def test_unique_tokens_against_brute_force():
    pb = _batch(lo=40, hi=300)
    for extra in (0, 1, 7):
        slots = set()
        for r in pb.rows:
            for pos in range(r.length + extra):
                slots.add((r.blocks[pos // 16], pos % 16))
        assert pb.unique_tokens(extra) == len(slots)
        assert pb.logical_tokens(extra) == sum(r.length + extra for r in pb.rows)
    assert pb.unique_tokens() < pb.logical_tokens()


def test_rotate_frees_private_blocks_and_keeps_the_prefix():
    pb = _batch(lo=100, hi=150)  # every row shares its group's prefix
    pre = pb.prefix_blocks[0]
    assert all(pb.alloc.refcount(i) == 1 + 8 for i in pre)  # the group + 8 rows
    old = [pb.rows[b].blocks[4:] for b in (0, 3)]
    pb.rotate([0, 3], lengths=[120, 20])
    assert pb.rows[0].blocks[:4] == pre and pb.rows[0].length == 120
    assert pb.rows[3].shared == 0 and pb.rows[3].length == 20  # too short to share
    assert all(pb.alloc.refcount(i) == 1 + 7 for i in pre)
    for ids in old:
        assert all(pb.alloc.refcount(i) in (0, 1) for i in ids)
    used_now = sum(len(r.blocks) - r.shared for r in pb.rows)
    assert pb.alloc.free_blocks == 400 - used_now - 2 * 4


def test_advance_past_the_headroom_raises():
    pb = _batch(headroom=4)
    pb.advance(4)
    with pytest.raises(RuntimeError):
        pb.advance(16)


def test_upload_keeps_device_tensor_addresses():
    pb = _batch()
    tables_d = torch.empty(16, pb.max_blocks, dtype=torch.int32)
    lens_d = torch.empty(16, dtype=torch.int32)
    p0, p1 = tables_d.data_ptr(), lens_d.data_ptr()
    pb.rotate([1, 9])
    pb.upload(tables_d, lens_d)
    assert (tables_d.data_ptr(), lens_d.data_ptr()) == (p0, p1)
    assert torch.equal(tables_d, pb.tables) and torch.equal(lens_d, pb.lens)


def test_upload_rows_equals_full_upload():
    """After a rotation, rewriting only the refilled rows gives the full table; stale entries past a
    refilled row's new blocks are cleared."""
    pb = _batch()
    tables_d = torch.empty(16, pb.max_blocks, dtype=torch.int32)
    lens_d = torch.empty(16, dtype=torch.int32)
    pb.upload(tables_d, lens_d)
    for k in range(1, 4):
        rows = [b for b in range(16) if b % 4 == k]
        pb.advance(2)
        pb.rotate(rows, lengths=[5 + 60 * j for j in range(len(rows))])
        pb.upload_rows(rows, tables_d, lens_d)
        assert torch.equal(tables_d, pb.tables) and torch.equal(lens_d, pb.lens)
    pb.upload_rows([], tables_d, lens_d)
    assert torch.equal(lens_d, pb.lens)


def test_given_lengths():
    pb = _batch(lengths=[70 + b for b in range(16)])
    assert pb.lens.tolist() == [70 + b for b in range(16)]
    with pytest.raises(ValueError):
        _batch(lengths=[70])


def test_bad_arguments():
    with pytest.raises(ValueError):
        _batch(batch=15)
    with pytest.raises(ValueError):
        _batch(prefix_tokens=60)
    with pytest.raises(ValueError):
        _batch(lo=0)
