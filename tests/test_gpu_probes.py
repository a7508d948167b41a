"""The calibration probes behind ``bench.py --workload probes`` (``csrc/probes.hip``) on the GPU:
each reads or writes exactly what it is asked to and nothing else."""

from __future__ import annotations

import pytest
import torch

from runtime_amd.phase2 import _hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_launch_probe_writes_its_share_and_nothing_more():
    lib = _hip.load()
    dst = torch.zeros(1 << 20, dtype=torch.uint8, device=DEV)
    st = _hip.stream_handle(DEV)
    _hip.check(lib.mx_launch_probe(dst.data_ptr(), dst.numel(), 64 * 1024, 16, st), "mx_launch_probe")
    _hip.check(lib.mx_launch_probe(None, 0, 0, 256, st), "mx_launch_probe")  # empty launch
    torch.cuda.synchronize()
    words = dst.view(torch.int32)
    want = torch.arange(16, dtype=torch.int32, device=DEV).repeat_interleave(64 * 1024 // 16 // 4)
    assert torch.equal(words[: want.numel()], want)  # workgroup w wrote w into its 4 KiB share
    assert int(words[want.numel():].abs().sum()) == 0


def test_stream_and_gather_probes_write_nothing():
    lib = _hip.load()
    src = torch.randint(0, 255, (8 << 20,), dtype=torch.uint8, device=DEV)
    sink = torch.zeros(2, dtype=torch.int32, device=DEV)
    st = _hip.stream_handle(DEV)
    before = src.clone()
    for threads in (256, 512, 1024):
        _hip.check(lib.mx_stream_probe(src.data_ptr(), src.numel(), 4096, 64 * 1024, 32, threads, sink.data_ptr(), st),
                   "mx_stream_probe")
    offs = (torch.randperm(1000, device=DEV)[:300] * 8192).to(torch.int64)
    offs[0] = -1  # out of range: read as run 0
    offs[1] = 1 << 40
    for pattern, inflight, streaming in ((0, 1, 1), (0, 2, 0), (0, 3, 1), (0, 6, 1), (1, 2, 1), (2, 2, 1), (3, 2, 1), (4, 2, 1)):
        _hip.check(lib.mx_run_gather_probe(src.data_ptr(), src.numel(), offs.data_ptr(), offs.numel(), 8192, 64,
                                           inflight, streaming, pattern, sink.data_ptr(), st), "mx_run_gather_probe")
    torch.cuda.synchronize()
    assert torch.equal(src, before)
    # the sink is stored only when a load sum hits the magic value, and only its first word
    assert int(sink[1]) == 0 and int(sink[0]) in (0, 0x9E3779B9 - (1 << 32))


def _handoff_want(workgroups: int, group: int) -> tuple[torch.Tensor, torch.Tensor]:
    """out[g][i] = sum over the group's workgroups w of (31 w + i) & 1023 (exact in fp32)."""
    w = torch.arange(workgroups, dtype=torch.int64)[:, None]
    i = torch.arange(2048, dtype=torch.int64)[None, :]
    part = ((31 * w + i) & 1023).to(torch.float32)
    return part, part.view(workgroups // group, group, 2048).sum(1)


@pytest.mark.parametrize("workgroups,group", [(256, 4), (1024, 8), (512, 16)])
def test_handoff_probe_sums_every_group(workgroups, group):
    """Every mode hands each group's partials to one summing workgroup (or launch), on two calls in a
    row: the tickets are left at zero for the next call."""
    lib = _hip.load()
    st = _hip.stream_handle(DEV)
    part = torch.full((workgroups, 2048), float("nan"), dtype=torch.float32, device=DEV)
    out = torch.full((workgroups // group, 2048), float("nan"), dtype=torch.float32, device=DEV)
    tickets = torch.zeros(workgroups // group, dtype=torch.int32, device=DEV)
    want_part, want_out = _handoff_want(workgroups, group)
    for mode in (0, 1, 2, 3, 4, 4, 2):
        print(f"handoff probe mode {mode}: {workgroups} workgroups, groups of {group}", flush=True)
        out.fill_(float("nan"))
        _hip.check(lib.mx_handoff_probe(part.data_ptr(), part.numel() * 4, out.data_ptr(), out.numel() * 4,
                                        tickets.data_ptr(), tickets.numel() * 4, workgroups, group, mode, st),
                   "mx_handoff_probe")
        torch.cuda.synchronize()
        assert torch.equal(part.cpu(), want_part)
        if mode == 0:
            assert bool(out.isnan().all())
        else:
            assert torch.equal(out.cpu(), want_out)
        assert int(tickets.abs().sum()) == 0


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
def test_barrier_probe_passes_every_round(mode):
    """256 resident workgroups pass 64 grid barriers of each kind, twice in a row, with no time-out
    and (modes 3, 4) every hand-off read holding the round's value; the sync words end at zero."""
    lib = _hip.load()
    st = _hip.stream_handle(DEV)
    n = 256
    sync = torch.zeros(16 + n, dtype=torch.int32, device=DEV)
    hand = torch.zeros(2 * n * 256, dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    for rounds in (64, 0, 5):
        print(f"barrier probe mode {mode}: {n} workgroups, {rounds} rounds", flush=True)
        _hip.check(lib.mx_barrier_probe(sync.data_ptr(), sync.numel() * 4, hand.data_ptr(), hand.numel() * 4, n, rounds,
                                        mode, err.data_ptr(), st), "mx_barrier_probe")
        torch.cuda.synchronize()
        assert int(err) == 0
        assert int(sync.abs().sum()) == 0
    if mode >= 3:  # the last round (4) of each workgroup w wrote 4 n + w + 1 into slot 0
        last = hand.view(2, n, 256)[0].cpu()
        assert torch.equal(last, (4 * n + torch.arange(n, dtype=torch.int32) + 1)[:, None].expand(n, 256))


@pytest.mark.parametrize("persistent", [0, 1])
@pytest.mark.parametrize("per_wg", [8 << 10, 64 << 10])
def test_chain_probe_hands_every_phase_on(persistent, per_wg):
    """Eight phases, as one call per phase (the graph of kernels) or one persistent launch: each
    phase reads the value the previous one handed over (err bit 2 otherwise) and the last phase's
    slot holds 8; the source is only read, and the persistent launch leaves its sync words at zero."""
    lib = _hip.load()
    st = _hip.stream_handle(DEV)
    n, phases = 256, 8
    src = torch.randint(0, 255, (phases * n * per_wg,), dtype=torch.uint8, device=DEV)
    before = src.clone()
    sync = torch.zeros(16, dtype=torch.int32, device=DEV)
    hand = torch.zeros(2 * n * 256, dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    sink = torch.zeros(1, dtype=torch.int32, device=DEV)
    for rep in range(2):
        print(f"chain probe persistent={persistent} per_wg={per_wg} call {rep}", flush=True)
        calls = [(0, phases)] if persistent else [(p, 1) for p in range(phases)]
        for p0, count in calls:
            _hip.check(lib.mx_chain_probe(src.data_ptr(), src.numel(), per_wg, n, p0, count, persistent,
                                          sync.data_ptr(), sync.numel() * 4, hand.data_ptr(), hand.numel() * 4,
                                          err.data_ptr(), sink.data_ptr(), st), "mx_chain_probe")
        torch.cuda.synchronize()
        assert int(err) == 0
        assert int(sync.abs().sum()) == 0
        assert bool((hand.view(2, n, 256)[(phases - 1) & 1] == phases).all())
    assert torch.equal(src, before)
