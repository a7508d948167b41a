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
