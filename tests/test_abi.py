"""CPU checks of the C ABI: the library loads, exports what the header declares,
and rejects bad arguments with status codes before touching the device."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from runtime_amd.phase2 import _hip
from runtime_amd.phase2.int8_linear import Int8Linear, int8_linear

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "mxdecode.h")


def _declared() -> list[str]:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(mx_\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _hip.load()
    names = _declared()
    assert "mx_paged_attn_decode" in names and "mx_w8a16_linear" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_hip.SIGNATURES), "ctypes prototypes must mirror the header"
    assert lib.mx_abi_version() == _hip.ABI_VERSION


def test_paged_attn_workspace_layout_is_host_computable():
    lib = _hip.load()
    small = lib.mx_paged_attn_workspace_bytes(4, 8, 2, 64, 8, 16, 0)
    big = lib.mx_paged_attn_workspace_bytes(32, 32, 8, 128, 256, 16, 256)
    assert 0 < small < big
    # Partial slots (fp32 m, l and a 16-bit output of D per head, G heads): a window of U per
    # segment and one overflow slot per worker. 65536 tiles at the table width in ranges of 16
    # tiles -> 4096 workers over 256 segments, more than 10 per segment -> U = 32.
    # Block size 16 also holds the tile plan of MX_PA_PLAN_WRITE / MX_PA_PLAN_READ: 64 entries and
    # a header of 16 bytes per worker; block sizes 4 and 8 have none.
    slots = 256 * 32 + 4096
    plan = 4096 * 65 * 16
    assert big >= slots * 4 * (2 * 4 + 128 * 2) + plan
    assert big < slots * 4 * (2 * 4 + 128 * 4) + plan  # half the bytes of an fp32 accumulator
    w8 = lib.mx_paged_attn_workspace_bytes(32, 32, 8, 128, 512, 8, 256)  # same tiles and workers, no plan
    assert w8 + plan == big
    assert lib.mx_paged_attn_workspace_bytes(32, 32, 8, 128, 256, 16, 512) < big
    # Default split: 2048 workers for config 2's table (ranges of 32 tiles = 512 tokens at full
    # width); a single short row gets ranges of 4 tiles (64 tokens).
    assert lib.mx_paged_attn_workspace_bytes(32, 32, 8, 128, 256, 16, 0) == \
        lib.mx_paged_attn_workspace_bytes(32, 32, 8, 128, 256, 16, 512)
    assert lib.mx_paged_attn_workspace_bytes(1, 8, 2, 64, 8, 16, 0) == \
        lib.mx_paged_attn_workspace_bytes(1, 8, 2, 64, 8, 16, 64)
    assert lib.mx_paged_attn_error_offset(4, 8, 2, 64, 8, 16, 0) % 256 == 0
    # Split-K partials when the n-groups (4 n-tiles of 16 channels each) alone would leave
    # fewer than 256 workgroups: qkv, o and down at M=32 split K 8 ways; gate_up (448
    # groups) and the GEMV (M <= 4) do not. o and down (64 groups) pair their 8 k ranges
    # into 2 parts of one workgroup (256 workgroups, one round) and write 4 partials; qkv
    # (96 groups: 384 paired workgroups) writes 8.
    assert lib.mx_w8a16_workspace_bytes(32, 4096, 14336) == 4 * 32 * 4096 * 4
    assert lib.mx_w8a16_workspace_bytes(32, 4096, 4096) == 4 * 32 * 4096 * 4
    assert lib.mx_w8a16_workspace_bytes(32, 6144, 4096) == 8 * 32 * 6144 * 4
    assert lib.mx_w8a16_workspace_bytes(32, 28672, 4096) == 0
    assert lib.mx_w8a16_workspace_bytes(1, 4096, 14336) == 0
    assert [lib.mx_w8a16_splits(32, n, k) for n, k in ((6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336))] \
        == [8, 4, 1, 4]
    # GEMV rows (M <= 4) never split; rows run in chunks of at most 128, and above one
    # chunk there is no partials entry, so splits reports 1.
    assert lib.mx_w8a16_splits(4, 4096, 4096) == 1 and lib.mx_w8a16_splits(65, 4096, 4096) == 8
    assert lib.mx_w8a16_splits(128, 4096, 4096) == 8 and lib.mx_w8a16_splits(129, 4096, 4096) == 1
    assert lib.mx_w8a16_workspace_bytes(200, 4096, 14336) == lib.mx_w8a16_workspace_bytes(128, 4096, 14336)
    assert lib.mx_w8a16_workspace_bytes(128, 4096, 14336) == 8 * 128 * 4096 * 4


def _status(rc: int, expected: int) -> None:
    assert rc == expected, (rc, _hip.load().mx_last_error())
    assert _hip.load().mx_last_error().decode()


def test_invalid_arguments_return_status_codes():
    lib = _hip.load()
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    _status(lib.mx_w8a16_linear(None, 1, 64, 64, fake, fake, None, fake, 16, 16, None, 0, None), _hip.MX_ERR_NULL)
    _status(lib.mx_w8a16_linear(fake, 1, 60, 64, fake, fake, None, fake, 16, 16, None, 0, None),
            _hip.MX_ERR_UNSUPPORTED)
    _status(lib.mx_w8a16_linear(fake, 1, 64, 32, fake, fake, None, fake, 16, 16, None, 0, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_w8a16_linear(ctypes.c_void_p(4098), 1, 64, 64, fake, fake, None, fake, 16, 16, None, 0, None),
            _hip.MX_ERR_ALIGNMENT)
    _status(lib.mx_w8a16_pack(fake, 15, 64, fake, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_w8a16_quantize(None, 4, 4, fake, fake, None), _hip.MX_ERR_NULL)
    args = dict(q=fake, q_sb=256, q_sh=64, k=fake, v=fake, kv_sblk=2048, kv_shead=1024, bt=fake, bt_sb=4, mb=4,
                sl=fake, B=1, Hq=8, Hkv=2, D=64, bs=16, npool=8, scale=0.125, out=fake, o_sb=512, o_sh=64,
                ws=None, wsb=0, ct=0, flags=0, st=None)

    def call(**over):
        a = dict(args, **over)
        return lib.mx_paged_attn_decode(a["q"], a["q_sb"], a["q_sh"], a["k"], a["v"], a["kv_sblk"], a["kv_shead"],
                                        a["bt"], a["bt_sb"], a["mb"], a["sl"], a["B"], a["Hq"], a["Hkv"], a["D"],
                                        a["bs"], a["npool"], a["scale"], a["out"], a["o_sb"], a["o_sh"], a["ws"],
                                        a["wsb"], a["ct"], a["flags"], a["st"])

    assert call(B=0) == _hip.MX_OK
    _status(call(q=None), _hip.MX_ERR_NULL)
    _status(call(Hq=7), _hip.MX_ERR_INVALID)
    # G = 18 passes validation (3 virtual kv-heads of 6 query heads per pool head) and stops at the
    # missing workspace, which is sized like the 6-kv-head layout.
    _status(call(Hq=36, Hkv=2), _hip.MX_ERR_WORKSPACE)
    assert lib.mx_paged_attn_workspace_bytes(4, 36, 2, 64, 8, 16, 0) == lib.mx_paged_attn_workspace_bytes(4, 36, 6, 64, 8, 16, 0)
    assert lib.mx_paged_attn_workspace_bytes(4, 22, 2, 64, 8, 16, 0) == lib.mx_paged_attn_workspace_bytes(4, 22, 22, 64, 8, 16, 0)
    _status(call(D=96), _hip.MX_ERR_UNSUPPORTED)
    _status(call(bs=12), _hip.MX_ERR_UNSUPPORTED)
    _status(call(ct=40), _hip.MX_ERR_INVALID)
    _status(call(ct=2048), _hip.MX_ERR_INVALID)  # split granularity is at most 64 tiles
    _status(call(flags=16), _hip.MX_ERR_INVALID)  # bits 0-3 are the defined flags
    _status(call(flags=4 | 8), _hip.MX_ERR_INVALID)  # PLAN_WRITE and PLAN_READ exclude each other
    _status(call(flags=8, bs=8), _hip.MX_ERR_UNSUPPORTED)  # the tile plan needs block_size >= 16
    _status(call(flags=4 | 1), _hip.MX_ERR_UNSUPPORTED)  # ... and no MX_PA_SHARED_BLOCKS
    _status(call(flags=4), _hip.MX_ERR_WORKSPACE)
    # The workspace-free entry point has no room for the plan (checked before it touches a device).
    a = args
    _status(lib.mx_paged_attn_decode_noalloc(a["q"], a["q_sb"], a["q_sh"], a["k"], a["v"], a["kv_sblk"],
                                             a["kv_shead"], a["bt"], a["bt_sb"], a["mb"], a["sl"], a["B"], a["Hq"],
                                             a["Hkv"], a["D"], a["bs"], a["npool"], a["scale"], a["out"], a["o_sb"],
                                             a["o_sh"], a["ct"], 8, None, a["st"]), _hip.MX_ERR_INVALID)
    _status(call(), _hip.MX_ERR_WORKSPACE)
    _status(call(q_sh=60), _hip.MX_ERR_ALIGNMENT)
    # Chunked argmax: the key workspace is M x ceil(N / 4096) x 8 bytes, and every argument is
    # checked before anything is launched.
    assert lib.mx_argmax_workspace_bytes(16, 151936) == 16 * 38 * 8
    assert lib.mx_argmax_workspace_bytes(1, 4096) == 8 and lib.mx_argmax_workspace_bytes(1, 4097) == 16
    assert lib.mx_argmax_workspace_bytes(0, 10) == 0
    assert lib.mx_argmax_rows_split(fake, 64, 0, 64, fake, None, None, 0, None) == _hip.MX_OK
    _status(lib.mx_argmax_rows_split(fake, 64, 2, 64, fake, None, None, 0, None), _hip.MX_ERR_NULL)
    _status(lib.mx_argmax_rows_split(fake, 64, 2, 64, fake, None, fake, 8, None), _hip.MX_ERR_WORKSPACE)
    _status(lib.mx_argmax_rows_split(fake, 60, 2, 60, fake, None, fake, 64, None), _hip.MX_ERR_ALIGNMENT)
    _status(lib.mx_argmax_rows_split(fake, 64, 2, 0, fake, None, fake, 64, None), _hip.MX_ERR_INVALID)
    with pytest.raises(ValueError):
        _hip.check(_hip.MX_ERR_INVALID, "probe")
    with pytest.raises(RuntimeError):
        _hip.check(_hip.MX_ERR_LAUNCH, "probe")


def test_python_wrappers_refuse_cpu_tensors():
    """No CPU fallback: host tensors are rejected before any launch."""
    from runtime_amd.phase2.paged_attention_hip import PagedDecodeBatchMetadata, paged_attention_decode_batched
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    with pytest.raises(ValueError):
        int8_linear(torch.zeros(1, 64, dtype=torch.float16), torch.zeros(1024, dtype=torch.uint8),
                    torch.ones(16, dtype=torch.float16), None, 16)
    pool = GpuKVBlockPool(num_blocks=2, block_size_tokens=16, num_layers=1, num_kv_heads=1, head_dim=64,
                          dtype=torch.float16, device="cpu")
    meta = PagedDecodeBatchMetadata(pool=pool, layer_idx=0, block_tables=torch.zeros(1, 1, dtype=torch.int32),
                                    seq_lens=torch.ones(1, dtype=torch.int32))
    with pytest.raises(ValueError):
        paged_attention_decode_batched(torch.zeros(1, 2, 1, 64, dtype=torch.float16), meta, 2, 0.125)
    with pytest.raises(ValueError):
        Int8Linear(100, 64)
    with pytest.raises(ValueError):
        Int8Linear.from_linear(torch.nn.Linear(64, 16), device="cpu")


def test_calibration_probes_reject_bad_arguments():
    """The probes check every range on the host before a launch (nothing here reaches the device)."""
    lib = _hip.load()
    fake = ctypes.c_void_p(1 << 20)
    _status(lib.mx_stream_probe(None, 1 << 20, 0, 4096, 1, 256, fake, None), _hip.MX_ERR_NULL)
    _status(lib.mx_stream_probe(fake, 1 << 20, 0, 4096, 1, 256, None, None), _hip.MX_ERR_NULL)
    _status(lib.mx_stream_probe(fake, 1 << 20, 0, 4008, 1, 256, fake, None), _hip.MX_ERR_INVALID)  # not 16-byte
    _status(lib.mx_stream_probe(fake, 1 << 20, 16, 1 << 20, 1, 256, fake, None), _hip.MX_ERR_INVALID)  # past the end
    _status(lib.mx_stream_probe(fake, 1 << 20, 0, 4096, 0, 256, fake, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_stream_probe(fake, 1 << 20, 0, 4096, 1, 128, fake, None), _hip.MX_ERR_UNSUPPORTED)
    _status(lib.mx_launch_probe(fake, 1 << 20, 100, 2, None), _hip.MX_ERR_INVALID)  # not 16 x workgroups
    _status(lib.mx_launch_probe(fake, 1 << 20, 2 << 20, 2, None), _hip.MX_ERR_INVALID)  # past the end
    _status(lib.mx_launch_probe(None, 1 << 20, 4096, 2, None), _hip.MX_ERR_NULL)
    _status(lib.mx_launch_probe(None, 0, 0, 0, None), _hip.MX_ERR_INVALID)
    # hand-off, barrier and chain probes: argument checks that come before any device query
    kb = 8 << 10
    _status(lib.mx_handoff_probe(fake, 256 * kb, fake, 64 * kb, fake, 256, 256, 4, 5, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_handoff_probe(fake, 256 * kb, fake, 64 * kb, fake, 256, 250, 4, 2, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_handoff_probe(None, 256 * kb, fake, 64 * kb, fake, 256, 256, 4, 2, None), _hip.MX_ERR_NULL)
    _status(lib.mx_handoff_probe(fake, 256 * kb, fake, 64 * kb, None, 256, 256, 4, 2, None), _hip.MX_ERR_NULL)
    _status(lib.mx_handoff_probe(fake, 255 * kb, fake, 64 * kb, fake, 256, 256, 4, 2, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_handoff_probe(fake, 256 * kb, fake, 64 * kb, fake, 252, 256, 4, 2, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_handoff_probe(ctypes.c_void_p((1 << 20) + 4), 256 * kb, fake, 64 * kb, fake, 256, 256, 4, 2, None),
            _hip.MX_ERR_ALIGNMENT)
    _status(lib.mx_barrier_probe(fake, 4096, fake, 1 << 20, 256, 10, 5, fake, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_barrier_probe(None, 4096, fake, 1 << 20, 256, 10, 0, fake, None), _hip.MX_ERR_NULL)
    _status(lib.mx_barrier_probe(fake, 4096, None, 1 << 20, 256, 10, 3, fake, None), _hip.MX_ERR_NULL)
    _status(lib.mx_barrier_probe(fake, 4096, fake, 1 << 20, 256, 10, 0, None, None), _hip.MX_ERR_NULL)
    _status(lib.mx_barrier_probe(fake, 4096, fake, 1 << 20, 256, -1, 0, fake, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_barrier_probe(fake, 4096, fake, 1 << 20, 0, 10, 0, fake, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_barrier_probe(fake, 4 * 271, fake, 1 << 20, 256, 10, 1, fake, None), _hip.MX_ERR_INVALID)
    _status(lib.mx_barrier_probe(fake, 4096, fake, 256 * 2048 - 16, 256, 10, 3, fake, None), _hip.MX_ERR_INVALID)

    def chain(src_bytes=8 * 256 * kb, per=kb, wgs=256, p0=0, phases=8, persistent=0, hand=fake, sync=fake):
        return lib.mx_chain_probe(fake, src_bytes, per, wgs, p0, phases, persistent, sync, 64, hand, 256 * 2048, fake,
                                  fake, None)

    _status(chain(phases=0), _hip.MX_ERR_INVALID)
    _status(chain(per=kb + 8), _hip.MX_ERR_INVALID)  # not 16-byte
    _status(chain(src_bytes=8 * 256 * kb - 16), _hip.MX_ERR_INVALID)  # past the end
    _status(chain(p0=1, phases=7, persistent=1), _hip.MX_ERR_INVALID)  # a persistent launch starts at phase 0
    _status(chain(hand=None), _hip.MX_ERR_NULL)
    _status(chain(sync=None, persistent=1), _hip.MX_ERR_NULL)


def test_fused_mlp_rejects_bad_arguments():
    """mx_w8a16_mlp_fused_partials refuses null pointers and shapes outside its plan on the host,
    before anything reaches the device."""
    lib = _hip.load()
    f = ctypes.c_void_p(1 << 20)
    k, i, n = 4096, 14336, 4096  # the Llama-3-8B MLP, which the fused launch takes at 5..32 rows

    def call(x=f, m=32, kk=k, ii=i, nn=n, act=f, part=f, sync=f):
        return lib.mx_w8a16_mlp_fused_partials(x, m, kk, kk, f, f, None, ii, act, ii, f, f, nn, part, 1 << 30, sync,
                                               None)

    _status(call(x=None), _hip.MX_ERR_NULL)
    _status(call(sync=None), _hip.MX_ERR_NULL)
    _status(call(part=None), _hip.MX_ERR_NULL)
    _status(call(m=4), _hip.MX_ERR_UNSUPPORTED)   # the VALU GEMV's rows
    _status(call(m=33), _hip.MX_ERR_UNSUPPORTED)  # three m-tiles
    _status(call(kk=4000), _hip.MX_ERR_UNSUPPORTED)
    _status(call(ii=14336 + 32), _hip.MX_ERR_UNSUPPORTED)  # gate||up groups of 64 channels
    _status(call(kk=1024, ii=4096, nn=1024), _hip.MX_ERR_UNSUPPORTED)  # gate||up would split K there
    assert lib.mx_w8a16_mlp_fused_supported(4, k, i, n) == 0
    assert lib.mx_w8a16_mlp_fused_supported(48, k, i, n) == 0
