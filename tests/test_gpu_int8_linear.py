"""GPU parity of the int8 quantize / pack / linear kernels against the CPU oracle.

Bar: quantize and pack bit-exact; fp16 linear outputs within atol 1e-2 and
rtol 1e-2 of the fp32-accumulated oracle (oracle/int8_quant.py).
"""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import int8_quant
from runtime_amd.phase2.int8_linear import Int8Linear, int8_linear, pack_weight, quantize_model_, quantize_weight

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
ATOL = 1e-2
RTOL = 1e-2


def _cuda(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _quantized(seed: int, n: int, k: int, scale: float = 0.02):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * scale).numpy().astype(np.float32)
    q, s = int8_quant.quantize_per_channel(w)
    return q, s


def test_quantize_and_pack_bit_exact_on_edge_rows():
    d = np.load(os.path.join(GOLDEN, "int8_edge.npz"))
    q, s = quantize_weight(_cuda(d["w"]))
    assert np.array_equal(q.cpu().numpy(), d["q"])
    assert np.array_equal(s.cpu().numpy().view(np.uint16), d["s"].view(np.uint16))
    assert np.array_equal(pack_weight(q).cpu().numpy(), d["packed"])


def test_quantize_rejects_non_finite():
    w = torch.zeros(16, 64, device="cuda")
    w[3, 5] = float("inf")
    with pytest.raises(ValueError):
        quantize_weight(w)


def test_quantize_and_pack_bit_exact_config1():
    doc = json.load(open(os.path.join(GOLDEN, "int8_config1.json")))
    g = torch.Generator().manual_seed(0)
    torch.randn(1, 4096, generator=g)
    w = torch.randn(4096, 4096, generator=g) * 0.02
    q, s = quantize_weight(w.cuda())
    qn, sn = q.cpu().numpy(), s.cpu().numpy()
    assert hashlib.sha256(qn.tobytes()).hexdigest() == doc["q_sha256"]
    assert hashlib.sha256(sn.tobytes()).hexdigest() == doc["s_sha256"]
    assert hashlib.sha256(pack_weight(q).cpu().numpy().tobytes()).hexdigest() == doc["packed_sha256"]


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 15, 16, 17, 31, 32, 33, 48, 64, 65, 80, 100, 112, 128, 129, 200])
def test_linear_matches_oracle_across_batch(m):
    n, k = 256, 512
    q, s = _quantized(100 + m, n, k)
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, k)).astype(np.float16)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float16)
    want = int8_quant.linear_ref_fp32(x, q, s, bias)
    got = int8_linear(_cuda(x), pack_weight(_cuda(q)), _cuda(s), _cuda(bias), n).float().cpu().numpy()
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


def test_linear_edge_fixture_and_no_bias():
    d = np.load(os.path.join(GOLDEN, "int8_edge.npz"))
    packed = _cuda(d["packed"])
    got = int8_linear(_cuda(d["x"]), packed, _cuda(d["s"]), _cuda(d["bias"]), 48).float().cpu().numpy()
    # Row 35 (scale clamped at 65504) overflows fp16 to +-inf in both the kernel and the fp16-rounded oracle.
    want16 = int8_quant.linear_ref(d["x"], d["q"], d["s"], d["bias"]).astype(np.float32)
    assert np.array_equal(np.isinf(got), np.isinf(want16)) and np.isinf(got).any()
    finite = np.isfinite(want16)
    np.testing.assert_allclose(got[finite], d["y"][finite], atol=ATOL, rtol=RTOL)
    got_nb = int8_linear(_cuda(d["x"]), packed, _cuda(d["s"]), None, 48).float().cpu().numpy()
    want_nb = int8_quant.linear_ref(d["x"], d["q"], d["s"]).astype(np.float32)
    np.testing.assert_allclose(got_nb, want_nb, atol=ATOL, rtol=RTOL)


def test_linear_config1_golden():
    doc = json.load(open(os.path.join(GOLDEN, "int8_config1.json")))
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 4096, generator=g).to(torch.float16)
    w = torch.randn(4096, 4096, generator=g) * 0.02
    lin = torch.nn.Linear(4096, 4096, bias=False)
    lin.weight.data.copy_(w)
    mod = Int8Linear.from_linear(lin, device="cuda")
    y = mod(x.cuda()).float().cpu().numpy()
    np.testing.assert_allclose(y[0, :16], doc["y_head"], atol=ATOL, rtol=RTOL)
    q, s = int8_quant.quantize_per_channel(w.numpy())
    np.testing.assert_allclose(y, int8_quant.linear_ref_fp32(x.numpy(), q, s), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("m", [5, 8, 16, 32, 48, 64, 80, 128, 150])
def test_linear_split_k_path_and_unsplit_fallback(m):
    """N=256, K=8192: few n-blocks and a long K, so the planner splits K over workgroups (fp32 partials +
    reduce); calling without a workspace must give the same answer through the unsplit kernel."""
    from runtime_amd.phase2 import _hip

    n, k = 256, 8192
    q, s = _quantized(300 + m, n, k)
    rng = np.random.default_rng(300 + m)
    x = rng.standard_normal((m, k)).astype(np.float16)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float16)
    lib = _hip.load()
    assert lib.mx_w8a16_workspace_bytes(m, n, k) > 0
    packed, sd, bd, xd = pack_weight(_cuda(q)), _cuda(s), _cuda(bias), _cuda(x)
    want = int8_quant.linear_ref_fp32(x, q, s, bias)
    got = int8_linear(xd, packed, sd, bd, n)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    y = torch.empty(m, n, dtype=torch.float16, device="cuda")
    _hip.check(lib.mx_w8a16_linear(xd.data_ptr(), m, k, k, packed.data_ptr(), sd.data_ptr(), bd.data_ptr(),
                                   y.data_ptr(), n, n, None, 0, _hip.stream_handle(xd.device)), "linear")
    np.testing.assert_allclose(y.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)


LLAMA_SHAPES = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 28672), ("down", 14336, 4096)]


@pytest.mark.parametrize("name,k,n", LLAMA_SHAPES)
def test_linear_llama_shapes(name, k, n):
    idx = [s[0] for s in LLAMA_SHAPES].index(name)
    q, s = _quantized(1000 + idx, n, k)
    packed, sd = pack_weight(_cuda(q)), _cuda(s)
    for m in (1, 8, 32, 64):
        x = np.random.default_rng(m + idx).standard_normal((m, k)).astype(np.float16)
        got = int8_linear(_cuda(x), packed, sd, None, n).float().cpu().numpy()
        np.testing.assert_allclose(got, int8_quant.linear_ref_fp32(x, q, s), atol=ATOL, rtol=RTOL,
                                   err_msg=f"{name} M={m}")


def test_linear_strided_rows_and_preallocated_out():
    n, k, m = 128, 256, 6
    q, s = _quantized(7, n, k)
    big = torch.randn(m, k + 64, dtype=torch.float16, device="cuda")
    x = big[:, 32:32 + k]  # row stride k + 64, 16-byte aligned start
    out_big = torch.zeros(m, n + 16, dtype=torch.float16, device="cuda")
    got = int8_linear(x, pack_weight(_cuda(q)), _cuda(s), None, n)
    want = int8_quant.linear_ref_fp32(x.cpu().numpy(), q, s)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    y3 = int8_linear(x.reshape(2, 3, k), pack_weight(_cuda(q)), _cuda(s), None, n)
    assert y3.shape == (2, 3, n)
    assert torch.equal(y3.reshape(m, n), got)
    int8_linear(x, pack_weight(_cuda(q)), _cuda(s), None, n, out=out_big[:, :n])  # row stride n + 16
    assert torch.equal(out_big[:, :n], got)
    assert out_big[:, n:].abs().sum().item() == 0


def test_quantize_model_swaps_linears():
    model = torch.nn.Sequential()
    model.add_module("q_proj", torch.nn.Linear(128, 64, bias=True))
    model.add_module("other", torch.nn.Linear(128, 64))
    w = model.q_proj.weight.detach().numpy().copy()
    b = model.q_proj.bias.detach().numpy().astype(np.float16)
    quantize_model_(model, device="cuda")
    assert isinstance(model.q_proj, Int8Linear) and isinstance(model.other, torch.nn.Linear)
    x = np.random.default_rng(3).standard_normal((3, 128)).astype(np.float16)
    y = model.q_proj(_cuda(x))
    assert y.shape == (3, 64) and y.dtype == torch.float16
    q, s = int8_quant.quantize_per_channel(w)
    np.testing.assert_allclose(y.float().cpu().numpy(), int8_quant.linear_ref_fp32(x, q, s, b), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("n,k,m", [(6144, 4096, 32), (4096, 4096, 32), (4096, 14336, 32), (4096, 4096, 100),
                                   (4096, 14336, 128)])
def test_split_partials_sum_to_linear_output(n, k, m):
    """qkv, o and down at M=32 (and up to one 128-row chunk) split K: the partials, summed
    bias-first in split order and rounded, are exactly mx_w8a16_linear's output (its reduce
    adds in that order)."""
    from runtime_amd.phase2.int8_linear import (int8_linear, int8_linear_partials, linear_splits, pack_weight,
                                                quantize_weight)

    g = torch.Generator(device="cuda").manual_seed(n + k)
    w = torch.randn(n, k, generator=g, device="cuda") * 0.02
    q, s = quantize_weight(w)
    packed = pack_weight(q)
    x = torch.randn(m, k, generator=g, device="cuda").half()
    bias = (torch.randn(n, generator=g, device="cuda") * 0.1).half()
    splits = linear_splits(m, n, k)
    assert splits > 1
    part = torch.full((splits * m * n,), float("nan"), dtype=torch.float32, device="cuda")
    assert int8_linear_partials(x, packed, s, n, part) == splits
    acc = bias.float().unsqueeze(0).expand(m, n).clone()
    for sp in part.view(splits, m, n):
        acc = acc + sp
    y = int8_linear(x, packed, s, bias, n)
    assert torch.equal(acc.half(), y)
    want = int8_quant.linear_ref(x.cpu().numpy(), q.cpu().numpy(), s.cpu().numpy(), bias.cpu().numpy())
    np.testing.assert_allclose(y.cpu().float().numpy(), want.astype(np.float32), atol=1e-2, rtol=1e-2)


def test_partials_reject_unsplit_shapes():
    from runtime_amd.phase2.int8_linear import int8_linear_partials, linear_splits, pack_weight, quantize_weight

    q, s = quantize_weight(torch.randn(28672, 64, device="cuda"))
    assert linear_splits(32, 28672, 64) == 1
    with pytest.raises(ValueError):
        int8_linear_partials(torch.zeros(32, 64, device="cuda").half(), pack_weight(q), s, 28672,
                             torch.empty(1 << 20, device="cuda"))


@pytest.mark.parametrize("m,n,k", [(32, 4096, 14336), (32, 4096, 1024), (5, 256, 128), (64, 896, 4864)])
def test_swiglu_linear_equals_silu_mul_then_linear(m, n, k):
    """The SwiGLU product formed in the GEMM's x staging rounds exactly as mx_silu_mul does,
    so the fused call equals silu_mul followed by the plain linear, bit for bit, and the
    partials variant sums to it."""
    from runtime_amd.phase2.decode_glue import silu_mul
    from runtime_amd.phase2.int8_linear import (int8_linear_partials_swiglu, int8_linear_swiglu, linear_splits,
                                                pack_weight, quantize_weight)

    g = torch.Generator(device="cuda").manual_seed(m * 7 + n + k)
    q, s = quantize_weight(torch.randn(n, k, generator=g, device="cuda") * 0.02)
    packed = pack_weight(q)
    gu = (2 * torch.randn(m, 2 * k, generator=g, device="cuda")).half()
    bias = (torch.randn(n, generator=g, device="cuda") * 0.1).half()
    want = int8_linear(silu_mul(gu), packed, s, bias, n)
    got = int8_linear_swiglu(gu, packed, s, bias, n)
    assert torch.equal(got, want)
    splits = linear_splits(m, n, k)
    if splits > 1:
        part = torch.empty(splits * m * n, dtype=torch.float32, device="cuda")
        int8_linear_partials_swiglu(gu, packed, s, n, part)
        acc = bias.float().unsqueeze(0).expand(m, n).clone()
        for sp in part.view(splits, m, n):
            acc = acc + sp
        assert torch.equal(acc.half(), want)
    with pytest.raises(ValueError):
        int8_linear_swiglu(gu[:4], packed, s, bias, n)  # M <= 4 takes the GEMV path, not fused


@pytest.mark.parametrize("m,inter,k", [(32, 14336, 4096), (7, 4864, 896), (64, 1024, 256), (128, 1024, 256),
                                        (70, 4864, 896), (100, 14336, 4096), (1, 4864, 896), (3, 4864, 896),
                                        (4, 4864, 896), (1, 14336, 4096), (4, 14336, 4096),
                                        (49, 14336, 4096), (64, 14336, 4096), (16, 8192, 1024)])
def test_gateup_swiglu_epilogue_equals_separate_ops(m, inter, k):
    """gate||up with interleaved rows and the SwiGLU product in the epilogue equals the plain
    [gate | up] projection followed by mx_silu_mul, bit for bit where both take the same K
    accumulation (within fp16 rounding where the plain projection splits K, or where the fused launch
    sums two k parts: its MFMA launch at up to 32 rows and an even count of at most 32 k-tiles). At M <= 4 on the Qwen2-0.5B
    MLP (a shape whose MFMA launch splits K) the VALU GEMV takes both, with the product in
    the GEMV's own epilogue; the Llama MLP at M <= 4 runs the unsplit MFMA kernel, and shapes whose
    plain projection splits K (the Qwen2 MLP at 7 and 70 rows) run one unsplit MFMA launch, in two k
    parts at 7 rows. (16, 8192, 1024): an unsplit plain projection beside the two-part fused launch.
    The Llama MLP at 49-64 rows takes the instance with two m-tiles per wave and the SwiGLU epilogue."""
    from runtime_amd.phase2.decode_glue import silu_mul
    from runtime_amd.phase2.int8_linear import (gateup_deinterleave, gateup_interleave, int8_gateup_swiglu,
                                                linear_splits)

    g = torch.Generator(device="cuda").manual_seed(m + inter + k)
    wg = torch.randn(inter, k, generator=g, device="cuda") * 0.02
    wu = torch.randn(inter, k, generator=g, device="cuda") * 0.02
    x = torch.randn(m, k, generator=g, device="cuda").half()
    plain_q, plain_s = quantize_weight(torch.cat([wg, wu]))
    inter_w = gateup_interleave(wg, wu)
    assert torch.equal(gateup_deinterleave(inter_w.t()).t(), torch.cat([wg, wu]))
    iq, iscale = quantize_weight(inter_w)
    assert torch.equal(gateup_interleave(plain_s[:inter], plain_s[inter:]), iscale)  # row-wise quantization
    want = silu_mul(int8_linear(x, pack_weight(plain_q), plain_s, None, 2 * inter))
    got = int8_gateup_swiglu(x, pack_weight(iq), iscale, None, inter)
    kt = k // 64
    two_parts = m <= 32 and kt <= 32 and kt % 2 == 0  # the fused MFMA launch's short-K shape
    if linear_splits(min(m, 128), 2 * inter, k) == 1 and not two_parts:
        assert torch.equal(got, want)
    else:
        # The plain projection sums scaled split partials, or the fused launch sums two k parts
        # before scaling: the same value up to fp32 rounding, so g and u may differ by an fp16 ulp.
        torch.testing.assert_close(got, want, atol=1e-2, rtol=1e-2)
        assert (got.float() - want.float()).abs().max() <= 4e-3 * want.float().abs().max()


# N chosen so that the unsplit launch takes each wide workgroup shape: about one
# workgroup per CU with (waves, n-tiles per wave) = (5,1), (6,1), (7,1), (8,1), (8,2),
# (8,4); 128032 (NT % 4 == 2) falls back to 4 waves of one n-tile.
WIDE_N = [20000, 24000, 28672, 32000, 64000, 128000, 128032]


@pytest.mark.parametrize("m", [1, 3, 16, 32, 64])
@pytest.mark.parametrize("n", WIDE_N)
def test_linear_wide_workgroup_shapes(m, n):
    from runtime_amd.phase2.int8_linear import linear_splits

    k = 128
    assert linear_splits(m, n, k) == 1
    q, s = _quantized(7 + n + m, n, k)
    rng = np.random.default_rng(n + m)
    x = rng.standard_normal((m, k)).astype(np.float16)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float16)
    want = int8_quant.linear_ref_fp32(x, q, s, bias)
    got = int8_linear(_cuda(x), pack_weight(_cuda(q)), _cuda(s), _cuda(bias), n).float().cpu().numpy()
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("m,inter", [(32, 10000), (16, 12000), (32, 16000), (2, 14336), (64, 14336)])
def test_gateup_swiglu_epilogue_wide_shapes(m, inter):
    """The SwiGLU epilogue at the 5-, 6- and 8-wave unsplit shapes equals the separate ops bit for bit."""
    from runtime_amd.phase2.decode_glue import silu_mul
    from runtime_amd.phase2.int8_linear import gateup_interleave, int8_gateup_swiglu, linear_splits

    k = 128
    g = torch.Generator(device="cuda").manual_seed(m + inter)
    wg = torch.randn(inter, k, generator=g, device="cuda") * 0.02
    wu = torch.randn(inter, k, generator=g, device="cuda") * 0.02
    x = torch.randn(m, k, generator=g, device="cuda").half()
    assert linear_splits(m, 2 * inter, k) == 1
    plain_q, plain_s = quantize_weight(torch.cat([wg, wu]))
    iq, iscale = quantize_weight(gateup_interleave(wg, wu))
    want = silu_mul(int8_linear(x, pack_weight(plain_q), plain_s, None, 2 * inter))
    got = int8_gateup_swiglu(x, pack_weight(iq), iscale, None, inter)
    assert torch.equal(got, want)


@pytest.mark.parametrize("m,inter,k", [(16, 4864, 896), (3, 1024, 256), (32, 14336, 4096), (100, 4864, 896)])
def test_swiglu_interleaved_equals_separate_ops(m, inter, k):
    """mx_swiglu_interleaved from the interleaved projection's fp16 output, and (where the shape
    splits K) from its split partials + bias, equals the [gate | up] projection followed by
    mx_silu_mul, bit for bit."""
    from runtime_amd.phase2.decode_glue import silu_mul, swiglu_interleaved
    from runtime_amd.phase2.int8_linear import gateup_interleave, int8_linear_partials, linear_splits

    g = torch.Generator(device="cuda").manual_seed(m * 7 + inter + k)
    wg = torch.randn(inter, k, generator=g, device="cuda") * 0.02
    wu = torch.randn(inter, k, generator=g, device="cuda") * 0.02
    bg = (torch.randn(inter, generator=g, device="cuda") * 0.1).half()
    bu = (torch.randn(inter, generator=g, device="cuda") * 0.1).half()
    x = torch.randn(m, k, generator=g, device="cuda").half()
    plain_q, plain_s = quantize_weight(torch.cat([wg, wu]))
    want = silu_mul(int8_linear(x, pack_weight(plain_q), plain_s, torch.cat([bg, bu]), 2 * inter))
    iq, iscale = quantize_weight(gateup_interleave(wg, wu))
    ibias = gateup_interleave(bg, bu)
    packed = pack_weight(iq)
    y = int8_linear(x, packed, iscale, ibias, 2 * inter)
    assert torch.equal(swiglu_interleaved(y, inter), want)
    splits = linear_splits(m, 2 * inter, k)
    if splits > 1:
        part = torch.full((splits * m * 2 * inter,), float("nan"), dtype=torch.float32, device="cuda")
        assert int8_linear_partials(x, packed, iscale, 2 * inter, part) == splits
        got = swiglu_interleaved(None, inter, partials=part, splits=splits, bias=ibias, rows=m)
        assert torch.equal(got, want)


def test_swiglu_interleaved_rejects_bad_arguments():
    from runtime_amd.phase2.decode_glue import swiglu_interleaved

    y = torch.zeros(4, 32, device="cuda").half()
    with pytest.raises(ValueError):
        swiglu_interleaved(y, 8)  # 2*inter != 32
    with pytest.raises(ValueError):
        swiglu_interleaved(y, 16, partials=torch.zeros(8, device="cuda"), splits=2, rows=4)  # both inputs
    with pytest.raises(ValueError):
        swiglu_interleaved(None, 16, partials=torch.zeros(8, device="cuda"), splits=2, rows=4)  # too small


def test_workspace_growth_keeps_captured_graphs_valid():
    """A graph captured while the split-K workspace was small still replays correctly after a larger
    shape has grown the workspace: the outgrown buffer stays allocated, so nothing else reuses the
    address the graph holds (checked over several replays with allocator churn in between)."""
    from runtime_amd.phase2.int8_linear import int8_linear, linear_splits, pack_weight, quantize_weight

    g = torch.Generator(device="cuda").manual_seed(91)
    n, k, m = 4096, 4096, 32
    assert linear_splits(m, n, k) > 1
    q, s = quantize_weight(torch.randn(n, k, generator=g, device="cuda") * 0.02)
    pk = pack_weight(q)
    x = torch.randn(m, k, generator=g, device="cuda").half()
    want = int8_linear(x, pk, s, None, n)
    y = torch.empty_like(want)
    int8_linear(x, pk, s, None, n, out=y)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        int8_linear(x, pk, s, None, n, out=y)
    # A larger split shape grows the workspace past the captured one.
    q2, s2 = quantize_weight(torch.randn(n, 14336, generator=g, device="cuda") * 0.02)
    int8_linear(torch.randn(128, 14336, generator=g, device="cuda").half(), pack_weight(q2), s2, None, n)
    for _ in range(3):
        junk = [torch.full((1 << 20,), float("nan"), device="cuda") for _ in range(8)]
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)
        del junk
