"""CPU checks that pin the int8 oracle (format, pack, linear) before it judges the GPU."""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

from oracle import int8_quant, int8_quant_c

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _edge():
    return np.load(os.path.join(GOLDEN, "int8_edge.npz"))


def _random_weights(seed: int, n: int, k: int, scale: float) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal((n, k)) * scale).astype(np.float32)


@pytest.mark.parametrize("n,k,scale,seed", [(16, 64, 0.02, 0), (48, 128, 1.0, 1), (64, 256, 3e-4, 2),
                                            (32, 192, 50.0, 3), (7, 33, 0.02, 4)])
def test_numpy_and_c_quantizers_agree(n, k, scale, seed):
    w = _random_weights(seed, n, k, scale)
    qn, sn = int8_quant.quantize_per_channel(w)
    qc, sc = int8_quant_c.quantize_per_channel(w)
    assert np.array_equal(qn, qc)
    assert np.array_equal(sn.view(np.uint16), sc.view(np.uint16))


def test_numpy_and_c_agree_on_edge_rows():
    w = _edge()["w"]
    qn, sn = int8_quant.quantize_per_channel(w)
    qc, sc = int8_quant_c.quantize_per_channel(w)
    assert np.array_equal(qn, qc)
    assert np.array_equal(sn.view(np.uint16), sc.view(np.uint16))


def test_fp16_conversion_matches_ieee_rne():
    """The C bit-level fp32->fp16 conversion and numpy's agree, including the boundaries."""
    rng = np.random.default_rng(5)
    special = np.array([0.0, -0.0, 2.0**-25, 2.0**-25 * 1.0000001, 2.0**-24, 1.5 * 2.0**-24, 2.5 * 2.0**-24,
                        2.0**-14, 2.0**-14 * (1 - 2.0**-11), 65504.0, 65519.0, 65520.0, 1e10, 1.0 + 2.0**-11,
                        1.0 + 3 * 2.0**-11, 1e-8, 3e-5, 6.1e-5], dtype=np.float32)
    vals = np.concatenate([special, -special, rng.standard_normal(2000).astype(np.float32) * 10.0,
                           (rng.random(2000) * 1e-4).astype(np.float32)])
    with np.errstate(over="ignore"):
        expected = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(int8_quant_c.f32_to_f16_bits(vals), expected)


def test_quantizer_invariants():
    w = np.concatenate([_random_weights(11, 64, 256, 0.02), _random_weights(12, 16, 256, 2.0)])
    q, s = int8_quant.quantize_per_channel(w)
    sf = s.astype(np.float32)
    assert q.dtype == np.int8 and s.dtype == np.float16
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    assert np.all(np.max(np.abs(q.astype(np.int32)), axis=1) == 127)  # normal, unclamped scales
    err = np.abs(w - q.astype(np.float32) * sf[:, None])
    assert np.all(err <= sf[:, None] * (0.5 + 1e-5))
    assert np.array_equal(s, (np.max(np.abs(w), axis=1) / np.float32(127)).astype(np.float16))


def test_edge_rows():
    d = _edge()
    q, s = int8_quant.quantize_per_channel(d["w"])
    sb = s.view(np.uint16)
    assert np.all(q[32] == 0) and s[32] == np.float16(1.0)  # zero row
    assert sb[34] == 0x0001  # underflowed scale -> smallest subnormal
    assert s[35] == np.float16(65504.0)  # clamped scale
    assert np.max(np.abs(q[35].astype(np.int32))) == 127
    assert q[36, 77] == -127 and np.count_nonzero(q[36]) == 1
    assert np.min(q[37]) == -127


def test_round_half_even_ties():
    """Row 33 holds w = (j + 0.5) * s exactly; q must be Python's banker's rounding of w / s."""
    d = _edge()
    w = d["w"][33].astype(np.float64)
    q, s = int8_quant.quantize_per_channel(d["w"])
    ratio = w / np.float64(s[33])
    expected = np.clip([round(v) for v in ratio], -127, 127)
    assert np.array_equal(q[33].astype(np.int64), expected)
    assert q[33, 2] == 0 and q[33, 3] == 0 and q[33, 4] == 2 and q[33, 5] == 2 and q[33, 1] == -126


def test_golden_edge_fixture_reproduces():
    d = _edge()
    q, s = int8_quant.quantize_per_channel(d["w"])
    assert np.array_equal(q, d["q"])
    assert np.array_equal(s.view(np.uint16), d["s"].view(np.uint16))
    assert np.array_equal(int8_quant.pack_tiles(q), d["packed"])
    y = int8_quant.linear_ref_fp32(d["x"], q, s, d["bias"])
    assert np.array_equal(y, d["y"])


def test_golden_config1_digests_reproduce():
    import torch

    doc = json.load(open(os.path.join(GOLDEN, "int8_config1.json")))
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 4096, generator=g).to(torch.float16).numpy()
    w = (torch.randn(4096, 4096, generator=g) * 0.02).numpy().astype(np.float32)
    assert hashlib.sha256(w.tobytes()).hexdigest() == doc["w_sha256"]
    q, s = int8_quant.quantize_per_channel(w)
    assert hashlib.sha256(q.tobytes()).hexdigest() == doc["q_sha256"]
    assert hashlib.sha256(s.tobytes()).hexdigest() == doc["s_sha256"]
    assert hashlib.sha256(int8_quant.pack_tiles(q).tobytes()).hexdigest() == doc["packed_sha256"]
    y = int8_quant.linear_ref_fp32(x, q, s)
    assert np.allclose(y[0, :16], doc["y_head"], rtol=0, atol=1e-5)


def test_pack_layout_definition():
    """Every byte lands where the layout formula says (independent scalar loop), and C agrees."""
    rng = np.random.default_rng(9)
    n, k = 32, 192
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    packed = int8_quant.pack_tiles(q)
    nt_count = n // 16
    for row in range(n):
        for col in range(0, k, 7):
            nt, r = divmod(row, 16)
            kt, rem = divmod(col, 64)
            g, j = divmod(rem, 16)
            off = (kt * nt_count + nt) * 1024 + (16 * g + r) * 16 + j
            assert packed[off] == (int(q[row, col]) & 0xFF) ^ 0x80
    assert np.array_equal(packed, int8_quant_c.pack_tiles(q))
    assert np.array_equal(int8_quant.unpack_tiles(packed, n, k), q)


def test_pack_rejects_bad_shapes():
    with pytest.raises(ValueError):
        int8_quant.pack_tiles(np.zeros((15, 64), np.int8))
    with pytest.raises(ValueError):
        int8_quant.pack_tiles(np.zeros((16, 96), np.int8))
    with pytest.raises(ValueError):
        int8_quant.quantize_per_channel(np.array([[1.0, np.nan]], np.float32))


def test_biased_byte_decode_exhaustive():
    """All 256 stored bytes decode exactly: fp16(0x6400 | b) = 1024 + b and minus 1152 = int8(b ^ 0x80)."""
    b = np.arange(256, dtype=np.uint16)
    raw = (np.uint16(0x6400) | b).view(np.float16).astype(np.float64)
    assert np.array_equal(raw, 1024.0 + b)
    dec = int8_quant.decode_biased_byte(b.astype(np.uint8)).astype(np.float64)
    assert np.array_equal(dec, (b.astype(np.uint8) ^ 0x80).view(np.int8).astype(np.float64))


def test_linear_ref_matches_float64_closed_form():
    rng = np.random.default_rng(13)
    w = _random_weights(14, 64, 256, 0.05)
    q, s = int8_quant.quantize_per_channel(w)
    x = rng.standard_normal((5, 256)).astype(np.float16)
    bias = rng.standard_normal(64).astype(np.float16)
    exact = x.astype(np.float64) @ (q.astype(np.float64) * s.astype(np.float64)[:, None]).T + bias.astype(np.float64)
    assert np.allclose(int8_quant.linear_ref_fp32(x, q, s, bias), exact, rtol=1e-5, atol=1e-5)


def test_checks_catch_planted_mistakes():
    """Plausible oracle mistakes (planted here, on the CPU) fail the checks above."""
    d = _edge()
    w = d["w"]
    s = int8_quant.quantize_per_channel(w)[1]
    # Round-half-away-from-zero instead of half-even breaks the tie row.
    ratio = w[33] / s[33].astype(np.float32)
    away = np.clip(np.sign(ratio) * np.floor(np.abs(ratio) + 0.5), -127, 127).astype(np.int8)
    assert not np.array_equal(away, d["q"][33])
    # Dividing by the fp32 scale instead of the fp16-rounded one changes some q.
    s32 = np.max(np.abs(w[:32]), axis=1) / np.float32(127)
    q_bad = np.clip(np.rint(w[:32] / s32[:, None]), -127, 127).astype(np.int8)
    assert not np.array_equal(q_bad, d["q"][:32])
    # A pack that forgets the 0x80 bias, or swaps rows and k-segments, is caught.
    good = int8_quant.pack_tiles(d["q"])
    assert not np.array_equal(good ^ np.uint8(0x80), d["packed"])
    t = (d["q"].view(np.uint8) ^ 0x80).reshape(3, 16, 2, 4, 16).transpose(0, 2, 1, 3, 4).reshape(-1)
    assert not np.array_equal(t, d["packed"])
    # A dropped bias term in the linear is caught by the fixture.
    y_bad = int8_quant.linear_ref_fp32(d["x"], d["q"], d["s"], None)
    assert not np.allclose(y_bad, d["y"], atol=1e-3)
