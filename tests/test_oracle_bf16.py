"""Pins the oracle's bf16 conversions (packages/bf16/root.zig:17-37).

Anchors: the reference's 4,119 PyTorch-generated (f32, bf16) pairs
(packages/bf16/vectors.zig, extracted to tests/golden/bf16_pairs.npy), the
reference's all-patterns round trip (root.zig:50-59) and its widen test
(root.zig:61-68), and PyTorch's own CPU float32 -> bfloat16 conversion, an
independent implementation, over every sign/exponent/high-mantissa pattern
with the low 16 bits set to the rounding-critical values.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bf16_pairs.npy")


def test_reference_vectors(oracle):
    pairs = np.load(GOLDEN)
    assert pairs.shape == (4119, 2)
    f = pairs[:, 0].astype(np.uint32).view(np.float32)
    got = oracle.bf16_from_f32(f)
    assert np.array_equal(got, pairs[:, 1].astype(np.uint16))


def test_every_pattern_round_trips(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = oracle.bf16_from_f32(oracle.bf16_to_f32(bits))
    nan = (bits & 0x7FFF) > 0x7F80
    expected = np.where(nan, np.uint16(0x7FC0), bits)
    assert np.array_equal(back, expected)


def test_widen_little_endian(oracle):
    raw = np.array([0x80, 0x3F, 0x00, 0xC0], np.uint8)
    out = np.empty(2, np.float32)
    oracle.lib().ncmo_widen_little_endian(out, raw, 2)
    assert out.tolist() == [1.0, -2.0]


def test_against_torch_rounding(oracle):
    torch = pytest.importorskip("torch")
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x4000, 0xC000,
                     0x1234, 0xFEDC, 0x7FFE, 0x8002], np.uint32)
    f = (hi[:, None] | lows[None, :]).ravel().view(np.float32)
    got = oracle.bf16_from_f32(f)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all(got[nan] == 0x7FC0)


def test_flush_subnormal(oracle):
    L = oracle.lib()
    assert L.ncmo_flush_f32_subnormal(1e-40) == 0.0
    neg = L.ncmo_flush_f32_subnormal(-1e-40)
    assert neg == 0.0 and np.signbit(np.float32(neg))
    assert L.ncmo_flush_f32_subnormal(1.5) == 1.5
    assert L.ncmo_flush_f32_subnormal(np.float32(1.1754944e-38)) == np.float32(1.1754944e-38)
