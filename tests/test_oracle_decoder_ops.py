"""Pins of the oracle's decoder ops (restatement of packages/kernels/root.zig:
150-270 and src/decoder.zig:210-211) against the reference's own checks."""
import numpy as np
import pytest


def test_cascade_kats(oracle):
    # root.zig:799-818: the pinned sum-of-squares order, bit for bit.
    x = ((np.arange(896) * 17) % 101 + 1).astype(np.float32) * np.float32(0.125)
    assert np.float32(oracle.sum_squares_pinned(x)).view(np.uint32) == 0x473BE6E0
    t = (np.arange(11) + 1).astype(np.float32) * np.float32(0.125)
    assert np.float32(oracle.sum_squares_pinned(t)).view(np.uint32) == 0x40FD0000


def test_rms_norm_constant_vector_exact(oracle):
    # root.zig:789-797
    y = oracle.rms_norm(np.full(4, 3, np.float32), np.ones(4, np.float32), 0.0, bf16=False)
    assert y.tolist() == [1, 1, 1, 1]
    yb = oracle.rms_norm(np.full(4, 3, np.float32), np.ones(4, np.float32), 0.0, bf16=True)
    assert yb.tolist() == [1, 1, 1, 1]


@pytest.mark.parametrize("n", [1, 7, 8, 31, 32, 33, 511, 8 * 4 * 16, 8 * 4 * 256 + 11,
                               8 * 4 * 4096 + 37])
def test_cascade_sums_every_term_once(oracle, n):
    # Small integers: every partial sum is an exact fp32 integer, so any order
    # gives the exact total; a dropped, repeated or misplaced term at any
    # level of the cascade (levels 1-3 need 16, 256 and 4096 row groups of
    # 32 elements) changes it.
    rng = np.random.default_rng(n)
    x = rng.integers(-8, 9, n).astype(np.float32)
    got = oracle.sum_squares_pinned(x)
    assert float(got) == float(np.sum(x.astype(np.int64) ** 2))


@pytest.mark.parametrize("n", [17, 2048, 8 * 4 * 300 + 5])
def test_rms_norm_d53_bound(oracle, n):
    # root.zig:873-889: |got - f64| <= (n + 8) 2^-24 |f64| elementwise (f32 mode).
    rng = np.random.default_rng(0xB22026 + n)
    x = ((rng.random(n, dtype=np.float32) * 2 - 1) * 2).astype(np.float32)
    w = (rng.random(n, dtype=np.float32) * 2 - 1).astype(np.float32)
    eps = 1e-5
    got = oracle.rms_norm(x, w, eps, bf16=False).astype(np.float64)
    x64 = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.sum(x64 * x64) / n + eps)
    ref = x64 * inv * w.astype(np.float64)
    assert np.all(np.abs(got - ref) <= (n + 8) * 2.0**-24 * np.abs(ref))
    # bf16 mode: three bf16 roundings (normalized value, weight, product;
    # unit roundoff 2^-8 each) on top.
    gb = oracle.rms_norm(x, w, eps, bf16=True).astype(np.float64)
    assert np.all(np.abs(gb - ref) <= (3 * 2.0**-8 + 2.0**-16) * np.abs(ref) + 1e-30)


def test_silu_zero_and_bound(oracle):
    # root.zig:781-787 (SiLU of zero is exactly zero) and the f64 check of
    # root.zig:891-903 widened by the final bf16 rounding.
    assert oracle.silu_bf16(np.zeros(1, np.float32))[0] == 0.0
    rng = np.random.default_rng(0xB22026)
    x = ((rng.random(4096, dtype=np.float32) * 2 - 1) * 8).astype(np.float32)
    got = oracle.silu_bf16(x).astype(np.float64)
    x64 = x.astype(np.float64)
    ref = x64 / (1.0 + np.exp(-x64))
    assert np.all(np.abs(got - ref) <= (2.0**-8 + 4 * 2.0**-24) * np.abs(ref))
    up = (rng.standard_normal(4096)).astype(np.float32)
    prod = oracle.silu_mul_bf16(x, up).astype(np.float64)
    assert np.all(np.abs(prod - ref * up) <= (2 * 2.0**-8 + 2.0**-16) * np.abs(ref * up) + 1e-30)
