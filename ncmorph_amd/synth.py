"""Deterministic synthetic inputs for the benchmark configurations.

Normals come from SplitMix64 (one 64-bit draw per uniform) and Box-Muller in
f64, then scaled and rounded to f32; bf16 tensors are the RNE rounding of
those f32 values. The same (seed, count) always yields the same bits, on any
host.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int, start: int = 0) -> np.ndarray:
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def normal_f64(seed: int, count: int) -> np.ndarray:
    pairs = (count + 1) // 2
    z = splitmix64(seed, 2 * pairs)
    u = (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return out[:count]


def normal_f32(seed: int, shape, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    return (normal_f64(seed, n) * std).astype(np.float32).reshape(shape)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """RNE f32 -> bf16 bit patterns, every NaN -> 0x7FC0."""
    x = np.ascontiguousarray(a, np.float32).view(np.uint32)
    nan = (x & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = ((x + np.uint32(0x7FFF) + ((x >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    r = r.astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(
        np.float32)


def normal_bf16(seed: int, shape, std: float = 1.0) -> np.ndarray:
    return bf16_bits(normal_f32(seed, shape, std))


# Seeds of the linear shapes (none are given by the configuration; fixed here).
LINEAR_SEED_X = 0x11E4_0001
LINEAR_SEED_W = 0x11E4_0002

# Codebook seed = input seed + this offset (the configuration names only the
# input seed).
RVQ_CODEBOOK_SEED_OFFSET = 0xC0DE_B00C


def rvq_inputs(seed: int, b: int, t: int, d: int, levels: int, v: int):
    """x f32 [b, t, d] ~N(0, 1); codebooks bf16 bits [levels, v, d] ~N(0, 1/d)."""
    x = normal_f32(seed, (b, t, d))
    cb = normal_bf16(seed + RVQ_CODEBOOK_SEED_OFFSET, (levels, v, d), std=1.0 / np.sqrt(d))
    return x, cb


# The two RVQ configurations: encode+decode of one sequence at full
# resolution, and the multiscale encode at scale.
RVQ_SMALL = dict(seed=0, b=1, t=128, d=256, levels=4, v=512, strides=(1, 1, 1, 1))
RVQ_LARGE = dict(seed=1, b=16, t=2048, d=2048, levels=8, v=4096,
                 strides=(128, 64, 32, 16, 8, 4, 2, 1))
