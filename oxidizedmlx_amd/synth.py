"""Seeded synthetic inputs for benchmarks and parity tests.

The reference has no generator for its configs' N(mu, sigma^2) / U(a, b)
inputs, so this one is documented instead: SplitMix64 (counter-based, so it
vectorises) gives 53-bit uniforms; Box-Muller turns pairs of them into
normals. Values are computed in float64 and rounded once to float32.
Also: round-to-nearest-even to bf16 / f16, as the GEMM inputs are stored.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of SplitMix64 started at ``seed``."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, n: int) -> np.ndarray:
    """float64 uniforms in [0, 1) with 53 random bits."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """float32 N(mean, std^2) by Box-Muller on SplitMix64 uniforms."""
    n = int(np.prod(shape)) if shape else 1
    m = (n + 1) // 2
    u = uniform01(seed, 2 * m)
    r = np.sqrt(-2.0 * np.log1p(-u[:m]))
    t = 2.0 * np.pi * u[m:]
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(t)
    z[1::2] = r * np.sin(t)
    return (mean + std * z[:n]).astype(np.float32).reshape(shape)


def uniform(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    """float32 U(lo, hi)."""
    n = int(np.prod(shape)) if shape else 1
    return (lo + (hi - lo) * uniform01(seed, n)).astype(np.float32).reshape(shape)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16 (RNE), kept as float32."""
    return bf16_to_f32(bf16_bits(x))


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def round_f16(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
