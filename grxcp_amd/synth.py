"""Seeded synthetic inputs for the benchmark configurations.

numpy's PCG64 generator, then round-to-nearest-even to bf16 by integer
arithmetic on the fp32 bit pattern, so the same seed gives the same bf16
bits on every machine. These are inputs, not results: nothing here computes
what the kernels compute.
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even, NaN kept quiet."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    out = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7F800000)) == np.uint32(0x7F800000)
    nan &= (u & np.uint32(0x7FFFFF)) != 0
    if nan.any():
        out[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(n: int, seed: int, mean: float = 0.0, std: float = 1.0, chunk: int = 1 << 24) -> np.ndarray:
    """n values ~ N(mean, std^2), generated in fp32 and rounded to bf16 bits."""
    g = rng(seed)
    out = np.empty(n, np.uint16)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        v = g.standard_normal(e - s, dtype=np.float32)
        if std != 1.0:
            v *= np.float32(std)
        if mean != 0.0:
            v += np.float32(mean)
        out[s:e] = f32_to_bf16_bits(v)
    return out


def uniform_int8(n: int, seed: int, lo: int = -127, hi: int = 127) -> np.ndarray:
    """n int8 values uniform on [lo, hi] inclusive."""
    return rng(seed).integers(lo, hi + 1, size=n, dtype=np.int8)


def uniform_f32(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    return rng(seed).uniform(lo, hi, size=n).astype(np.float32)
