"""Seeded synthetic workloads for the ternary linear path (numpy only).

Generator: SplitMix64 over a counter, seeded per tensor with FNV-1a-64 of
"<workload>/<tensor>". Uniform integers use the high 32 bits; normals use
Box-Muller in float64 (one normal per two draws), rounded to f32 and, for
bf16 tensors, round-to-nearest-even to bf16. The CPU oracle consumes the same
bf16 values widened to f32, so input rounding never counts as error.
"""
from __future__ import annotations

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform_int(seed: int, n: int, k: int) -> np.ndarray:
    """n integers uniform in [0, k) (multiply-shift on the high 32 bits)."""
    hi = splitmix64(seed, n) >> np.uint64(32)
    return ((hi * np.uint64(k)) >> np.uint64(32)).astype(np.int64)


def normal(seed: int, n: int, std: float = 1.0) -> np.ndarray:
    z = splitmix64(seed, 2 * n)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2) * std).astype(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def seed_of(workload: str, tensor: str) -> int:
    return fnv1a64(f"{workload}/{tensor}")


def ternary_uniform(workload: str, tensor: str, n: int, k: int) -> np.ndarray:
    """[n, k] int8 i.i.d. uniform over {-1, 0, +1}."""
    return (uniform_int(seed_of(workload, tensor), n * k, 3) - 1).astype(np.int8).reshape(n, k)


def sparse24_uniform(workload: str, tensor: str, n: int, k: int) -> np.ndarray:
    """[n, k] int8 with exactly two nonzeros per group of 4: pattern uniform
    over the 6 two-of-four patterns, values uniform over {-1, +1}."""
    assert k % 4 == 0
    g = n * k // 4
    seed = seed_of(workload, tensor)
    pat = uniform_int(seed, g, 6)
    sg = uniform_int(seed ^ 0x5A5A5A5A5A5A5A5A, 2 * g, 2).reshape(g, 2) * 2 - 1
    pos = np.array([[0, 1], [0, 2], [0, 3], [1, 2], [1, 3], [2, 3]], dtype=np.int64)[pat]
    out = np.zeros((g, 4), dtype=np.int8)
    rows = np.arange(g)
    out[rows, pos[:, 0]] = sg[:, 0]
    out[rows, pos[:, 1]] = sg[:, 1]
    return out.reshape(n, k)


def row_scales(workload: str, tensor: str, n: int, samples: int = 2048, std: float = 0.02) -> np.ndarray:
    """Per-row scale = mean |W_fp| of a `samples`-long N(0, std) row."""
    z = normal(seed_of(workload, tensor), n * samples, std).reshape(n, samples)
    return np.abs(z).mean(axis=1, dtype=np.float64).astype(np.float32)


def activations(workload: str, tensor: str, m: int, k: int, std: float = 1.0, bf16: bool = True):
    """[m, k] N(0, std) activations; returns (f32 values, bf16 bits or None)."""
    x = normal(seed_of(workload, tensor), m * k, std).reshape(m, k)
    if bf16:
        b = f32_to_bf16_bits(x)
        return bf16_bits_to_f32(b), b
    return x, None


def pack_rows_u32(values: np.ndarray) -> np.ndarray:
    """Vectorised row-aligned u32 packing (K % 16 == 0), codes as in
    src/model/ternary.rs:134-140; identical to the library packer."""
    v = np.asarray(values, dtype=np.int8)
    n, k = v.shape
    assert k % 16 == 0
    code = np.where(v == -1, 0, np.where(v == 1, 2, 1)).astype(np.uint32).reshape(n, k // 16, 16)
    shifts = (2 * np.arange(16, dtype=np.uint32))
    return np.bitwise_or.reduce(code << shifts, axis=2).astype(np.uint32)
