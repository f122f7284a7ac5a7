"""Seeded, platform-independent synthetic inputs (numpy Philox) for the parity tests.

The distributions follow the benchmark configurations of the fused per-layer
kernels and the reference validators' patterns (tools/kt_utils.h:117-191,
tools/v_rmsnorm_validate.cpp:51-101).
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(seed))


def normal(seed, shape, sigma=1.0, mean=0.0):
    return rng(seed).normal(mean, sigma, size=shape).astype(np.float32)


def uniform(seed, shape, lo, hi):
    return rng(seed).uniform(lo, hi, size=shape).astype(np.float32)


def norm_weight(seed, n):
    """1 + N(0, 0.1), the RMSNorm weight of the benchmark configurations."""
    return (1.0 + rng(seed).normal(0.0, 0.1, size=n)).astype(np.float32)


def q8_table(seed, vocab, dim):
    """int8 codes uniform in [-127, 127]; f32 scales U(0.001, 0.02), one per 64 codes."""
    g = rng(seed)
    q = g.integers(-127, 128, size=(vocab, dim), dtype=np.int8)
    s = g.uniform(0.001, 0.02, size=vocab * dim // 64).astype(np.float32)
    return q, s


# The seven quantizer patterns of tools/kt_utils.h:139-191, with the libc rand()
# draws replaced by the seeded generator (same value sets).
KT_PATTERNS = ["small_pos", "wide_rand", "all_zero", "alternating", "ramp", "large_mix", "positional"]


def kt_pattern(name: str, n: int, seed: int) -> np.ndarray:
    g = rng(seed)
    i = np.arange(n)
    if name == "small_pos":
        return (np.float32(0.1) + (g.integers(0, 100, n).astype(np.float32) / np.float32(1000.0))).astype(np.float32)
    if name == "wide_rand":
        return ((g.integers(0, 10000, n) - 5000).astype(np.float32) / np.float32(1000.0)).astype(np.float32)
    if name == "all_zero":
        return np.zeros(n, np.float32)
    if name == "alternating":
        return np.where(i % 2 == 0, 1.0, -1.0).astype(np.float32)
    if name == "ramp":
        return (i % 64).astype(np.float32)
    if name == "large_mix":
        return ((g.integers(0, 100000, n) - 50000).astype(np.float32) / np.float32(1000.0)).astype(np.float32)
    if name == "positional":
        return ((i % 64) - 32).astype(np.float32)
    raise ValueError(name)


def validator_row(seed, n):
    """x in [-1, 1] on a 0.001 grid, as tools/kt_utils.h:1052-1055."""
    return ((rng(seed).integers(0, 2001, n).astype(np.float32) / np.float32(1000.0)) - np.float32(1.0)).astype(np.float32)


def validator_weight(seed, n):
    """w in [0.5, 1.5] on a 0.001 grid, as tools/kt_utils.h:1056-1057."""
    return (np.float32(0.5) + rng(seed).integers(0, 1001, n).astype(np.float32) / np.float32(1000.0)).astype(np.float32)


def validator_rope_tables(max_pos, head_dim, rope_max_dim, base=10000.0):
    """The validator's tables (tools/kt_utils.h:957-971): float powf/cosf/sinf, rows zero-padded to rope_max_dim."""
    half = head_dim // 2
    c = np.zeros((max_pos + 1, rope_max_dim), np.float32)
    s = np.zeros((max_pos + 1, rope_max_dim), np.float32)
    j = np.arange(half, dtype=np.float32)
    theta = np.power(np.float32(base), (np.float32(-2.0) * j / np.float32(head_dim)).astype(np.float32)).astype(np.float32)
    for p in range(max_pos + 1):
        ang = (np.float32(p) * theta).astype(np.float32)
        c[p, :half] = np.cos(ang)
        s[p, :half] = np.sin(ang)
    return c, s
