"""Seeded synthetic inputs for the workloads (numpy, host side).

Every GPU run and its CPU check draw from the same generator, so both see the
same bytes: numpy's PCG64 ``default_rng(SEED_BASE + config_id)``.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x5EEDF8

# binary32 specials injected into the conversion workload (bit patterns):
# +-inf, +-NaN, binary32 subnormals (+-1e-40, +-2^-149), subnormals that are
# exact in bf16 (+-2^-133), signed zeros.
SPECIAL_BITS = np.array([
    0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000,
    0x000116C2, 0x800116C2, 0x00000001, 0x80000001,
    0x00010000, 0x80010000, 0x00000000, 0x80000000,
], dtype=np.uint32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round binary32 to bf16 bit patterns, nearest-even; NaN -> sign|0x7FC0."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = (((u[nan] >> 16) & 0x8000) | 0x7FC0).astype(np.uint16)
    return r


def normal(shape, std=1.0, seed=SEED_BASE, mean=0.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    if mean != 0.0:
        x += np.float32(mean)
    return x.reshape(shape)


def conversion_input(n: int, seed: int = SEED_BASE + 2) -> np.ndarray:
    """Config 2 input: N(0,1), 0.1% of positions (seeded, with repeats) x1000,
    then the SPECIAL_BITS at seeded positions.  float32."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n, dtype=np.float32)
    k = max(1, n // 1000)
    idx = rng.integers(0, n, size=k)
    x[idx] *= np.float32(1000.0)
    if n >= len(SPECIAL_BITS):
        pos = rng.integers(0, n, size=len(SPECIAL_BITS))
        x.view(np.uint32)[pos] = SPECIAL_BITS
    return x
