"""Shared helpers for the parity tests."""
import numpy as np


def ulp_distance_f32(a, b) -> np.ndarray:
    """Distance in units in the last place between float32 arrays (monotone
    integer mapping of the IEEE bit patterns, so it also counts across
    binades and across zero)."""
    def key(x):
        i = np.ascontiguousarray(x, np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)

    return np.abs(key(a) - key(b))


def seeded_uniform_f32(n, lo, hi, seed=42):
    """Config inputs: numpy's PCG64 generator (np.random.default_rng(seed))."""
    return np.random.default_rng(seed).uniform(lo, hi, n).astype(np.float32)


def seeded_bytes(n, seed=42):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)
