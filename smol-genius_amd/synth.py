"""Seeded synthetic inputs shared by the tests and the bench.

One documented generator so the GPU path and the CPU oracle consume the same
bits: splitmix64 -> Box-Muller in float64 -> float32 -> (where a bf16 tensor is
specified) bf16 by round-to-nearest-even. The CPU side widens bf16 back to
float32 losslessly.
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, n):
    """n consecutive splitmix64 outputs for state = seed (uint64 arithmetic wraps)."""
    with np.errstate(over="ignore"):
        state = np.uint64(seed) + _GOLDEN * np.arange(1, n + 1, dtype=np.uint64)
        z = state
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed, shape, std=1.0):
    """float32 N(0, std^2) samples of the given shape."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    bits = splitmix64(seed, 2 * m)
    u1 = ((bits[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (bits[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:n] * std).astype(np.float32).reshape(shape)


def uniform_int(seed, n, lo, hi):
    """n integers in [lo, hi] (inclusive): lo + (u64 % (hi - lo + 1))."""
    return (np.uint64(lo) + splitmix64(seed, n) % np.uint64(hi - lo + 1)).astype(np.int64)


def f32_to_bf16_bits(x):
    """float32 -> bf16 bit patterns (uint16), round-to-nearest-even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    rounding = ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)
    return ((u + rounding) >> np.uint64(16)).astype(np.uint16)


def bf16_bits_to_f32(b):
    """bf16 bit patterns -> float32 (exact)."""
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x):
    """float32 values rounded to the nearest bf16, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
