"""Seeded synthetic operands (SplitMix64 streams) for tests and the benchmark.

Each operand uses its own SplitMix64 stream (Steele, Lea & Flood 2014); the
state after i draws is seed + i * 0x9e3779b97f4a7c15, so draws are computed
independently and vectorised. Range maps:
  int_range(bits):  int64 uniform in [-2^bits, 2^bits)   via (x >> (63-bits)) - 2^bits
  uint_range(bits): uint64 uniform in [0, 2^bits)        via x >> (64-bits)
  full:             all 64 bits
  bytes_below(L):   uint8 uniform in [0, L) by rejection of (x & 0xff) >= L
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int, start: int = 0) -> np.ndarray:
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def int_range(seed: int, shape, bits: int) -> np.ndarray:
    x = splitmix64(seed, int(np.prod(shape)))
    v = (x >> np.uint64(63 - bits)).astype(np.int64) - np.int64(1 << bits)
    return v.reshape(shape)


def uint_range(seed: int, shape, bits: int) -> np.ndarray:
    x = splitmix64(seed, int(np.prod(shape)))
    return (x >> np.uint64(64 - bits)).reshape(shape) if bits < 64 else x.reshape(shape)


def full_int64(seed: int, shape) -> np.ndarray:
    return splitmix64(seed, int(np.prod(shape))).view(np.int64).reshape(shape)


def bytes_below(seed: int, shape, limit: int) -> np.ndarray:
    count = int(np.prod(shape))
    out = np.empty(0, dtype=np.uint8)
    drawn = 0
    while out.size < count:
        need = count - out.size
        batch = splitmix64(seed, need + need // 8 + 1024, start=drawn)
        drawn += batch.size
        b = (batch & np.uint64(0xFF)).astype(np.uint8)
        out = np.concatenate([out, b[b < limit]])
    return out[:count].reshape(shape)


def operand_seed(seed: int, which: str) -> int:
    """Per-operand stream: seed ^ 0xA for A, seed ^ 0xB for B."""
    return seed ^ {"A": 0xA, "B": 0xB}[which]
