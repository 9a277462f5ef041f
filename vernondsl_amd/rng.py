"""Seeded synthetic inputs: counter-based splitmix64, evaluated with numpy on the host.

Draw i of stream `seed` is mix64(seed + (i + 1) * 0x9E3779B97F4A7C15), so any slice of a stream
can be produced independently and the bytes do not depend on numpy's own generators or version.
The same host bytes are uploaded to the HIP device and handed to the CPU oracle.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def u64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Draws start .. start+n-1 of stream `seed` as uint64."""
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        return _mix(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN)


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """f32 values lo + (hi - lo) * u, u = top 24 bits / 2^24 in [0, 1) (computed in f64)."""
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, _CHUNK):
        e = min(n, s + _CHUNK)
        u = (u64(seed, e - s, s) >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))
        out[s:e] = (lo + (hi - lo) * u).astype(np.float32)
    return out


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """f32 normals by f64 Box-Muller over draw pairs (2k, 2k+1): cos for element 2k, sin for 2k+1."""
    out = np.empty(n, dtype=np.float32)
    pairs = (n + 1) // 2
    for s in range(0, pairs, _CHUNK):
        e = min(pairs, s + _CHUNK)
        d = u64(seed, 2 * (e - s), 2 * s)
        u1 = ((d[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / (1 << 53))  # (0, 1]
        u2 = (d[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
        r = np.sqrt(-2.0 * np.log(u1))
        th = 2.0 * np.pi * u2
        blk = np.empty(2 * (e - s), dtype=np.float64)
        blk[0::2] = r * np.cos(th)
        blk[1::2] = r * np.sin(th)
        lo, hi = 2 * s, min(n, 2 * e)
        out[lo:hi] = (mean + std * blk[: hi - lo]).astype(np.float32)
    return out


def int_uniform(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Integers in [lo, hi] (inclusive) as int64: lo + draw mod (hi - lo + 1)."""
    span = np.uint64(hi - lo + 1)
    out = np.empty(n, dtype=np.int64)
    for s in range(0, n, _CHUNK):
        e = min(n, s + _CHUNK)
        out[s:e] = (u64(seed, e - s, s) % span).astype(np.int64) + lo
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16); NaN -> 0x7FC0."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
