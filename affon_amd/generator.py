"""Affon's seeded tensor initializer, vectorized: ``Tensor.randn(shape, {seed})``.

Restates src/js/compute/program.ts:339-345 (randn) and :1385-1426
(seededRandom = mulberry32, normal() = Box-Muller with a cached spare, cos
first): the state after i increments is seed + i*0x6d2b79f5 (mod 2^32), so
the whole stream is computed at once instead of sequentially. Each f64 value is
rounded to f32, and to bf16 (round to nearest even) for bf16 tensors
(src/js/compute/native.zig:1166-1177).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x6D2B79F5)
_MASK = np.uint64(0xFFFFFFFF)
_EPSILON = 2.220446049250313e-16
_CHUNK = 1 << 22


_MAX_SAFE_INTEGER = 2**53 - 1


def js_seed(seed) -> int:
    """The generator state a seed starts from: `(Number.isSafeInteger(seed) ?
    seed : 0) >>> 0` (program.ts:1386). Integral values within +-(2^53 - 1)
    (ints, or floats with no fraction) keep their low 32 bits; anything else
    (fractions, larger magnitudes, non-numbers) starts from 0."""
    if isinstance(seed, bool) or not isinstance(seed, (int, float, np.integer, np.floating)):
        return 0
    if isinstance(seed, (float, np.floating)):
        if not np.isfinite(seed) or seed != np.floor(seed):
            return 0
        seed = int(seed)
    seed = int(seed)
    return seed & 0xFFFFFFFF if abs(seed) <= _MAX_SAFE_INTEGER else 0


def uniforms(seed: int, start: int, count: int) -> np.ndarray:
    """Uniforms number start .. start+count-1 of the mulberry32 stream."""
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    t = (np.uint64(js_seed(seed)) + i * _GOLDEN) & _MASK
    t = ((t ^ (t >> np.uint64(15))) * (t | np.uint64(1))) & _MASK
    t = t ^ ((t + (((t ^ (t >> np.uint64(7))) * (t | np.uint64(61))) & _MASK)) & _MASK)
    return ((t ^ (t >> np.uint64(14))) & _MASK).astype(np.float64) / 4294967296.0


def normal_f32(seed: int, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """count values of mean + std * normal(), rounded to f32."""
    out = np.empty(count, dtype=np.float32)
    pairs = (count + 1) // 2
    for p0 in range(0, pairs, _CHUNK):
        p1 = min(pairs, p0 + _CHUNK)
        u = uniforms(seed, 2 * p0, 2 * (p1 - p0)).reshape(-1, 2)
        radius = np.sqrt(-2.0 * np.log(np.maximum(u[:, 0], _EPSILON)))
        angle = 2.0 * np.pi * u[:, 1]
        values = np.empty((p1 - p0, 2), dtype=np.float64)
        values[:, 0] = radius * np.cos(angle)
        values[:, 1] = radius * np.sin(angle)
        flat = (mean + std * values).reshape(-1)
        n = min(count - 2 * p0, flat.size)
        out[2 * p0:2 * p0 + n] = flat[:n].astype(np.float32)
    return out
