"""Shared test helpers: deterministic operand builders and tolerance checks.

The fixture formulas restate the reference's deterministic generators:
  parity fixture   test/parity/fixtures/quantized_fixture.py:4-18
  e2e generators   test/e2e/program/operations/quantized-matmul.test.ts:95-204
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def pack_codes(q: np.ndarray, bits: int) -> np.ndarray:
    """Packs integer codes [N,K] LSB-first into u32 words [N,K/P]."""
    per_word = 32 // bits
    n, k = q.shape
    lanes = q.reshape(n, k // per_word, per_word).astype(np.uint64)
    shifts = (np.arange(per_word, dtype=np.uint64) * bits)
    return (lanes << shifts).sum(axis=-1).astype(np.uint32)


def unpack_bytes_le(packed: np.ndarray, bits: int) -> np.ndarray:
    """Independent decode through little-endian bytes (as
    tools/test-quantized-checkpoint.py:51-55 does), not u32 shifts."""
    raw = np.ascontiguousarray(packed.astype("<u4")).view(np.uint8).reshape(packed.shape[0], -1)
    if bits == 8:
        return raw.astype(np.int64)
    per_byte = 8 // bits
    mask = (1 << bits) - 1
    parts = [(raw >> (bits * i)) & mask for i in range(per_byte)]
    return np.stack(parts, axis=-1).reshape(packed.shape[0], -1).astype(np.int64)


def storage(values, dtype: str) -> np.ndarray:
    """Host storage array for an operand given as f64 values: f32, or bf16 bits."""
    f32 = np.asarray(values, dtype=np.float64).astype(np.float32)
    return O.bf16_from_f32(f32) if dtype == "bf16" else f32


def widened(arr: np.ndarray) -> np.ndarray:
    return O.f32_from_bf16(arr).astype(np.float64) if arr.dtype == np.uint16 else arr.astype(np.float64)


def fixture_operands(rows: int, inner: int, outputs: int, bits: int, group: int):
    """quantized_fixture.py:4-18: x, codes, scales, biases as f64 values."""
    r = np.arange(rows)[:, None]
    c = np.arange(inner)[None, :]
    x = ((r * 3 + c) % 9 - 4) / 8
    o = np.arange(outputs)[:, None]
    q = (o * 3 + c * 5) & ((1 << bits) - 1)
    blk = np.arange(inner // group)[None, :]
    scales = (1 + (o + blk) % 3) / 4
    biases = ((o + blk) % 3 - 1) / 8
    return x, q, scales, biases


def reference_f64(x: np.ndarray, q: np.ndarray, scales: np.ndarray, biases: np.ndarray, group: int) -> np.ndarray:
    """The f64 product of test/parity/reference/check-cuda-quantized-general.py:71-78."""
    s = np.repeat(scales, group, axis=1)
    b = np.repeat(biases, group, axis=1)
    return x @ (q * s + b).T


def peak_tolerance(expected: np.ndarray, dtype: str) -> float:
    """Peak-scaled absolute tolerance of the reference's catalog oracle
    (test/parity/reference/probe-capabilities.py:454-457)."""
    relative = 0.02 if dtype == "bf16" else 2e-6
    return relative * max(1.0, float(np.abs(expected).max()))


def assert_close_rtol_atol(actual: np.ndarray, expected: np.ndarray, rtol: float, atol: float) -> None:
    err = np.abs(actual.astype(np.float64) - expected.astype(np.float64))
    bound = atol + rtol * np.abs(expected.astype(np.float64))
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{int(bad.sum())} of {err.size} elements out of tolerance; worst at {i}: "
                             f"actual {actual[i]!r} expected {expected[i]!r} (rtol {rtol}, atol {atol})")
