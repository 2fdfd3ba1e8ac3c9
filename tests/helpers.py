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


def tie_group(bits: int, group: int) -> tuple[np.ndarray, np.ndarray]:
    """One quantization group of f32 values whose (w - b) / s is exactly k + 1/2
    for the scale s = 2^-3 and bias b = -1.5 that quantizing it stores (both
    exact in bf16, as is every value here): the group's minimum b, its
    maximum b + (2^bits - 1) s, then a tie for each k = 0, 1, ... (at most
    128 of them), the rest b. Returns (values, codes under round half to
    even: k for even k, k + 1 for odd k). Rounding half away from zero gives
    k + 1 for every tie, so it differs on every even k."""
    levels = (1 << bits) - 1
    s, b = 0.125, -1.5
    values = np.full(group, b, np.float32)
    codes = np.zeros(group, np.int64)
    values[1], codes[1] = b + levels * s, levels
    for k in range(max(0, min(levels, group - 2, 128))):
        values[2 + k] = b + (k + 0.5) * s
        codes[2 + k] = k if k % 2 == 0 else k + 1
    return values, codes


def _stored_param(value: np.float32, param_dtype: str) -> np.float32:
    return O.f32_from_bf16(O.bf16_from_f32(value)).reshape(-1)[0] if param_dtype == "bf16" else value


def near_tie_group(bits: int, group: int, param_dtype: str) -> np.ndarray:
    """One quantization group of f32 values with minimum 0 and maximum
    (2^bits - 1) * c, for the first c of a fixed list whose stored scale s
    admits values w within 64 ulps of (k + 1/2) s where rint(w * RN(1/s))
    differs from rint(RN(w / s)): those values first, then values 1 to 3 ulps
    either side of (k + 1/2) s, k = 0, 1, ... A quantizer that multiplies by
    a reciprocal of the scale instead of dividing gets some of the first
    values wrong."""
    levels = (1 << bits) - 1
    f32 = np.float32
    for c in (0.0237, 0.0313, 0.0411, 0.0191, 0.0667):
        hi = f32(levels * c)
        s = _stored_param(f32(hi / f32(levels)), param_dtype)
        inv = f32(f32(1) / s)
        ties = (np.arange(levels, dtype=f32) + f32(0.5)) * s
        down, up, near = ties.copy(), ties.copy(), [ties]
        for _ in range(64):
            down = np.nextafter(down, f32(-np.inf), dtype=f32)
            up = np.nextafter(up, f32(np.inf), dtype=f32)
            near += [down, up]
        cand = np.concatenate(near)
        split = cand[np.rint(cand / s) != np.rint(cand * inv)]
        if split.size:
            break
    values = np.zeros(group, f32)
    values[min(1, group - 1)] = hi
    steps = (-3, -2, -1, 1, 2, 3)
    for i in range(2, group):
        if i - 2 < split.size:
            values[i] = split[i - 2]
            continue
        k = (i - 2) % levels
        v = f32(f32(k + 0.5) * s)
        j = steps[((i - 2) // levels) % len(steps)]
        for _ in range(abs(j)):
            v = np.nextafter(v, f32(np.inf if j > 0 else -np.inf), dtype=f32)
        values[i] = v
    return values


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


class HipRuntime:
    """The few HIP runtime calls GPU tests need directly: device memory
    figures and stream capture into graphs."""

    def __init__(self):
        import ctypes
        self.ctypes = ctypes
        self.lib = ctypes.CDLL("libamdhip64.so")
        vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        psz = ctypes.POINTER(ctypes.c_size_t)
        for name, args in {"hipMemGetInfo": [psz, psz], "hipStreamBeginCapture": [vp, ctypes.c_int],
                           "hipStreamEndCapture": [vp, pvp],
                           "hipGraphInstantiate": [pvp, vp, vp, ctypes.c_char_p, ctypes.c_size_t],
                           "hipGraphLaunch": [vp, vp], "hipGraphExecDestroy": [vp], "hipGraphDestroy": [vp],
                           "hipStreamSynchronize": [vp]}.items():
            fn = getattr(self.lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int

    def check(self, status: int, what: str) -> None:
        if status != 0:
            raise RuntimeError(f"{what} failed with HIP status {status}")

    def free_bytes(self) -> int:
        free, total = self.ctypes.c_size_t(), self.ctypes.c_size_t()
        self.check(self.lib.hipMemGetInfo(self.ctypes.byref(free), self.ctypes.byref(total)), "hipMemGetInfo")
        return free.value

    def capture(self, stream: int, enqueue) -> tuple:
        """Captures what `enqueue()` puts on `stream` into an instantiated graph."""
        ct = self.ctypes
        s = ct.c_void_p(stream)
        graph, exe = ct.c_void_p(), ct.c_void_p()
        self.check(self.lib.hipStreamBeginCapture(s, 2), "hipStreamBeginCapture")  # relaxed mode
        try:
            enqueue()
        finally:
            self.check(self.lib.hipStreamEndCapture(s, ct.byref(graph)), "hipStreamEndCapture")
        self.check(self.lib.hipGraphInstantiate(ct.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
        return graph, exe

    def replay(self, stream: int, graph_exe: tuple) -> None:
        s = self.ctypes.c_void_p(stream)
        self.check(self.lib.hipGraphLaunch(graph_exe[1], s), "hipGraphLaunch")
        self.check(self.lib.hipStreamSynchronize(s), "hipStreamSynchronize")

    def destroy(self, graph_exe: tuple) -> None:
        self.lib.hipGraphExecDestroy(graph_exe[1])
        self.lib.hipGraphDestroy(graph_exe[0])


def oracle_columns(x, packed, scales, biases, bits: int, group: int, cols, threads: int = 16) -> np.ndarray:
    """The oracle's output for the given output columns only ([M, len(cols)]):
    the columns' weight rows are gathered into a smaller problem, which is
    split over threads (the oracle call releases the interpreter lock)."""
    from concurrent.futures import ThreadPoolExecutor
    cols = np.asarray(cols)
    sub = (np.ascontiguousarray(packed[cols]), np.ascontiguousarray(scales[cols]), np.ascontiguousarray(biases[cols]))
    out = np.zeros((x.shape[0], len(cols)), dtype=np.float32)
    parts = max(1, min(threads, len(cols)))
    bounds = [(len(cols) * i // parts, len(cols) * (i + 1) // parts) for i in range(parts)]
    with ThreadPoolExecutor(parts) as pool:
        list(pool.map(lambda r: O.quantized_matmul(x, *sub, bits, group, n_range=r, out=out), bounds))
    return out


def assert_bf16_product_close(actual: np.ndarray, expected: np.ndarray) -> None:
    """Tolerance for bf16 activations: rtol 1e-2, atol 1e-2 * rms(expected)."""
    rms = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
    assert_close_rtol_atol(actual, expected, rtol=1e-2, atol=1e-2 * rms)
