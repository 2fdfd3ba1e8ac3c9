"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker (or the timed CPU baseline),
never by the product package.

Arrays are numpy: f32 operands as float32, bf16 operands as uint16 bit patterns,
packed weights as uint32, all C-contiguous row-major.
"""
from __future__ import annotations

import ctypes
import math
import pathlib

import numpy as np

LIBRARY_PATH = pathlib.Path(__file__).resolve().with_name("liboracle.so")
F32, BF16 = 0, 1
_lib = None

c_void_p, c_size_t, c_int, c_uint, c_double, c_uint32 = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                                         ctypes.c_uint, ctypes.c_double, ctypes.c_uint32)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY_PATH.exists():
            raise RuntimeError(f"{LIBRARY_PATH} is missing: run `make -C oracle`")
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        lib.oracle_bf16_from_f32.restype = ctypes.c_uint16
        lib.oracle_bf16_from_f32.argtypes = [ctypes.c_float]
        lib.oracle_f32_from_bf16.restype = ctypes.c_float
        lib.oracle_f32_from_bf16.argtypes = [ctypes.c_uint16]
        lib.oracle_bf16_from_f32_array.argtypes = [c_void_p, c_void_p, c_size_t]
        lib.oracle_mulberry32_next.restype = c_double
        lib.oracle_mulberry32_next.argtypes = [ctypes.POINTER(c_uint32)]
        lib.oracle_randn.argtypes = [c_uint32, c_double, c_double, c_size_t, c_void_p, c_void_p]
        lib.oracle_quantized_matmul.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                                c_size_t, c_size_t, c_size_t, c_uint, c_size_t, c_size_t, c_size_t]
        lib.oracle_quantized_matmul_f64.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                                    c_size_t, c_size_t, c_size_t, c_uint, c_size_t]
        lib.baseline_quantized_matmul.restype = c_int
        lib.baseline_quantized_matmul.argtypes = lib.oracle_quantized_matmul.argtypes
        lib.oracle_quantize.argtypes = [c_void_p, c_int, c_size_t, c_size_t, c_uint, c_size_t, c_int, c_void_p,
                                        c_void_p, c_void_p]
        lib.oracle_dequantize.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_size_t, c_size_t, c_uint, c_size_t,
                                          c_int, c_void_p]
        _lib = lib
    return _lib


def _code(arr: np.ndarray) -> int:
    if arr.dtype == np.float32:
        return F32
    if arr.dtype == np.uint16:
        return BF16
    raise TypeError(f"oracle operands must be float32 or uint16 (bf16 bits), got {arr.dtype}")


def _c(arr: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(arr)


def bf16_from_f32(values: np.ndarray) -> np.ndarray:
    values = _c(np.asarray(values, dtype=np.float32))
    out = np.empty(values.shape, dtype=np.uint16)
    load().oracle_bf16_from_f32_array(values.ctypes.data, out.ctypes.data, values.size)
    return out


def f32_from_bf16(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def seed_state(seed) -> int:
    """program.ts:1386: `(Number.isSafeInteger(seed) ? seed : 0) >>> 0`."""
    if isinstance(seed, bool) or not isinstance(seed, (int, float)):
        return 0
    if isinstance(seed, float) and not (math.isfinite(seed) and seed == math.floor(seed)):
        return 0
    seed = int(seed)
    return seed % 2**32 if -(2**53 - 1) <= seed <= 2**53 - 1 else 0


def randn(seed: int, count: int, mean: float = 0.0, std: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """Affon's Tensor.randn stream: (f32 values, their RNE bf16 bit patterns)."""
    f32 = np.empty(count, dtype=np.float32)
    bf16 = np.empty(count, dtype=np.uint16)
    load().oracle_randn(seed_state(seed), mean, std, count, f32.ctypes.data, bf16.ctypes.data)
    return f32, bf16


def uniforms(seed: int, count: int) -> np.ndarray:
    state = c_uint32(seed_state(seed))
    fn = load().oracle_mulberry32_next
    return np.array([fn(ctypes.byref(state)) for _ in range(count)], dtype=np.float64)


def quantized_matmul(x: np.ndarray, packed: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int,
                     group_size: int, n_range: tuple[int, int] | None = None,
                     out: np.ndarray | None = None) -> np.ndarray:
    x, packed, scales, biases = _c(x), _c(packed.astype(np.uint32, copy=False)), _c(scales), _c(biases)
    M, K = x.shape
    N = packed.shape[0]
    if out is None:
        out = np.zeros((M, N), dtype=np.float32)
    begin, end = n_range if n_range is not None else (0, N)
    load().oracle_quantized_matmul(x.ctypes.data, _code(x), packed.ctypes.data, scales.ctypes.data,
                                   biases.ctypes.data, _code(scales), out.ctypes.data, M, K, N, bits, group_size,
                                   begin, end)
    return out


def baseline_quantized_matmul(x: np.ndarray, packed: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int,
                              group_size: int, n_range: tuple[int, int] | None = None,
                              out: np.ndarray | None = None) -> np.ndarray:
    """The CPU baseline loop (cpu_baseline.c): specialised per bit width and
    dtype pair, bit-identical to quantized_matmul. Releases the GIL while it
    runs, so threads may split N."""
    x, packed, scales, biases = _c(x), _c(packed.astype(np.uint32, copy=False)), _c(scales), _c(biases)
    M, K = x.shape
    N = packed.shape[0]
    if out is None:
        out = np.zeros((M, N), dtype=np.float32)
    begin, end = n_range if n_range is not None else (0, N)
    status = load().baseline_quantized_matmul(x.ctypes.data, _code(x), packed.ctypes.data, scales.ctypes.data,
                                              biases.ctypes.data, _code(scales), out.ctypes.data, M, K, N, bits,
                                              group_size, begin, end)
    if status != 0:
        raise ValueError("baseline_quantized_matmul does not take these arguments")
    return out


def quantized_matmul_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int,
                         group_size: int) -> np.ndarray:
    x, packed, scales, biases = _c(x), _c(packed.astype(np.uint32, copy=False)), _c(scales), _c(biases)
    M, K = x.shape
    N = packed.shape[0]
    out = np.zeros((M, N), dtype=np.float64)
    load().oracle_quantized_matmul_f64(x.ctypes.data, _code(x), packed.ctypes.data, scales.ctypes.data,
                                       biases.ctypes.data, _code(scales), out.ctypes.data, M, K, N, bits, group_size)
    return out


def quantize(weights: np.ndarray, bits: int, group_size: int, param_dtype: str = "bf16"):
    weights = _c(weights)
    N, K = weights.shape
    pdt = np.uint16 if param_dtype == "bf16" else np.float32
    packed = np.zeros((N, K * bits // 32), dtype=np.uint32)
    scales = np.zeros((N, K // group_size), dtype=pdt)
    biases = np.zeros((N, K // group_size), dtype=pdt)
    load().oracle_quantize(weights.ctypes.data, _code(weights), N, K, bits, group_size,
                           BF16 if param_dtype == "bf16" else F32, packed.ctypes.data, scales.ctypes.data,
                           biases.ctypes.data)
    return packed, scales, biases


def dequantize(packed: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int, group_size: int,
               out_dtype: str = "f32") -> np.ndarray:
    packed, scales, biases = _c(packed.astype(np.uint32, copy=False)), _c(scales), _c(biases)
    N = packed.shape[0]
    K = packed.shape[1] * (32 // bits)
    out = np.zeros((N, K), dtype=np.uint16 if out_dtype == "bf16" else np.float32)
    load().oracle_dequantize(packed.ctypes.data, scales.ctypes.data, biases.ctypes.data, _code(scales), N, K, bits,
                             group_size, BF16 if out_dtype == "bf16" else F32, out.ctypes.data)
    return out


# ---- the element-wise ops the reference applies after quantized_matmul ----

def add_output_bias(y: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """``add(projected, output_bias)`` (docs/core/quantized-inference.md:37-42):
    one f32 add per element, bias broadcast over rows (bf16 bias widened
    exactly). Pinned in tests/test_oracle.py by exact dyadic sums and the zero
    bias identity."""
    b = f32_from_bf16(bias) if bias.dtype == np.uint16 else np.asarray(bias, dtype=np.float32)
    return (np.asarray(y, dtype=np.float32) + b[None, :]).astype(np.float32)


def silu(g: np.ndarray) -> np.ndarray:
    """f32 ``silu(g) = g * sigmoid(g)`` written g / (1 + e^-g)
    (packages/@affon/models/src/llama/model.ts:82 applies ``silu`` to the gate
    projection). Pinned in tests/test_oracle.py by silu(0) = 0, the limits
    silu(g) -> g and -> 0, the odd-part identity silu(g) - silu(-g) = g, and
    an f64 evaluation of g * sigmoid(g) (within 4 ulp)."""
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def silu_gate(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``mul(silu(gate), up)`` in f32 (model.ts:82)."""
    return (silu(gate) * np.asarray(up, dtype=np.float32)).astype(np.float32)


# ---- the other ops of a decode step (rms_norm, softmax, index_select) ----
# Restated from the reference's capability-probe oracle
# (test/parity/reference/probe-capabilities.py): values widened to f64, the
# op computed in f64, the result rounded to the input's dtype (f32, or bf16
# round-to-nearest-even as its `rounded`, :111-116).

def _widen(x: np.ndarray) -> np.ndarray:
    return f32_from_bf16(x).astype(np.float64) if x.dtype == np.uint16 else np.asarray(x, dtype=np.float64)


def _narrow(values: np.ndarray, like: np.ndarray) -> np.ndarray:
    f32 = np.asarray(values, dtype=np.float64).astype(np.float32)
    return bf16_from_f32(f32) if like.dtype == np.uint16 else f32


def rms_norm(x: np.ndarray, epsilon: float = 1e-5) -> np.ndarray:
    """Along the last axis: x / sqrt(sum(x^2)/cols + epsilon)
    (probe-capabilities.py:320-327). Pinned in tests/test_oracle.py by the
    constant-row closed form, scale invariance and the unit mean square."""
    v = _widen(x)
    denominator = np.sqrt((v * v).sum(axis=-1, keepdims=True) / v.shape[-1] + epsilon)
    return _narrow(v / denominator, x)


def softmax(x: np.ndarray) -> np.ndarray:
    """Along the last axis: exp(x - max) / sum(exp(x - max))
    (probe-capabilities.py:347-354). Pinned in tests/test_oracle.py by rows
    summing to 1, shift invariance, the uniform and two-point closed forms,
    and no overflow at large inputs."""
    v = _widen(x)
    scaled = np.exp(v - v.max(axis=-1, keepdims=True))
    return _narrow(scaled / scaled.sum(axis=-1, keepdims=True), x)


def index_select(x: np.ndarray, axis: int, indices: np.ndarray) -> np.ndarray:
    """Rows (axis 0) or columns (axis 1) at the given indices, zeros for an
    index outside the axis (probe-capabilities.py:149-176). Pinned in
    tests/test_oracle.py by identity and reversal permutations, the zero fill
    and the axis-1 / transposed-axis-0 equivalence."""
    x = np.asarray(x)
    indices = np.asarray(indices, dtype=np.int64)
    size = x.shape[axis]
    valid = (indices >= 0) & (indices < size)
    taken = np.take(x, np.where(valid, indices, 0), axis=axis)
    mask = valid[:, None] if axis == 0 else valid[None, :]
    return np.where(mask, taken, np.zeros((), dtype=x.dtype)).astype(x.dtype)
