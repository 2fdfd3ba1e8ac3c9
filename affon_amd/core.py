"""Host-side mirror of Affon's Session / Tensor / Program surface for the rocm device.

The reference surface is TypeScript (``affon:core``, src/js/compute/program.ts,
typings packages/@types/affon/affon-compute-program.d.ts). This module keeps
its names, argument meaning and error behaviour for the parts the quantized
linear path touches:

* ``Session(device='rocm')`` owns one native session (one HIP stream) and the
  device tensors created through it (src/js/compute/program.ts:1775-1911);
* ``Tensor`` is an evaluated, Session-owned device tensor; views (transpose,
  slice) share storage and carry element strides and a byte offset
  (docs/core/quantized-inference.md:47-49);
* ``TensorSpec`` / ``program`` / ``Executable`` author and run a formal
  Program of ``quantized_matmul`` nodes (src/js/compute/program.ts:481-494,
  1856-1885, 1704-1737), with one or several outputs; ``add`` / ``mul`` /
  ``silu`` nodes after them are lowered into the kernels' output epilogues
  (lowering.py).

Device memory comes from the native library; there is no CPU execution path.
"""
from __future__ import annotations

import ctypes
import itertools
import weakref
from dataclasses import dataclass
from typing import Any, Callable, Mapping, Sequence

import numpy as np

from . import _native

DTYPES = ("bf16", "f32", "u32", "i64")
_NATIVE_DTYPE = {"f32": _native.F32, "bf16": _native.BF16, "u32": _native.U32}
_ITEMSIZE = {"f32": 4, "bf16": 2, "u32": 4, "i64": 8}
_STORAGE = {"f32": np.float32, "bf16": np.uint16, "u32": np.uint32, "i64": np.int64}

COMPILE_OPTION_VALUES = {
    "optimizationLevel": ("none", "safe"),
    "numericalPolicy": ("exact_only", "backend_equivalent", "approximate"),
    "explanationLevel": ("summary", "detailed"),
}
_POLICY = {"exact_only": _native.EXACT_ONLY, "backend_equivalent": _native.BACKEND_EQUIVALENT,
           "approximate": _native.APPROXIMATE}


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """f32 -> bf16 round to nearest even, as bit patterns (NaN stays quiet)."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((bits >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def host_storage(values: Any, dtype: str) -> np.ndarray:
    """Converts host values to the storage array of dtype: f64 -> f32 rounding
    first, then bf16 rounding (src/js/compute/native.zig:1166-1177)."""
    if dtype == "u32":
        return np.ascontiguousarray(np.asarray(values, dtype=np.float64).astype(np.uint64).astype(np.uint32))
    if dtype == "i64":
        return np.ascontiguousarray(np.asarray(values, dtype=np.int64))
    f32 = np.ascontiguousarray(np.asarray(values, dtype=np.float64).astype(np.float32))
    return bf16_bits(f32) if dtype == "bf16" else f32


class _Buffer:
    """One device allocation; freed when the last tensor using it is gone, or
    by the native session when the Session is disposed first (the session
    frees every allocation it still owns)."""

    def __init__(self, session: "Session", nbytes: int):
        self.session = session
        self.nbytes = nbytes
        ptr = ctypes.c_void_p()
        _native.check(_native.load().affon_rocm_alloc(session._handle, max(nbytes, 1), ctypes.byref(ptr)), "alloc")
        self.ptr = ptr.value
        session._buffers.add(self)

    def release(self) -> None:
        if self.ptr is not None and self.session._handle is not None:
            _native.load().affon_rocm_free(self.session._handle, self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


@dataclass(frozen=True)
class TensorSpec:
    dtype: str
    shape: tuple[int, ...]

    @staticmethod
    def f32(shape: Sequence[int]) -> "TensorSpec":
        return TensorSpec("f32", tuple(int(d) for d in shape))

    @staticmethod
    def bf16(shape: Sequence[int]) -> "TensorSpec":
        return TensorSpec("bf16", tuple(int(d) for d in shape))

    @staticmethod
    def u32(shape: Sequence[int]) -> "TensorSpec":
        return TensorSpec("u32", tuple(int(d) for d in shape))

    @staticmethod
    def i64(shape: Sequence[int]) -> "TensorSpec":
        return TensorSpec("i64", tuple(int(d) for d in shape))


class Tensor:
    """An evaluated device tensor (or a view of one) owned by a Session."""

    def __init__(self, session: "Session", buffer: _Buffer, dtype: str, shape: Sequence[int],
                 strides: Sequence[int], offset_elements: int = 0):
        self.session = session
        self._buffer = buffer
        self.dtype = dtype
        self.shape = tuple(int(d) for d in shape)
        self.strides = tuple(int(s) for s in strides)
        self.offset = int(offset_elements)
        self._disposed = False

    @property
    def spec(self) -> TensorSpec:
        return TensorSpec(self.dtype, self.shape)

    def _check_live(self) -> None:
        if self._disposed or self._buffer.ptr is None:
            raise RuntimeError("tensor has been disposed")

    def view(self) -> _native.View:
        self._check_live()
        if len(self.shape) != 2 or self.dtype not in _NATIVE_DTYPE:
            raise TypeError("rank-two f32/bf16/u32 tensor required")
        return _native.View(self._buffer.ptr, self._buffer.nbytes, self.offset * _ITEMSIZE[self.dtype],
                            (ctypes.c_int64 * 2)(*self.shape), (ctypes.c_int64 * 2)(*self.strides),
                            _NATIVE_DTYPE[self.dtype])

    @property
    def data_ptr(self) -> int:
        self._check_live()
        return self._buffer.ptr + self.offset * _ITEMSIZE[self.dtype]

    def is_contiguous(self) -> bool:
        expected = 1
        for dim, stride in zip(reversed(self.shape), reversed(self.strides)):
            if dim != 1 and stride != expected:
                return False
            expected *= dim
        return True

    def storage(self) -> np.ndarray:
        """Reads the view back as a host array of the storage dtype (synchronizes)."""
        self._check_live()
        lib = _native.load()
        raw = np.empty(self._buffer.nbytes // _ITEMSIZE[self.dtype], dtype=_STORAGE[self.dtype])
        _native.check(lib.affon_rocm_memcpy_d2h(self.session._handle, raw.ctypes.data, self._buffer.ptr,
                                                raw.nbytes), "readback")
        item = raw.itemsize
        return np.lib.stride_tricks.as_strided(raw[self.offset:], shape=self.shape,
                                               strides=tuple(s * item for s in self.strides)).copy()

    def numpy(self) -> np.ndarray:
        """Host values: f32 for f32/bf16 (bf16 widened exactly), u32 for u32."""
        values = self.storage()
        return bf16_to_f32(values) if self.dtype == "bf16" else values

    def to_array(self) -> Any:
        return self.numpy().tolist()

    def item(self) -> Any:
        values = self.numpy()
        if values.size != 1:
            raise ValueError("item() requires exactly one element")
        return values.reshape(-1)[0].item()

    def dispose(self) -> None:
        self._disposed = True


class Session:
    """A rocm compute session: one native session (device ordinal, HIP stream)."""

    def __init__(self, device: str = "rocm"):
        if device != "rocm" and not device.startswith("rocm:"):
            raise TypeError(f"unsupported device: {device}")
        ordinal = int(device.split(":", 1)[1]) if ":" in device else 0
        lib = _native.load()
        handle = ctypes.c_void_p()
        status = lib.affon_rocm_session_create(ordinal, ctypes.byref(handle))
        if status != _native.OK:
            message = _native.last_error()
            raise RuntimeError(message if "backend unavailable" in message else f"backend unavailable: {message}")
        self.device = device
        self._handle = handle.value
        self._executables: dict[tuple, "Executable"] = {}
        self._buffers: "weakref.WeakSet[_Buffer]" = weakref.WeakSet()

    @property
    def stream(self) -> int:
        return _native.load().affon_rocm_session_stream(self._handle)

    def _check_open(self) -> None:
        if self._handle is None:
            raise RuntimeError("session has been disposed")

    def empty(self, dtype: str, shape: Sequence[int]) -> Tensor:
        self._check_open()
        if dtype not in DTYPES:
            raise TypeError(f"unsupported dtype: {dtype}")
        shape = tuple(int(d) for d in shape)
        count = int(np.prod(shape)) if shape else 1
        strides = tuple(int(np.prod(shape[i + 1:])) for i in range(len(shape)))
        return Tensor(self, _Buffer(self, count * _ITEMSIZE[dtype]), dtype, shape, strides)

    def tensor(self, values: Any, dtype: str = "f32") -> Tensor:
        """Creates a device tensor from host values (nested lists or arrays)."""
        storage = host_storage(values, dtype)
        t = self.empty(dtype, storage.shape)
        _native.check(_native.load().affon_rocm_memcpy_h2d(self._handle, t._buffer.ptr, storage.ctypes.data,
                                                           storage.nbytes), "upload")
        return t

    def randn(self, shape: Sequence[int], *, seed: int = 0, mean: float = 0.0, std: float = 1.0,
              dtype: str = "f32") -> Tensor:
        """Tensor.randn (src/js/compute/program.ts:339-345) with mean/std as
        the "normal" initializer (program.ts:1413)."""
        from .generator import normal_f32
        if dtype not in ("f32", "bf16"):
            raise TypeError("Tensor.randn requires a floating-point dtype")
        shape = tuple(int(d) for d in shape)
        values = normal_f32(seed, int(np.prod(shape)), mean, std).reshape(shape)
        return self.from_bytes(bf16_bits(values) if dtype == "bf16" else values, TensorSpec(dtype, shape))

    def from_bytes(self, data: bytes | np.ndarray, spec: TensorSpec) -> Tensor:
        """Creates a device tensor from raw little-endian storage bytes."""
        if isinstance(data, np.ndarray):
            raw = np.ascontiguousarray(data).reshape(-1).view(np.uint8).view(_STORAGE[spec.dtype])
        else:
            raw = np.frombuffer(bytes(data), dtype=_STORAGE[spec.dtype])
        expected = int(np.prod(spec.shape)) if spec.shape else 1
        if raw.size != expected:
            raise TypeError("byte length does not match tensor spec")
        t = self.empty(spec.dtype, spec.shape)
        _native.check(_native.load().affon_rocm_memcpy_h2d(self._handle, t._buffer.ptr, raw.ctypes.data,
                                                           raw.nbytes), "upload")
        return t

    def synchronize(self) -> None:
        self._check_open()
        _native.check(_native.load().affon_rocm_synchronize(self._handle), "synchronize")

    def compile(self, source: "Program", **options: Any) -> "Executable":
        normalized = normalized_compile_options(options)
        key = (id(source), tuple(sorted(normalized.items())))
        cached = self._executables.get(key)
        if cached is not None and cached.program is source:
            return cached
        executable = Executable(self, source, normalized)
        self._executables[key] = executable
        return executable

    def dispose(self) -> None:
        """Ends the session. Device memory of tensors still alive is freed
        with it; those tensors then report that they have been disposed."""
        if self._handle is not None:
            _native.load().affon_rocm_session_destroy(self._handle)
            self._handle = None
            for buffer in list(self._buffers):
                buffer.ptr = None
            self._buffers = weakref.WeakSet()

    def __enter__(self) -> "Session":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.dispose()


def normalized_compile_options(options: Mapping[str, Any]) -> dict[str, str]:
    """src/js/compute/program.ts:75-102 for the options this path reads."""
    result = {"optimizationLevel": options.get("optimizationLevel", "safe"),
              "numericalPolicy": options.get("numericalPolicy", "backend_equivalent"),
              "explanationLevel": options.get("explanationLevel", "summary")}
    for name, values in COMPILE_OPTION_VALUES.items():
        if result[name] not in values:
            raise TypeError(f"unsupported {name}: {result[name]}")
    unknown = set(options) - set(COMPILE_OPTION_VALUES)
    if unknown:
        raise TypeError(f"unsupported compile option: {sorted(unknown)[0]}")
    return result


def policy_code(policy: str) -> int:
    return _POLICY[policy]


# ---- formal Programs -------------------------------------------------------

class FormalTensor:
    """A symbolic value inside a Program under construction."""

    _ids = itertools.count()

    def __init__(self, builder: "ProgramBuilder", spec: TensorSpec, node: int):
        self.builder = builder
        self.spec = spec
        self.node = node

    @property
    def shape(self) -> tuple[int, ...]:
        return self.spec.shape

    @property
    def dtype(self) -> str:
        return self.spec.dtype


class ProgramBuilder:
    def __init__(self, name: str):
        self.name = name
        self.nodes: list[dict[str, Any]] = []

    def argument(self, name: str, spec: TensorSpec) -> FormalTensor:
        if any(n["kind"] == "argument" and n["name"] == name for n in self.nodes):
            raise TypeError(f"duplicate argument: {name}")
        self.nodes.append({"id": len(self.nodes), "kind": "argument", "name": name, "spec": spec})
        return FormalTensor(self, spec, len(self.nodes) - 1)

    def emit(self, op: str, operands: Sequence[FormalTensor], spec: TensorSpec, options: dict[str, Any]) -> FormalTensor:
        self.nodes.append({"id": len(self.nodes), "kind": "operation", "op": op,
                           "operands": [o.node for o in operands], "spec": spec, "options": dict(options)})
        return FormalTensor(self, spec, len(self.nodes) - 1)


@dataclass
class Program:
    name: str
    nodes: list[dict[str, Any]]
    outputs: list[int]
    multiple: bool = False  # the body returned a sequence of outputs

    @property
    def output(self) -> int:
        return self.outputs[0]

    def inspect(self) -> dict[str, Any]:
        return {"name": self.name, "nodes": [dict(n) for n in self.nodes], "outputs": list(self.outputs)}


def program(name: str, fn: Callable[[ProgramBuilder], Any]) -> Program:
    """Authors a Program; the body returns one formal tensor or a sequence of
    them (src/js/compute/program.ts:1704-1737: Programs may return several
    outputs)."""
    builder = ProgramBuilder(name)
    result = fn(builder)
    multiple = isinstance(result, (list, tuple))
    results = list(result) if multiple else [result]
    if not results or any(not isinstance(r, FormalTensor) or r.builder is not builder for r in results):
        raise TypeError("program body must return formal tensors of the same Program")
    return Program(name, builder.nodes, [r.node for r in results], multiple)


class Executable:
    """A compiled Program: validated once, run with named arguments."""

    def __init__(self, session: Session, source: Program, options: dict[str, str]):
        from . import lowering, ops  # local: ops imports core
        self.session = session
        self.program = source
        self.options = options
        self._ops = ops
        self._steps = lowering.lower(source.nodes, source.outputs)
        # Selection happens at compile time from the formal specs, so an
        # unsupported policy fails here as in the reference compiler.
        self._implementations = [self._select(step) for step in self._steps]

    def _select(self, step: Any) -> str:
        specs = [self.program.nodes[i]["spec"] for i in step.operands]
        policy = self.options["numericalPolicy"]
        if step.kind == "quantized_matmul":
            return self._ops.select_for_specs(specs, step.options, policy)
        if step.kind in ("rms_norm", "softmax", "index_select"):
            return f"rocm_{step.kind}"
        if step.kind == "grouped":
            members = [[self.program.nodes[i]["spec"] for i in m.operands] for m in step.members]
            return self._ops.grouped_select_for_specs(members, step.options, policy)
        return self._ops.fused_select_for_specs(step.kind, specs, step.options, policy)

    def explain(self) -> dict[str, Any]:
        names = {"quantized_matmul": "quantized_matmul", "bias": "quantized_matmul+add",
                 "silu_gate": "quantized_matmul+silu+quantized_matmul+mul", "rms_norm": "rms_norm",
                 "softmax": "softmax", "index_select": "index_select"}

        def op(step):
            if step.kind == "grouped":
                return "grouped(" + ",".join(names[m.kind] for m in step.members) + ")"
            return names[step.kind]
        physical = [{"op": op(step), "implementation_id": impl, "implementation_version": 1,
                     "options": step.options, "nodes": step.nodes}
                    for step, impl in zip(self._steps, self._implementations)]
        return {"program": self.program.name, "device": self.session.device, "options": dict(self.options),
                "executable": {"physical_nodes": physical}}

    def run(self, arguments: Mapping[str, Tensor]) -> Tensor:
        values: dict[int, Tensor] = {}
        for node in self.program.nodes:
            if node["kind"] == "argument":
                if node["name"] not in arguments:
                    raise TypeError(f"missing argument: {node['name']}")
                value = arguments[node["name"]]
                if not isinstance(value, Tensor) or value.session is not self.session:
                    raise TypeError("arguments must be tensors of the same Session")
                if value.spec != node["spec"]:
                    raise TypeError(f"argument {node['name']} does not match its spec")
                values[node["id"]] = value
        policy = self.options["numericalPolicy"]
        for step in self._steps:
            operands = [values[i] for i in step.operands]
            if step.kind == "rms_norm":
                values[step.node] = self._ops._run_rms_norm(operands[0], step.options["epsilon"])
                continue
            if step.kind == "softmax":
                values[step.node] = self._ops._run_softmax(operands[0])
                continue
            if step.kind == "index_select":
                values[step.node] = self._ops._run_index_select(operands[0], step.options["axis"], operands[1])
                continue
            bits, group = step.options["bits"], step.options["group_size"]
            if step.kind == "quantized_matmul":
                values[step.node] = self._ops._run_quantized_matmul(*operands, bits, group, policy=policy)
            elif step.kind == "grouped":
                projections = [tuple(values[i] for i in m.operands[1:]) for m in step.members]
                outs = self._ops.quantized_matmul_grouped(operands[0], projections, bits=bits, group_size=group,
                                                          policy=policy)
                for m, out in zip(step.members, outs):
                    values[m.node] = out
            elif step.kind == "bias":
                self._ops._check_bias(operands[4], operands[1].shape[0])
                epi = self._ops._epilogue(output_bias=operands[4])
                values[step.node] = self._ops._run_fused(*operands[:4], bits, group, epi, policy=policy,
                                                         implementation="auto", out=None)
            else:
                epi = self._ops._epilogue(up=tuple(operands[4:7]))
                values[step.node] = self._ops._run_fused(*operands[:4], bits, group, epi, policy=policy,
                                                         implementation="auto", out=None)
        results = [values[i] for i in self.program.outputs]
        return results if self.program.multiple else results[0]
