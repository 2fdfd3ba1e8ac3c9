"""Safetensors checkpoints onto the rocm device, and the MLX-affine adapter.

``inspect`` and ``load`` follow the reference's ``checkpoint.inspect`` /
``checkpoint.load`` reader (src/js/compute/native.zig:1772-1885,
checkpointDType at :1658-1665): the same header rules, checked in the same
order, with the same messages. The reference loads onto its CPU session; here
tensors are created on the given rocm Session (device-resident), read with a
memory map so a tensor is copied once, host to device. F64 and I64 entries
are valid in a header (``inspect`` lists them) but have no rocm tensor type,
so loading one raises.

``quantized_linears`` is the MLX-affine adapter the reference describes
(docs/core/quantized-inference.md:85-112; tools/test-quantized-checkpoint.py:
21-55): a quantized linear layer is a ``<prefix>.weight`` U32 tensor
[out, in/P] with ``<prefix>.scales`` and ``<prefix>.biases`` [out, in/g] of
one floating dtype. bits and group_size come from configuration (header
shapes alone do not identify the scheme), and only layers that have all
three tensors are bound; each is applied with ``quantized_matmul``.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass
from typing import Any, Iterable, Mapping, Sequence

import numpy as np

from .core import Session, Tensor, TensorSpec

# Header dtype names the reference accepts (native.zig:1658-1665) and their
# element sizes; the rocm tensor dtype for the ones a device tensor can hold.
_DTYPE_SIZE = {"BF16": 2, "F32": 4, "F64": 8, "U32": 4, "I64": 8}
_ROCM_DTYPE = {"BF16": "bf16", "F32": "f32", "U32": "u32"}
_MAX_HEADER = 16 * 1024 * 1024
_MAX_USIZE = (1 << 64) - 1


class CheckpointError(RuntimeError):
    """A checkpoint file or request the reader rejects (reference messages)."""


@dataclass(frozen=True)
class Entry:
    name: str
    dtype: str
    shape: tuple[int, ...]
    start: int  # byte offsets into the data section
    end: int


def _read_header(path: str) -> tuple[int, dict[str, Any], int]:
    """(header size, parsed header, data-section size), or CheckpointError."""
    if not isinstance(path, (str, os.PathLike)):
        raise TypeError("checkpoint.load expects a string path")
    try:
        f = open(path, "rb")
    except OSError:
        raise CheckpointError("checkpoint.load failed to open file") from None
    with f:
        try:
            file_size = os.fstat(f.fileno()).st_size
        except OSError:
            raise CheckpointError("checkpoint.load failed to stat file") from None
        if file_size < 8:
            raise CheckpointError("checkpoint.load file is too small")
        prefix = f.read(8)
        if len(prefix) != 8:
            raise CheckpointError("checkpoint.load truncated header")
        header_size = int.from_bytes(prefix, "little")
        if header_size > _MAX_HEADER or header_size > file_size - 8:
            raise CheckpointError("checkpoint.load has an invalid header")
        raw = f.read(header_size)
        if len(raw) != header_size:
            raise CheckpointError("checkpoint.load truncated header")
    try:
        parsed = json.loads(raw)
    except (UnicodeDecodeError, ValueError):
        raise CheckpointError("checkpoint.load has invalid metadata") from None
    return header_size, parsed, file_size - 8 - header_size


def _is_int(value: Any) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def _entries(parsed: Any, raw_size: int) -> list[Entry]:
    """Validates every header entry in file order (native.zig:1821-1853)."""
    if not isinstance(parsed, dict):
        raise CheckpointError("checkpoint.load header must be an object")
    entries = []
    for name, metadata in parsed.items():
        if not isinstance(metadata, dict):
            raise CheckpointError("checkpoint.load metadata must be an object")
        if name == "__metadata__":
            if any(not isinstance(v, str) for v in metadata.values()):
                raise CheckpointError("checkpoint.load __metadata__ values must be strings")
            continue
        if "dtype" not in metadata:
            raise CheckpointError("checkpoint.load metadata is missing dtype")
        dtype = metadata["dtype"]
        if not isinstance(dtype, str):
            raise CheckpointError("checkpoint.load dtype must be a string")
        if dtype not in _DTYPE_SIZE:
            raise CheckpointError("checkpoint.load has unsupported dtype")
        if "shape" not in metadata:
            raise CheckpointError("checkpoint.load metadata is missing shape")
        shape = metadata["shape"]
        if not isinstance(shape, list):
            raise CheckpointError("checkpoint.load shape must be an array")
        elements = 1
        for d in shape:
            if not _is_int(d) or d < 0:
                raise CheckpointError("checkpoint.load shape must contain non-negative integers")
            if d > _MAX_USIZE:
                raise CheckpointError("checkpoint.load dimension is too large")
            elements *= d
            if elements > _MAX_USIZE:
                raise CheckpointError("checkpoint.load shape is too large")
        if "data_offsets" not in metadata:
            raise CheckpointError("checkpoint.load metadata is missing offsets")
        offsets = metadata["data_offsets"]
        if not isinstance(offsets, list) or len(offsets) != 2:
            raise CheckpointError("checkpoint.load expects two offsets")
        if any(not _is_int(v) or v < 0 for v in offsets):
            raise CheckpointError("checkpoint.load offsets must be non-negative integers")
        start, end = offsets
        if start > _MAX_USIZE or end > _MAX_USIZE:
            raise CheckpointError("checkpoint.load offset is too large")
        if end < start or end > raw_size:
            raise CheckpointError("checkpoint.load offsets exceed file size")
        byte_count = elements * _DTYPE_SIZE[dtype]
        if byte_count > _MAX_USIZE:
            raise CheckpointError("checkpoint.load tensor is too large")
        if byte_count != end - start:
            raise CheckpointError("checkpoint.load tensor byte length mismatch")
        entries.append(Entry(name, dtype, tuple(shape), start, end))
    return entries


def _selection(names: Any) -> list[str] | None:
    if names is None:
        return None
    if not isinstance(names, (list, tuple)):
        raise TypeError("checkpoint.load names must be an array")
    selected: list[str] = []
    for name in names:
        if not isinstance(name, str):
            raise TypeError("checkpoint names must be strings")
        if name in selected:
            raise CheckpointError("Duplicate checkpoint name")
        selected.append(name)
    return selected


def inspect(path: str) -> dict[str, dict[str, Any]]:
    """{name: {"shape": [...], "dtype": "BF16" | ...}} of every tensor."""
    _, parsed, raw_size = _read_header(path)
    return {e.name: {"shape": list(e.shape), "dtype": e.dtype} for e in _entries(parsed, raw_size)}


def load(session: Session, path: str, names: Sequence[str] | None = None) -> dict[str, Tensor]:
    """Device tensors for every tensor of the file, or for the requested names
    (all of which must exist)."""
    header_size, parsed, raw_size = _read_header(path)
    selected = _selection(names)
    entries = _entries(parsed, raw_size)
    wanted = [e for e in entries if selected is None or e.name in selected]
    if selected is not None and len(wanted) != len(selected):
        raise CheckpointError("Missing requested checkpoint tensor")
    data = np.memmap(path, dtype=np.uint8, mode="r", offset=8 + header_size, shape=(raw_size,)) if raw_size else None
    result: dict[str, Tensor] = {}
    for e in wanted:
        dtype = _ROCM_DTYPE.get(e.dtype)
        if dtype is None:
            raise TypeError(f"checkpoint.load: {e.dtype} tensor {e.name!r} has no rocm tensor type")
        raw = data[e.start:e.end] if e.end > e.start else np.zeros(0, np.uint8)
        result[e.name] = session.from_bytes(np.asarray(raw), TensorSpec(dtype, e.shape))
    return result


# ---- MLX-affine quantized linear layers -------------------------------------------------------

def quantization_config(config: Mapping[str, Any] | str) -> tuple[int, int]:
    """(bits, group_size) from an MLX model configuration: the
    ``"quantization": {"bits": b, "group_size": g}`` entry of config.json (a
    path or the parsed mapping)."""
    if isinstance(config, (str, os.PathLike)):
        with open(config) as f:
            config = json.load(f)
    q = config.get("quantization") if isinstance(config, Mapping) else None
    if not isinstance(q, Mapping) or "bits" not in q or "group_size" not in q:
        raise CheckpointError("model configuration has no quantization {bits, group_size}")
    bits, group = q["bits"], q["group_size"]
    if not _is_int(bits) or bits not in (2, 4, 8):
        raise TypeError("quantized_matmul bits must be 2, 4, or 8")
    if not _is_int(group) or group <= 0:
        raise TypeError("quantized_matmul group_size must be a positive integer")
    return bits, group


@dataclass(frozen=True)
class LinearSpec:
    prefix: str
    out_features: int
    in_features: int
    param_dtype: str  # "BF16" or "F32"


def quantized_layer_specs(header: Mapping[str, Mapping[str, Any]], bits: int, group_size: int,
                          prefixes: Iterable[str] | None = None) -> list[LinearSpec]:
    """The quantized linear layers of an inspected header. Without prefixes,
    every ``<p>.weight`` of dtype U32 that has ``<p>.scales`` and ``<p>.biases``
    is one; named prefixes must be complete layers. Shapes must agree with
    (bits, group_size): weight [out, in/P], scales and biases [out, in/g] of
    one floating dtype."""
    if bits not in (2, 4, 8):
        raise TypeError("quantized_matmul bits must be 2, 4, or 8")
    if not _is_int(group_size) or group_size <= 0:
        raise TypeError("quantized_matmul group_size must be a positive integer")
    per_word = 32 // bits
    if prefixes is None:
        candidates = [n[:-len(".weight")] for n, spec in header.items()
                      if n.endswith(".weight") and spec.get("dtype") == "U32"
                      and n[:-len(".weight")] + ".scales" in header and n[:-len(".weight")] + ".biases" in header]
    else:
        candidates = list(prefixes)
    specs = []
    for p in candidates:
        names = (p + ".weight", p + ".scales", p + ".biases")
        if any(n not in header for n in names):
            raise CheckpointError(f"{p}: a quantized linear layer needs .weight, .scales and .biases")
        w, s, b = (header[n] for n in names)
        if w["dtype"] != "U32" or len(w["shape"]) != 2:
            raise CheckpointError(f"{p}.weight must be a rank-2 U32 tensor")
        if s["dtype"] != b["dtype"] or s["dtype"] not in ("BF16", "F32"):
            raise CheckpointError(f"{p}: scales and biases must share one dtype, BF16 or F32")
        out_features, words = w["shape"]
        in_features = words * per_word
        if in_features % group_size != 0 or list(s["shape"]) != [out_features, in_features // group_size] \
                or list(b["shape"]) != list(s["shape"]):
            raise CheckpointError(f"{p}: shapes do not match bits={bits}, group_size={group_size}")
        specs.append(LinearSpec(p, out_features, in_features, s["dtype"]))
    return specs


@dataclass
class QuantizedLinear:
    """One bound layer: y[M, out] = x[M, in] . dequant(weight)^T, f32."""
    prefix: str
    packed: Tensor
    scales: Tensor
    biases: Tensor
    bits: int
    group_size: int

    @property
    def in_features(self) -> int:
        return self.packed.shape[1] * (32 // self.bits)

    @property
    def out_features(self) -> int:
        return self.packed.shape[0]

    def __call__(self, x: Tensor) -> Tensor:
        from .ops import quantized_matmul
        return quantized_matmul(x, self.packed, self.scales, self.biases, bits=self.bits, group_size=self.group_size)


def quantized_linears(session: Session, path: str, *, bits: int, group_size: int,
                      prefixes: Iterable[str] | None = None) -> dict[str, QuantizedLinear]:
    """Binds the checkpoint's quantized linear layers to device tensors."""
    header = inspect(path)
    specs = quantized_layer_specs(header, bits, group_size, prefixes)
    names = [n for spec in specs for n in (spec.prefix + ".weight", spec.prefix + ".scales", spec.prefix + ".biases")]
    tensors = load(session, path, names) if names else {}
    return {spec.prefix: QuantizedLinear(spec.prefix, tensors[spec.prefix + ".weight"],
                                         tensors[spec.prefix + ".scales"], tensors[spec.prefix + ".biases"],
                                         bits, group_size)
            for spec in specs}
