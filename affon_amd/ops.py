"""``affon:ops`` subset for the weight-quantized linear path on the rocm device.

``quantized_matmul`` mirrors src/js/ops.ts:69-79 and the formal validation of
src/js/compute/program.ts:481-494 (same checks, same TypeError messages):
four rank-two operands, f32/bf16 input, u32 packed weights, matching f32/bf16
scales and biases, bits in {2, 4, 8}, a positive integer group_size, K divisible
into whole words and groups, exact packed and parameter shapes; the result is
f32 [M, N]. Evaluated operands run immediately on the Session's stream;
formal operands add a node to the Program being built.

``quantize`` and ``dequantize`` have no counterpart op in the reference (it
packs only in test harnesses and states dequantization as a formula,
docs/core/quantized-inference.md:59-61); they produce and expand the same
packed format.

``transpose`` and ``slice`` create strided views without copying, as the
reference's view ops do for evaluated tensors.

``add``, ``mul`` and ``silu`` (src/js/ops.ts:51,53,91) author formal nodes
only: on the rocm device they run as quantized_matmul output epilogues (an
output bias, the SiLU-gated product of two projections; see lowering.py),
and ``quantized_linear`` / ``quantized_silu_gate`` are their evaluated forms.
"""
from __future__ import annotations

import ctypes
from typing import Any, Mapping, Sequence

import numpy as np

from . import _native
from .core import FormalTensor, Tensor, TensorSpec, policy_code

_IMPLEMENTATIONS = {
    "auto": _native.IMPL_AUTO,
    "generic": _native.IMPL_GENERIC,
    "gemv": _native.IMPL_GEMV,
    "gemv_mfma": _native.IMPL_GEMV_MFMA,
    "mfma": _native.IMPL_MFMA,
}


def _options(options: Any, bits: Any, group_size: Any) -> dict[str, Any]:
    if options is None:
        options = {"bits": bits, "group_size": group_size}
    elif not isinstance(options, Mapping):
        raise TypeError("quantized_matmul options must be an object")
    return dict(options)


def _validate(specs: Sequence[TensorSpec], config: Mapping[str, Any]) -> TensorSpec:
    """src/js/compute/program.ts:483-493, message for message."""
    bits = config.get("bits") if config else None
    if not config or bits not in (2, 4, 8) or isinstance(bits, bool):
        raise TypeError("quantized_matmul bits must be 2, 4, or 8")
    group = config.get("group_size")
    if not isinstance(group, int) or isinstance(group, bool) or group <= 0:
        raise TypeError("quantized_matmul group_size must be a positive integer")
    if len(specs) != 4 or any(len(s.shape) != 2 for s in specs):
        raise TypeError("quantized_matmul requires four rank-two tensors")
    x, w, s, b = specs
    if x.dtype not in ("f32", "bf16") or w.dtype != "u32" or s.dtype not in ("f32", "bf16") or b.dtype != s.dtype:
        raise TypeError("quantized_matmul requires f32/bf16 input, u32 weights, and matching f32/bf16 scales and biases")
    rows, inner = x.shape
    outputs = w.shape[0]
    per_word = 32 // bits
    if (not rows or not inner or not outputs or inner % per_word or inner % group or
            w.shape[1] != inner // per_word or s.shape[0] != outputs or s.shape[1] != inner // group or
            b.shape[0] != outputs or b.shape[1] != inner // group):
        raise TypeError("quantized_matmul packed or group dimensions do not match input features")
    return TensorSpec("f32", (rows, outputs))


def quantized_matmul(input: Any, packed: Any, scales: Any, biases: Any, options: Mapping[str, Any] | None = None,
                     *, bits: int | None = None, group_size: int | None = None) -> Any:
    """Y[M,N] = input[M,K] . dequant(packed, scales, biases)^T with f32 accumulation."""
    operands = (input, packed, scales, biases)
    config = _options(options, bits, group_size)
    formal = [isinstance(o, FormalTensor) for o in operands]
    if any(formal) and not all(formal):
        raise TypeError("quantized_matmul cannot mix formal and evaluated tensors")
    if all(formal):
        builder = operands[0].builder
        if any(o.builder is not builder for o in operands):
            raise TypeError("quantized_matmul operands must belong to the same Program")
        result = _validate([o.spec for o in operands], config)
        return builder.emit("quantized_matmul", operands, result,
                            {"bits": config["bits"], "group_size": config["group_size"]})
    if not all(isinstance(o, Tensor) for o in operands):
        raise TypeError("quantized_matmul requires tensors")
    session = operands[0].session
    if any(o.session is not session for o in operands):
        raise TypeError("quantized_matmul operands must belong to the same Session")
    _validate([o.spec for o in operands], config)
    return _run_quantized_matmul(*operands, config["bits"], config["group_size"])


def _descriptor(x: Tensor, w: Tensor, s: Tensor, b: Tensor, bits: int, group: int, out: Tensor | None,
                implementation: str, policy: str) -> _native.QmmDesc:
    desc = _native.QmmDesc()
    desc.input, desc.packed, desc.scales, desc.biases = x.view(), w.view(), s.view(), b.view()
    if out is not None:
        desc.output = out.data_ptr
        desc.output_bytes = out._buffer.nbytes - out.offset * 4
    desc.bits = bits
    desc.group_size = group
    desc.implementation = _IMPLEMENTATIONS[implementation]
    desc.numerical_policy = policy_code(policy)
    return desc


def _run_quantized_matmul(x: Tensor, w: Tensor, s: Tensor, b: Tensor, bits: int, group: int, *,
                          policy: str = "backend_equivalent", implementation: str = "auto",
                          out: Tensor | None = None) -> Tensor:
    session = x.session
    if out is None:
        out = session.empty("f32", (x.shape[0], w.shape[0]))
    desc = _descriptor(x, w, s, b, bits, group, out, implementation, policy)
    _native.check(_native.load().affon_rocm_quantized_matmul(session._handle, ctypes.byref(desc)),
                  "Program execution failed")
    return out


def quantized_matmul_into(out: Tensor, input: Tensor, packed: Tensor, scales: Tensor, biases: Tensor, *,
                          bits: int, group_size: int, implementation: str = "auto",
                          policy: str = "backend_equivalent") -> Tensor:
    """Runs into a caller-owned f32 [M,N] output (no allocation), optionally
    forcing one physical implementation."""
    _validate([t.spec for t in (input, packed, scales, biases)], {"bits": bits, "group_size": group_size})
    if out.dtype != "f32" or out.shape != (input.shape[0], packed.shape[0]) or not out.is_contiguous():
        raise TypeError("quantized_matmul output must be a contiguous f32 [M,N] tensor")
    return _run_quantized_matmul(input, packed, scales, biases, bits, group_size, policy=policy,
                                 implementation=implementation, out=out)


# ---- fused output epilogues ------------------------------------------------
# The reference authors a linear layer's output bias and the SiLU-gated
# feed-forward product as separate ops after quantized_matmul
# (docs/core/quantized-inference.md:37-42, packages/@affon/models/src/llama/
# model.ts:82); these run them in the kernel that stores the output.

def _check_triple(name: str, triple: Any) -> tuple[Tensor, Tensor, Tensor]:
    if not isinstance(triple, (tuple, list)) or len(triple) != 3 or not all(isinstance(t, Tensor) for t in triple):
        raise TypeError(f"{name} must be a (packed, scales, biases) tuple of tensors")
    return tuple(triple)  # type: ignore[return-value]


def _epilogue(output_bias: Tensor | None = None, up: tuple[Tensor, Tensor, Tensor] | None = None) -> _native.Epilogue:
    epi = _native.Epilogue()
    epi.kind = _native.EPILOGUE_NONE
    if output_bias is not None:
        epi.kind = _native.EPILOGUE_BIAS
        epi.bias = output_bias.data_ptr
        epi.bias_bytes = output_bias._buffer.nbytes - output_bias.offset * (2 if output_bias.dtype == "bf16" else 4)
        epi.bias_dtype = {"f32": _native.F32, "bf16": _native.BF16}.get(output_bias.dtype, -1)
    if up is not None:
        epi.kind = _native.EPILOGUE_SILU_GATE
        epi.up_packed, epi.up_scales, epi.up_biases = (t.view() for t in up)
    return epi


def _check_bias(bias: Tensor, outputs: int) -> None:
    if bias.dtype not in ("f32", "bf16") or len(bias.shape) != 1 or bias.shape[0] != outputs or not bias.is_contiguous():
        raise TypeError("quantized_matmul output bias must be a contiguous f32/bf16 [N] tensor")


def _run_fused(x: Tensor, w: Tensor, s: Tensor, b: Tensor, bits: int, group: int, epi: _native.Epilogue, *,
               policy: str, implementation: str, out: Tensor | None) -> Tensor:
    session = x.session
    if out is None:
        out = session.empty("f32", (x.shape[0], w.shape[0]))
    elif out.dtype != "f32" or out.shape != (x.shape[0], w.shape[0]) or not out.is_contiguous():
        raise TypeError("quantized_matmul output must be a contiguous f32 [M,N] tensor")
    desc = _descriptor(x, w, s, b, bits, group, out, implementation, policy)
    _native.check(_native.load().affon_rocm_quantized_matmul_fused(session._handle, ctypes.byref(desc),
                                                                    ctypes.byref(epi)), "Program execution failed")
    return out


def quantized_linear(input: Tensor, packed: Tensor, scales: Tensor, biases: Tensor, output_bias: Tensor, *,
                     bits: int, group_size: int, implementation: str = "auto", policy: str = "backend_equivalent",
                     out: Tensor | None = None) -> Tensor:
    """``add(quantized_matmul(input, packed, scales, biases), output_bias)`` in
    one launch: Y[m,n] = qmm[m,n] + output_bias[n] (one f32 add, the same
    rounding as the separate ``add``)."""
    operands = (input, packed, scales, biases, output_bias)
    if not all(isinstance(o, Tensor) for o in operands):
        raise TypeError("quantized_linear requires evaluated tensors")
    if any(o.session is not input.session for o in operands):
        raise TypeError("quantized_linear operands must belong to the same Session")
    _validate([t.spec for t in operands[:4]], {"bits": bits, "group_size": group_size})
    _check_bias(output_bias, packed.shape[0])
    return _run_fused(input, packed, scales, biases, bits, group_size, _epilogue(output_bias=output_bias),
                      policy=policy, implementation=implementation, out=out)


def quantized_silu_gate(input: Tensor, gate: Any, up: Any, *, bits: int, group_size: int,
                        implementation: str = "auto", policy: str = "backend_equivalent",
                        out: Tensor | None = None) -> Tensor:
    """``mul(silu(quantized_matmul(input, *gate)), quantized_matmul(input, *up))``:
    the SiLU-gated feed-forward input. ``gate`` and ``up`` are (packed, scales,
    biases) tuples of the same shapes and dtypes. Runs in one launch where the
    selected kernel pairs rows of both projections (M = 1), else in two, the
    second storing silu(gate) * up."""
    gate = _check_triple("gate", gate)
    up = _check_triple("up", up)
    operands = (input, *gate, *up)
    if any(o.session is not input.session for o in operands):
        raise TypeError("quantized_silu_gate operands must belong to the same Session")
    _validate([t.spec for t in (input, *gate)], {"bits": bits, "group_size": group_size})
    _validate([t.spec for t in (input, *up)], {"bits": bits, "group_size": group_size})
    if tuple(t.spec for t in gate) != tuple(t.spec for t in up):
        raise TypeError("quantized_silu_gate gate and up projections must have the same shapes and dtypes")
    return _run_fused(input, *gate, bits, group_size, _epilogue(up=up), policy=policy,
                      implementation=implementation, out=out)


def fused_plan(input: Tensor, packed: Tensor, scales: Tensor, biases: Tensor, *, bits: int, group_size: int,
               output_bias: Tensor | None = None, up: Any = None, implementation: str = "auto",
               policy: str = "backend_equivalent") -> str:
    """The launches a fused call makes: implementation ids with the epilogue
    in brackets, separated by ';'."""
    desc = _descriptor(input, packed, scales, biases, bits, group_size, None, implementation, policy)
    desc.output = 1
    desc.output_bytes = input.shape[0] * packed.shape[0] * 4
    epi = _epilogue(output_bias=output_bias, up=_check_triple("up", up) if up is not None else None)
    name = ctypes.create_string_buffer(256)
    _native.check(_native.load().affon_rocm_quantized_matmul_fused_select(ctypes.byref(desc), ctypes.byref(epi),
                                                                           name, 256), "select")
    return name.value.decode()


def _projection_parts(projection: Any) -> tuple[tuple[Tensor, Tensor, Tensor], Tensor | None]:
    if not isinstance(projection, (tuple, list)) or len(projection) not in (3, 4) or \
            not all(isinstance(t, Tensor) for t in projection):
        raise TypeError("a grouped projection is (packed, scales, biases) or (packed, scales, biases, output_bias)")
    return tuple(projection[:3]), (projection[3] if len(projection) == 4 else None)  # type: ignore[return-value]


def _grouped_arrays(input: Tensor, projections: Sequence[Any], bits: int, group: int, outs: Sequence[Tensor] | None,
                    implementation: str, policy: str):
    if not projections:
        raise TypeError("quantized_matmul_grouped needs at least one projection")
    descs = (_native.QmmDesc * len(projections))()
    epis = (_native.Epilogue * len(projections))()
    for i, projection in enumerate(projections):
        (w, s, b), bias = _projection_parts(projection)
        if any(t.session is not input.session for t in (w, s, b)):
            raise TypeError("quantized_matmul_grouped operands must belong to the same Session")
        _validate([input.spec, w.spec, s.spec, b.spec], {"bits": bits, "group_size": group})
        if bias is not None:
            _check_bias(bias, w.shape[0])
        descs[i] = _descriptor(input, w, s, b, bits, group, outs[i] if outs is not None else None, implementation,
                               policy)
        if outs is None:
            descs[i].output = 1
            descs[i].output_bytes = input.shape[0] * w.shape[0] * 4
        epis[i] = _epilogue(output_bias=bias)
    return descs, epis


def quantized_matmul_grouped(input: Tensor, projections: Sequence[Any], *, bits: int, group_size: int,
                             implementation: str = "auto", policy: str = "backend_equivalent") -> list[Tensor]:
    """Several projections of one input (a decoder block's query, key and
    value), each ``quantized_matmul(input, packed, scales, biases)`` plus an
    optional output bias; one launch where the M = 1 kernel takes them all."""
    if not isinstance(input, Tensor):
        raise TypeError("quantized_matmul_grouped requires evaluated tensors")
    outs = [input.session.empty("f32", (input.shape[0], _projection_parts(p)[0][0].shape[0])) for p in projections]
    descs, epis = _grouped_arrays(input, projections, bits, group_size, outs, implementation, policy)
    _native.check(_native.load().affon_rocm_quantized_matmul_grouped(input.session._handle, descs, epis,
                                                                      len(projections)), "Program execution failed")
    return outs


def grouped_plan(input: Tensor, projections: Sequence[Any], *, bits: int, group_size: int,
                 implementation: str = "auto", policy: str = "backend_equivalent") -> str:
    descs, epis = _grouped_arrays(input, projections, bits, group_size, None, implementation, policy)
    name = ctypes.create_string_buffer(512)
    _native.check(_native.load().affon_rocm_quantized_matmul_grouped_select(descs, epis, len(projections), name, 512),
                  "select")
    return name.value.decode()


def selected_implementation(input: Tensor, packed: Tensor, scales: Tensor, biases: Tensor, *, bits: int,
                            group_size: int, implementation: str = "auto",
                            policy: str = "backend_equivalent") -> str:
    desc = _descriptor(input, packed, scales, biases, bits, group_size, None, implementation, policy)
    # Selection validates the output too; describe a conforming one.
    desc.output = 1
    desc.output_bytes = input.shape[0] * packed.shape[0] * 4
    name = ctypes.create_string_buffer(128)
    _native.check(_native.load().affon_rocm_quantized_matmul_select(ctypes.byref(desc), name, 128), "select")
    return name.value.decode()


def _dense_view(spec: TensorSpec, address: int) -> _native.View:
    """A dense row-major view at an aligned address, as a Program's arguments
    are when run (selection reads only shapes, strides and alignment)."""
    rows, cols = spec.shape
    itemsize = 2 if spec.dtype == "bf16" else 4
    code = {"f32": _native.F32, "bf16": _native.BF16, "u32": _native.U32}[spec.dtype]
    return _native.View(address, rows * cols * itemsize, 0, (ctypes.c_int64 * 2)(rows, cols),
                        (ctypes.c_int64 * 2)(cols, 1), code)


def select_for_specs(specs: Sequence[TensorSpec], options: Mapping[str, Any], policy: str) -> str:
    """Compile-time selection from formal specs: dense row-major operands at
    an aligned base, as a Program's arguments are when run."""
    _validate(specs, options)
    desc = _native.QmmDesc()
    views = [_dense_view(spec, 256) for spec in specs]
    desc.input, desc.packed, desc.scales, desc.biases = views
    desc.output = 256
    desc.output_bytes = specs[0].shape[0] * specs[1].shape[0] * 4
    desc.bits = options["bits"]
    desc.group_size = options["group_size"]
    desc.implementation = _native.IMPL_AUTO
    desc.numerical_policy = policy_code(policy)
    name = ctypes.create_string_buffer(128)
    status = _native.load().affon_rocm_quantized_matmul_select(ctypes.byref(desc), name, 128)
    if status != _native.OK:
        raise TypeError(f"no rocm quantized_matmul implementation: {_native.last_error()}")
    return name.value.decode()


def fused_select_for_specs(kind: str, specs: Sequence[TensorSpec], options: Mapping[str, Any], policy: str) -> str:
    """Compile-time plan of a fused step from formal specs: ``kind`` "bias"
    (specs: x, packed, scales, biases, bias) or "silu_gate" (x, gate packed,
    scales, biases, up packed, scales, biases)."""
    _validate(specs[:4], options)
    desc = _native.QmmDesc()
    desc.input, desc.packed, desc.scales, desc.biases = (_dense_view(spec, 256 * (i + 1))
                                                         for i, spec in enumerate(specs[:4]))
    desc.output = 256
    desc.output_bytes = specs[0].shape[0] * specs[1].shape[0] * 4
    desc.bits = options["bits"]
    desc.group_size = options["group_size"]
    desc.implementation = _native.IMPL_AUTO
    desc.numerical_policy = policy_code(policy)
    epi = _native.Epilogue()
    if kind == "bias":
        epi.kind = _native.EPILOGUE_BIAS
        epi.bias = 4096
        epi.bias_dtype = _native.BF16 if specs[4].dtype == "bf16" else _native.F32
        epi.bias_bytes = specs[4].shape[0] * (2 if specs[4].dtype == "bf16" else 4)
    else:
        epi.kind = _native.EPILOGUE_SILU_GATE
        epi.up_packed, epi.up_scales, epi.up_biases = (_dense_view(spec, 8192 * (i + 1))
                                                       for i, spec in enumerate(specs[4:7]))
    name = ctypes.create_string_buffer(256)
    status = _native.load().affon_rocm_quantized_matmul_fused_select(ctypes.byref(desc), ctypes.byref(epi), name, 256)
    if status != _native.OK:
        raise TypeError(f"no rocm quantized_matmul implementation: {_native.last_error()}")
    return name.value.decode()


def grouped_select_for_specs(members: Sequence[Sequence[TensorSpec]], options: Mapping[str, Any], policy: str) -> str:
    """Compile-time plan of a grouped step: each member is (x, packed,
    scales, biases[, bias]) specs sharing x."""
    count = len(members)
    descs = (_native.QmmDesc * count)()
    epis = (_native.Epilogue * count)()
    x_view = _dense_view(members[0][0], 256)
    for i, specs in enumerate(members):
        _validate(specs[:4], options)
        d = descs[i]
        d.input = x_view
        d.packed, d.scales, d.biases = (_dense_view(spec, (1 << 20) * (4 * i + j + 1)) for j, spec in enumerate(specs[1:4]))
        d.output = (1 << 30) + (1 << 24) * i
        d.output_bytes = specs[0].shape[0] * specs[1].shape[0] * 4
        d.bits = options["bits"]
        d.group_size = options["group_size"]
        d.implementation = _native.IMPL_AUTO
        d.numerical_policy = policy_code(policy)
        epis[i].kind = _native.EPILOGUE_NONE
        if len(specs) == 5:
            epis[i].kind = _native.EPILOGUE_BIAS
            epis[i].bias = (1 << 31) + (1 << 20) * i
            epis[i].bias_dtype = _native.BF16 if specs[4].dtype == "bf16" else _native.F32
            epis[i].bias_bytes = specs[4].shape[0] * (2 if specs[4].dtype == "bf16" else 4)
    name = ctypes.create_string_buffer(512)
    status = _native.load().affon_rocm_quantized_matmul_grouped_select(descs, epis, count, name, 512)
    if status != _native.OK:
        raise TypeError(f"no rocm quantized_matmul implementation: {_native.last_error()}")
    return name.value.decode()


# ---- formal element-wise ops (lowered into quantized_matmul epilogues) ----

def _formal_pair(name: str, a: Any, b: Any) -> None:
    if not isinstance(a, FormalTensor) or not isinstance(b, FormalTensor):
        if isinstance(a, FormalTensor) != isinstance(b, FormalTensor):
            raise TypeError(f"{name} cannot mix formal and evaluated tensors")
        raise TypeError(f"{name} of evaluated tensors has no rocm kernel: author it in a Program after "
                        "quantized_matmul, or call quantized_linear / quantized_silu_gate")
    if a.builder is not b.builder:
        raise TypeError(f"{name} operands must belong to the same Program")


def _broadcast(name: str, a: TensorSpec, b: TensorSpec) -> TensorSpec:
    """Same shape, or a rank-one operand matching the other's last axis."""
    if a.shape == b.shape:
        shape = a.shape
    elif len(b.shape) == 1 and len(a.shape) >= 1 and b.shape[0] == a.shape[-1]:
        shape = a.shape
    elif len(a.shape) == 1 and len(b.shape) >= 1 and a.shape[0] == b.shape[-1]:
        shape = b.shape
    else:
        raise TypeError(f"{name} operand shapes {a.shape} and {b.shape} do not broadcast")
    if a.dtype == "u32" or b.dtype == "u32":
        raise TypeError(f"{name} requires f32/bf16 tensors")
    return TensorSpec("f32" if "f32" in (a.dtype, b.dtype) else a.dtype, shape)


def add(a: Any, b: Any) -> FormalTensor:
    """Formal element-wise add (src/js/ops.ts:51)."""
    _formal_pair("add", a, b)
    return a.builder.emit("add", (a, b), _broadcast("add", a.spec, b.spec), {})


def mul(a: Any, b: Any) -> FormalTensor:
    """Formal element-wise multiply (src/js/ops.ts:53)."""
    _formal_pair("mul", a, b)
    return a.builder.emit("mul", (a, b), _broadcast("mul", a.spec, b.spec), {})


def silu(x: Any) -> FormalTensor:
    """Formal silu (src/js/ops.ts:91)."""
    if not isinstance(x, FormalTensor):
        raise TypeError("silu of an evaluated tensor has no rocm kernel: author it in a Program after "
                        "quantized_matmul, or call quantized_silu_gate")
    if x.dtype == "u32":
        raise TypeError("silu requires an f32/bf16 tensor")
    return x.builder.emit("silu", (x,), x.spec, {})


def quantize(weights: Tensor, *, bits: int, group_size: int, param_dtype: str = "bf16") -> tuple[Tensor, Tensor, Tensor]:
    """Affine group-wise quantize of a contiguous [N,K] f32/bf16 tensor into
    (packed u32 [N,K/P], scales [N,K/g], biases [N,K/g])."""
    if weights.dtype not in ("f32", "bf16") or len(weights.shape) != 2 or not weights.is_contiguous():
        raise TypeError("quantize requires a contiguous rank-two f32/bf16 tensor")
    if bits not in (2, 4, 8):
        raise TypeError("quantize bits must be 2, 4, or 8")
    if not isinstance(group_size, int) or group_size <= 0:
        raise TypeError("quantize group_size must be a positive integer")
    if param_dtype not in ("f32", "bf16"):
        raise TypeError("quantize parameters must be f32 or bf16")
    rows, cols = weights.shape
    per_word = 32 // bits
    if cols % per_word or cols % group_size:
        raise TypeError("quantize columns must divide into complete words and groups")
    session = weights.session
    packed = session.empty("u32", (rows, cols // per_word))
    scales = session.empty(param_dtype, (rows, cols // group_size))
    biases = session.empty(param_dtype, (rows, cols // group_size))
    code = {"f32": _native.F32, "bf16": _native.BF16}
    _native.check(_native.load().affon_rocm_quantize(
        session._handle, weights.data_ptr, code[weights.dtype], rows, cols, bits, group_size, packed.data_ptr,
        scales.data_ptr, biases.data_ptr, code[param_dtype]), "quantize")
    return packed, scales, biases


def dequantize(packed: Tensor, scales: Tensor, biases: Tensor, *, bits: int, group_size: int,
               dtype: str = "f32") -> Tensor:
    """Expands packed weights to a [N,K] f32/bf16 tensor: w = s*q + b."""
    for t in (packed, scales, biases):
        if len(t.shape) != 2 or not t.is_contiguous():
            raise TypeError("dequantize requires contiguous rank-two tensors")
    if packed.dtype != "u32" or scales.dtype not in ("f32", "bf16") or biases.dtype != scales.dtype:
        raise TypeError("dequantize requires u32 packed weights and matching f32/bf16 scales and biases")
    if bits not in (2, 4, 8):
        raise TypeError("dequantize bits must be 2, 4, or 8")
    if not isinstance(group_size, int) or group_size <= 0:
        raise TypeError("dequantize group_size must be a positive integer")
    if dtype not in ("f32", "bf16"):
        raise TypeError("dequantize output must be f32 or bf16")
    rows = packed.shape[0]
    cols = packed.shape[1] * (32 // bits)
    if cols % group_size or scales.shape != (rows, cols // group_size) or biases.shape != scales.shape:
        raise TypeError("dequantize parameter dimensions do not match the packed weights")
    session = packed.session
    out = session.empty(dtype, (rows, cols))
    code = {"f32": _native.F32, "bf16": _native.BF16}
    _native.check(_native.load().affon_rocm_dequantize(
        session._handle, packed.data_ptr, scales.data_ptr, biases.data_ptr, code[scales.dtype], rows, cols, bits,
        group_size, out.data_ptr, code[dtype]), "dequantize")
    return out


def transpose(t: Tensor, permutation: Sequence[int]) -> Tensor:
    if sorted(permutation) != list(range(len(t.shape))):
        raise TypeError("transpose permutation must list every axis once")
    return Tensor(t.session, t._buffer, t.dtype, [t.shape[p] for p in permutation],
                  [t.strides[p] for p in permutation], t.offset)


def slice(t: Tensor, ranges: Sequence[Mapping[str, int]]) -> Tensor:  # noqa: A001 - reference op name
    if len(ranges) != len(t.shape):
        raise TypeError("slice needs one range per axis")
    shape, strides, offset = [], [], t.offset
    for dim, stride, r in zip(t.shape, t.strides, ranges):
        start, stop, step = int(r.get("start", 0)), int(r.get("stop", dim)), int(r.get("step", 1))
        if not (0 <= start <= stop <= dim) or step <= 0:
            raise TypeError("slice range out of bounds")
        shape.append((stop - start + step - 1) // step)
        strides.append(stride * step)
        offset += start * stride
    return Tensor(t.session, t._buffer, t.dtype, shape, strides, offset)


# ---- the other ops of a decode step (rms_norm, softmax, index_select) ----
# src/js/ops.ts:97,99,119; catalogued for a decode step in
# test/parity/catalogs/cuda-apertus-decode-ops.json:1-26. Rank-two f32/bf16
# tensors; rms_norm and softmax along the last axis.

def _last_axis(name: str, x: Any, axis: Any) -> None:
    if not isinstance(axis, int) or isinstance(axis, bool):
        raise TypeError(f"{name} axis must be an integer")
    rank = len(x.shape)
    if rank != 2:
        raise TypeError(f"{name} on rocm requires a rank-two tensor")
    if axis not in (-1, rank - 1):
        raise TypeError(f"{name} on rocm runs along the last axis")
    if x.dtype not in ("f32", "bf16"):
        raise TypeError(f"{name} requires an f32 or bf16 tensor")


def _contiguous_input(name: str, x: Tensor) -> None:
    if not x.is_contiguous():
        raise TypeError(f"{name} on rocm requires a contiguous tensor")


def rms_norm(x: Any, axis: int, epsilon: float = 1e-5) -> Any:
    """x / sqrt(mean(x^2 along axis) + epsilon), computed in f32."""
    _last_axis("rms_norm", x, axis)
    epsilon = float(epsilon)
    if not np.isfinite(epsilon) or epsilon <= 0:  # program.ts:578-579
        raise TypeError("invalid rms_norm options: epsilon must be finite and positive")
    if isinstance(x, FormalTensor):
        return x.builder.emit("rms_norm", (x,), x.spec, {"axis": axis, "epsilon": epsilon})
    if not isinstance(x, Tensor):
        raise TypeError("rms_norm requires a tensor")
    return _run_rms_norm(x, epsilon)


def _run_rms_norm(x: Tensor, epsilon: float) -> Tensor:
    _contiguous_input("rms_norm", x)
    out = x.session.empty(x.dtype, x.shape)
    code = {"f32": _native.F32, "bf16": _native.BF16}[x.dtype]
    _native.check(_native.load().affon_rocm_rms_norm(x.session._handle, x.data_ptr, code, x.shape[0], x.shape[1],
                                                     epsilon, out.data_ptr), "Program execution failed")
    return out


def softmax(x: Any, axis: int) -> Any:
    """exp(x - max) / sum(exp(x - max)) along axis, computed in f32."""
    _last_axis("softmax", x, axis)
    if isinstance(x, FormalTensor):
        return x.builder.emit("softmax", (x,), x.spec, {"axis": axis})
    if not isinstance(x, Tensor):
        raise TypeError("softmax requires a tensor")
    return _run_softmax(x)


def _run_softmax(x: Tensor) -> Tensor:
    _contiguous_input("softmax", x)
    out = x.session.empty(x.dtype, x.shape)
    code = {"f32": _native.F32, "bf16": _native.BF16}[x.dtype]
    _native.check(_native.load().affon_rocm_softmax(x.session._handle, x.data_ptr, code, x.shape[0], x.shape[1],
                                                    out.data_ptr), "Program execution failed")
    return out


def index_select(x: Any, axis: int, indices: Any) -> Any:
    """Rows (axis 0) or columns (axis 1) of x at i64 indices; indices outside
    the axis select zeros."""
    if isinstance(x, FormalTensor) != isinstance(indices, FormalTensor):
        raise TypeError("index_select cannot mix formal and evaluated tensors")
    if not isinstance(axis, int) or isinstance(axis, bool) or len(x.shape) != 2 or axis not in (0, 1, -1, -2):
        raise TypeError("index_select on rocm takes a rank-two tensor and axis 0 or 1")
    axis = axis % 2
    if x.dtype not in ("f32", "bf16"):
        raise TypeError("index_select requires an f32 or bf16 tensor")
    if indices.dtype != "i64" or len(indices.shape) != 1 or indices.shape[0] <= 0:
        raise TypeError("index_select indices must be a non-empty rank-one i64 tensor")
    count = indices.shape[0]
    shape = (count, x.shape[1]) if axis == 0 else (x.shape[0], count)
    if isinstance(x, FormalTensor):
        if x.builder is not indices.builder:
            raise TypeError("index_select operands must belong to the same Program")
        return x.builder.emit("index_select", (x, indices), TensorSpec(x.dtype, shape), {"axis": axis})
    if not isinstance(x, Tensor) or not isinstance(indices, Tensor):
        raise TypeError("index_select requires tensors")
    if indices.session is not x.session:
        raise TypeError("index_select operands must belong to the same Session")
    return _run_index_select(x, axis, indices)


def _run_index_select(x: Tensor, axis: int, indices: Tensor) -> Tensor:
    _contiguous_input("index_select", x)
    _contiguous_input("index_select", indices)
    count = indices.shape[0]
    out = x.session.empty(x.dtype, (count, x.shape[1]) if axis == 0 else (x.shape[0], count))
    code = {"f32": _native.F32, "bf16": _native.BF16}[x.dtype]
    _native.check(_native.load().affon_rocm_index_select(x.session._handle, x.data_ptr, code, x.shape[0], x.shape[1],
                                                         axis, indices.data_ptr, count, out.data_ptr),
                  "Program execution failed")
    return out
