"""C-ABI library checks that need no GPU: it loads, exports every symbol the
header declares, and validates / selects exactly as the reference does
(src/js/compute/program.ts:481-494, src/support/compute_core_cyna.zig:1000-1045).
"""
import ctypes
import json
import pathlib
import re

import numpy as np
import pytest

from affon_amd import _native
from affon_amd.ops import select_for_specs
from affon_amd.core import TensorSpec

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "affon_rocm.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_]+\s*\*?\s*([a-z_0-9]+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = declared_functions()
    assert "affon_rocm_quantized_matmul" in names and "compute_core_run_quantized_matmul_f32" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native.SIGNATURES), "ctypes signatures and header disagree"


def test_capabilities_registry():
    caps = json.loads(_native.load().affon_rocm_quantized_matmul_capabilities().decode())
    ids = [c["id"] for c in caps]
    assert ids == ["rocm_quantized_matmul.mfma", "rocm_quantized_matmul.gemv_mfma", "rocm_quantized_matmul.gemv",
                   "rocm_quantized_matmul.generic"]
    classes = {c["id"]: c["numerical_class"] for c in caps}
    assert classes["rocm_quantized_matmul.generic"] == "exact"
    assert all("host_" not in i for i in ids)


def _view(ptr, shape, strides, dtype, buffer_bytes=None, offset=0):
    size = {_native.F32: 4, _native.BF16: 2, _native.U32: 4}[dtype]
    if buffer_bytes is None:
        buffer_bytes = offset + ((shape[0] - 1) * strides[0] + (shape[1] - 1) * strides[1] + 1) * size
    return _native.View(ptr, buffer_bytes, offset, (ctypes.c_int64 * 2)(*shape), (ctypes.c_int64 * 2)(*strides),
                        dtype)


def make_desc(M=1, K=64, N=8, bits=4, group=64, x_dtype=_native.BF16, p_dtype=_native.BF16, impl=0, policy=0):
    per_word = 32 // bits
    d = _native.QmmDesc()
    d.input = _view(4096, (M, K), (K, 1), x_dtype)
    d.packed = _view(4096, (N, K // per_word), (K // per_word, 1), _native.U32)
    d.scales = _view(4096, (N, K // group), (K // group, 1), p_dtype)
    d.biases = _view(4096, (N, K // group), (K // group, 1), p_dtype)
    d.output = 4096
    d.output_bytes = M * N * 4
    d.bits, d.group_size, d.implementation, d.numerical_policy = bits, group, impl, policy
    return d


def select(d):
    name = ctypes.create_string_buffer(96)
    status = _native.load().affon_rocm_quantized_matmul_select(ctypes.byref(d), name, 96)
    return status, (name.value.decode() if status == 0 else _native.last_error())


def test_selection_rules():
    assert select(make_desc(M=1)) == (0, "rocm_quantized_matmul.gemv")
    assert select(make_desc(M=1, x_dtype=_native.F32, p_dtype=_native.F32)) == (0, "rocm_quantized_matmul.gemv")
    # exact_only admits only the ordered-loop candidate.
    assert select(make_desc(M=1, policy=_native.EXACT_ONLY)) == (0, "rocm_quantized_matmul.generic")
    # groups crossing words go to the generic candidate.
    assert select(make_desc(M=2, K=24, N=3, bits=4, group=3)) == (0, "rocm_quantized_matmul.generic")
    # forcing a candidate that cannot run the shape is "unsupported", not a silent fallback.
    status, message = select(make_desc(M=2, K=24, N=3, bits=4, group=3, impl=_native.IMPL_GEMV))
    assert status == _native.UNSUPPORTED and "gemv" in message
    status, message = select(make_desc(impl=_native.IMPL_GEMV, policy=_native.EXACT_ONLY))
    assert status == _native.UNSUPPORTED and "numerical policy" in message


@pytest.mark.parametrize("mutate,message", [
    (lambda d: setattr(d, "bits", 3), "bits must be 2, 4, or 8"),
    (lambda d: setattr(d, "group_size", 0), "group_size must be a positive integer"),
    (lambda d: setattr(d.input, "dtype", _native.U32), "requires f32/bf16 input"),
    (lambda d: setattr(d.biases, "dtype", _native.F32), "matching f32/bf16 scales and biases"),
    (lambda d: setattr(d, "group_size", 48), "packed or group dimensions"),
    (lambda d: d.packed.shape.__setitem__(1, 7), "packed or group dimensions"),
    (lambda d: d.scales.shape.__setitem__(0, 7), "packed or group dimensions"),
    (lambda d: setattr(d.input, "buffer_bytes", 16), "exceeds its buffer"),
    (lambda d: setattr(d.packed, "byte_offset", 2), "element aligned"),
    (lambda d: d.input.stride.__setitem__(1, -1), "negative stride"),
    (lambda d: setattr(d, "output_bytes", 4), "output buffer"),
    (lambda d: d.input.shape.__setitem__(0, 2**62), "extent overflows"),
])
def test_validation_rejects_with_reference_messages(mutate, message):
    d = make_desc(M=2, K=64, N=8)
    mutate(d)
    status, text = select(d)
    assert status == _native.INVALID_SHAPE
    assert message in text


@pytest.mark.parametrize("case", ["group_does_not_divide_input_features", "bits_do_not_match_packed_width",
                                  "three_bits_rejected"])
def test_reference_invalid_cases(kats, case):
    c = next(x for x in kats["invalid"] if x["name"] == case)
    d = make_desc(M=1, K=4, N=1, bits=8, group=4)
    d.bits, d.group_size = c["bits"], c["group_size"]
    assert select(d)[0] == _native.INVALID_SHAPE


def _drop_in(rows, depth, columns, bits, group, counts=None, buffers=None):
    lib = _native.load()
    a = np.arange(1, 17, dtype=np.float32) if buffers is None else buffers[0]
    w = np.array([0x01010101] * 2 + [0x02020202] * 2 + [0x03030303] * 2, dtype=np.uint32)
    s = np.ones(6, np.float32)
    b = np.zeros(6, np.float32)
    out = np.full(6, -1.0, np.float32)
    counts = counts or (a.size, w.size, s.size, b.size, out.size)
    status = lib.compute_core_run_quantized_matmul_f32(
        a.ctypes.data, counts[0], w.ctypes.data, counts[1], s.ctypes.data, counts[2], b.ctypes.data, counts[3],
        out.ctypes.data, counts[4], rows, depth, columns, bits, group)
    return status, out


def test_drop_in_invalid_shapes_leave_output_untouched():
    """compute_core_cyna_smoke.zig:979-983."""
    for args in [(2, 8, 3, 3, 4), (2, 8, 3, 8, 0), (2**64 - 1, 8, 3, 8, 4), (2, 8, 3, 4, 4)]:
        status, out = _drop_in(*args)
        assert status == 1, args
        assert out.tolist() == [-1.0] * 6
    status, out = _drop_in(2, 8, 3, 8, 4, counts=(15, 6, 6, 6, 6))
    assert status == 1 and out.tolist() == [-1.0] * 6


def test_host_validation_messages_match_reference():
    from affon_amd import program, quantized_matmul
    with pytest.raises(TypeError, match="bits must be 2, 4, or 8"):
        program("q", lambda p: quantized_matmul(p.argument("x", TensorSpec.f32([1, 4])),
                                                p.argument("w", TensorSpec.u32([1, 1])),
                                                p.argument("s", TensorSpec.f32([1, 1])),
                                                p.argument("b", TensorSpec.f32([1, 1])), {"bits": 3, "group_size": 4}))
    with pytest.raises(TypeError, match="packed or group dimensions"):
        program("q", lambda p: quantized_matmul(p.argument("x", TensorSpec.f32([1, 4])),
                                                p.argument("w", TensorSpec.u32([1, 1])),
                                                p.argument("s", TensorSpec.f32([1, 1])),
                                                p.argument("b", TensorSpec.f32([1, 1])), {"bits": 8, "group_size": 3}))
    with pytest.raises(TypeError, match="matching f32/bf16 scales and biases"):
        program("q", lambda p: quantized_matmul(p.argument("x", TensorSpec.f32([1, 4])),
                                                p.argument("w", TensorSpec.u32([1, 1])),
                                                p.argument("s", TensorSpec.f32([1, 1])),
                                                p.argument("b", TensorSpec.bf16([1, 1])), {"bits": 8, "group_size": 4}))
    with pytest.raises(TypeError, match="group_size must be a positive integer"):
        program("q", lambda p: quantized_matmul(p.argument("x", TensorSpec.f32([1, 4])),
                                                p.argument("w", TensorSpec.u32([1, 1])),
                                                p.argument("s", TensorSpec.f32([1, 1])),
                                                p.argument("b", TensorSpec.f32([1, 1])), bits=8, group_size=2.5))


def test_formal_program_authors_one_native_node_and_selects_rocm():
    from affon_amd import program, quantized_matmul
    source = program("quantized_linear", lambda p: quantized_matmul(
        p.argument("x", TensorSpec.f32([1, 4])), p.argument("w", TensorSpec.u32([1, 1])),
        p.argument("s", TensorSpec.bf16([1, 1])), p.argument("b", TensorSpec.bf16([1, 1])),
        {"bits": 8, "group_size": 4}))
    ops = [n["op"] for n in source.inspect()["nodes"] if n["kind"] == "operation"]
    assert ops == ["quantized_matmul"]
    specs = [TensorSpec.f32([1, 4]), TensorSpec.u32([1, 1]), TensorSpec.bf16([1, 1]), TensorSpec.bf16([1, 1])]
    impl = select_for_specs(specs, {"bits": 8, "group_size": 4}, "backend_equivalent")
    assert impl.startswith("rocm_quantized_matmul") and "host_" not in impl
    assert select_for_specs(specs, {"bits": 8, "group_size": 4}, "exact_only") == "rocm_quantized_matmul.generic"


def test_rms_norm_rejects_non_positive_epsilon():
    """program.ts:578-579: rms_norm needs a finite epsilon > 0 (an all-zero row
    would otherwise give 0/0). Rejected before any device work."""
    from affon_amd import program, rms_norm
    lib = _native.load()
    for eps in (0.0, -1e-5, float("inf"), float("nan")):
        assert lib.affon_rocm_rms_norm(None, 4096, _native.F32, 2, 4, eps, 4096) == _native.INVALID_SHAPE, eps
        assert "invalid rms_norm options" in _native.last_error()
        with pytest.raises(TypeError, match="invalid rms_norm options"):
            program("norm", lambda p, eps=eps: rms_norm(p.argument("x", TensorSpec.f32([2, 4])), 1, epsilon=eps))
    program("norm", lambda p: rms_norm(p.argument("x", TensorSpec.f32([2, 4])), 1, epsilon=1e-6))


def kernel_supports(d, kernel):
    ok = ctypes.c_int(-1)
    status = _native.load().affon_rocm_kernel_supports(ctypes.byref(d), kernel.encode(), ctypes.byref(ok))
    assert status == 0, _native.last_error()
    return ok.value


def test_kernel_supports_names_and_validation():
    d = make_desc(M=512, K=4096, N=256)
    assert kernel_supports(d, "gemm_re") == 1
    assert kernel_supports(d, "generic") == 1
    ok = ctypes.c_int(-1)
    assert _native.load().affon_rocm_kernel_supports(ctypes.byref(d), b"nope", ctypes.byref(ok)) == _native.INVALID_SHAPE
    bad = make_desc(M=2, K=64, N=8)
    bad.bits = 3
    assert _native.load().affon_rocm_kernel_supports(ctypes.byref(bad), b"gemv", ctypes.byref(ok)) == _native.INVALID_SHAPE


def test_reassociated_gemm_declines_offsets_past_31_bits():
    """The reassociated prefill GEMM feeds its transfers 32-bit byte offsets
    from a scalar base: the last activation row and the last packed-word row
    must start below 2^31 bytes. Strided views (no memory is touched on the
    CPU) put them just below and just at the bound."""
    K, N, M = 4096, 256, 512
    limit = 2**31
    for xs0, accepted in ((limit // (2 * M) - 8, 1), (limit // (2 * M), 0)):
        d = make_desc(M=M, K=K, N=N)
        d.input = _view(4096, (M, K), (xs0, 1), _native.BF16)
        assert kernel_supports(d, "gemm_re") == accepted, xs0
    words = K // 8
    for ws0, accepted in ((limit // (4 * N) - 4, 1), (limit // (4 * N), 0)):
        d = make_desc(M=M, K=K, N=N)
        d.packed = _view(4096, (N, words), (ws0, 1), _native.U32)
        assert kernel_supports(d, "gemm_re") == accepted, ws0


def test_group32_gemm_guard():
    """The group-32 prefill GEMM (both classes) takes 4-bit codes with bf16
    activations and parameters, groups of 32, K a multiple of 128, and feeds
    its transfers 32-bit byte offsets from a scalar base: the last activation
    row, packed-word row and parameter rows must start below 2^31 bytes.
    Strided views (no memory is touched on the CPU) put them just below and
    just at the bound."""
    K, N, M = 4096, 256, 512
    assert kernel_supports(make_desc(M=M, K=K, N=N, group=32), "gemm_re32") == 1
    assert kernel_supports(make_desc(M=M, K=K, N=N, group=64), "gemm_re32") == 0
    assert kernel_supports(make_desc(M=M, K=K + 64, N=N, group=32), "gemm_re32") == 0
    assert kernel_supports(make_desc(M=M, K=K, N=N, group=32, p_dtype=_native.F32), "gemm_re32") == 0
    assert kernel_supports(make_desc(M=M, K=K, N=N, bits=8, group=32), "gemm_re32") == 0
    limit = 2**31
    for xs0, accepted in ((limit // (2 * M) - 8, 1), (limit // (2 * M), 0)):
        d = make_desc(M=M, K=K, N=N, group=32)
        d.input = _view(4096, (M, K), (xs0, 1), _native.BF16)
        assert kernel_supports(d, "gemm_re32") == accepted, xs0
    words = K // 8
    for ws0, accepted in ((limit // (4 * N) - 4, 1), (limit // (4 * N), 0)):
        d = make_desc(M=M, K=K, N=N, group=32)
        d.packed = _view(4096, (N, words), (ws0, 1), _native.U32)
        assert kernel_supports(d, "gemm_re32") == accepted, ws0
    groups = K // 32
    for ss0, accepted in ((limit // (2 * N) - 2, 1), (limit // (2 * N), 0)):
        for field in ("scales", "biases"):
            d = make_desc(M=M, K=K, N=N, group=32)
            setattr(d, field, _view(4096, (N, groups), (ss0, 1), _native.BF16))
            assert kernel_supports(d, "gemm_re32") == accepted, (field, ss0)


def test_group32_prefill_selection():
    """Groups of 32 past 128 rows: the approximate candidate under the
    approximate policy (whose 4-bit prefill runs the group-32 GEMM's
    rounded-weight form), the decode-batch candidate under the default
    policy (which runs its exact-code form)."""
    d = make_desc(M=512, K=4096, N=1024, group=32, policy=_native.APPROXIMATE)
    assert select(d) == (0, "rocm_quantized_matmul.mfma")
    d = make_desc(M=512, K=4096, N=1024, group=32, policy=_native.BACKEND_EQUIVALENT)
    assert select(d) == (0, "rocm_quantized_matmul.gemv_mfma")
