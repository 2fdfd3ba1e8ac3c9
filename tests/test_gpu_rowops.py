"""GPU parity of the other decode-step ops on the rocm device (rms_norm,
softmax, index_select) against the CPU oracle and the reference's
decode-op catalog (test/parity/catalogs/cuda-apertus-decode-ops.json).

Tolerances: catalog cells use the catalog oracle's peak-scaled bound
(2e-2 * max(1, peak) for bf16, 2e-6 * max(1, peak) for f32,
test/parity/reference/probe-capabilities.py:454-457); against the oracle,
f32 results are within rtol 1e-5 / atol 1e-7 (rms_norm: an f32 sum of up to
14336 squares) and rtol 1e-5 / atol 1e-9 (softmax: f32 exp against f64),
bf16 results within one bf16 ulp
(the f32 result before rounding differs from the f64 one by a few f32
ulps); index_select is bit-exact.
"""
import json
import pathlib

import numpy as np
import pytest

import affon_amd as A
from affon_amd import _native
from oracle import oracle as O
from tests.helpers import peak_tolerance
from tests.test_gpu_parity import upload

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def probe_values(shape, dtype):
    """The probe's input formula for the catalog cells: rounded(1 + row/8 +
    col/8) (probe-capabilities.py:117-125, seed 1, plain layout)."""
    rows, cols = shape
    v = 1 + np.arange(rows)[:, None] / 8 + np.arange(cols)[None, :] / 8
    f32 = v.astype(np.float32)
    return O.bf16_from_f32(f32) if dtype == "bf16" else f32


def as_values(arr):
    return O.f32_from_bf16(arr).astype(np.float64) if arr.dtype == np.uint16 else arr.astype(np.float64)


def within_bf16_ulp(actual_bits, expected_bits):
    a = O.f32_from_bf16(actual_bits).astype(np.float64)
    e = O.f32_from_bf16(expected_bits).astype(np.float64)
    ulp = np.abs(e) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(a - e) <= ulp), float(np.max(np.abs(a - e) / ulp))


def test_decode_op_catalog(session):
    for case in json.loads((GOLDEN / "cuda-apertus-decode-ops.json").read_text())["cases"]:
        dtype, shape = case["dtype"], tuple(case["shape"])
        x = probe_values(shape, dtype)
        xt = upload(session, x, dtype)
        if case["op"] == "index_select":
            axis = case.get("index_axis", 0)
            index = np.array([(c * 3 + 1) % shape[axis] for c in range(case["index_shape"][0])], np.int64)
            out = A.index_select(xt, axis, session.tensor(index, "i64"))
            expected = O.index_select(x, axis, index)
            np.testing.assert_array_equal(out.storage(), expected, err_msg=case["id"])
            continue
        out = A.rms_norm(xt, 1) if case["op"] == "rms_norm" else A.softmax(xt, 1)
        expected = O.rms_norm(x) if case["op"] == "rms_norm" else O.softmax(x)
        tol = peak_tolerance(as_values(expected), dtype)
        assert np.abs(as_values(out.storage()) - as_values(expected)).max() <= tol, case["id"]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(32, 128), (5, 4096), (3, 1), (7, 14336), (1, 65)])
def test_rms_norm_and_softmax_against_oracle(session, dtype, shape, rng):
    values = (rng.standard_normal(shape) * 3).astype(np.float32)
    x = O.bf16_from_f32(values) if dtype == "bf16" else values
    xt = upload(session, x, dtype)
    for name, got, expected in (("rms_norm", A.rms_norm(xt, -1), O.rms_norm(x)),
                                ("rms_norm eps", A.rms_norm(xt, 1, epsilon=0.5), O.rms_norm(x, 0.5)),
                                ("softmax", A.softmax(xt, 1), O.softmax(x))):
        out = got.storage()
        if dtype == "bf16":
            within_bf16_ulp(out, expected)
        elif name.startswith("rms_norm"):
            np.testing.assert_allclose(out, expected, rtol=1e-5, atol=1e-7, err_msg=name)
        else:
            np.testing.assert_allclose(out, expected, rtol=1e-5, atol=1e-9, err_msg=name)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_index_select_against_oracle(session, dtype, rng):
    values = rng.standard_normal((320, 128)).astype(np.float32)
    x = O.bf16_from_f32(values) if dtype == "bf16" else values
    xt = upload(session, x, dtype)
    for axis, index in ((0, np.array([1, 319, 0, 7, 320, -3, 5], np.int64)), (1, np.array([127, 0, 128, 64], np.int64)),
                        (0, np.arange(320, dtype=np.int64)[::-1].copy())):
        out = A.index_select(xt, axis, session.tensor(index, "i64"))
        np.testing.assert_array_equal(out.storage(), O.index_select(x, axis, index))


def test_decode_ops_in_a_program(session, rng):
    """rms_norm -> quantized projection -> softmax, and an embedding-style
    index_select, as one Program; every node lowers to a rocm kernel."""
    x = O.bf16_from_f32(rng.standard_normal((2, 256)).astype(np.float32))
    _, wb = O.randn(9, 64 * 256, 0.0, 0.02)
    packed, s, b = O.quantize(wb.reshape(64, 256), 4, 64, "bf16")

    def body(p):
        h = A.rms_norm(p.argument("x", A.TensorSpec.bf16([2, 256])), 1)
        y = A.quantized_matmul(h, p.argument("w", A.TensorSpec.u32(packed.shape)),
                               p.argument("s", A.TensorSpec.bf16(s.shape)), p.argument("b", A.TensorSpec.bf16(b.shape)),
                               bits=4, group_size=64)
        rows = A.index_select(p.argument("table", A.TensorSpec.f32([64, 8])), 0, p.argument("ids", A.TensorSpec.i64([3])))
        return [A.softmax(y, 1), rows]
    executable = session.compile(A.program("decode_ops", body))
    ops = [n["op"] for n in executable.explain()["executable"]["physical_nodes"]]
    assert ops == ["rms_norm", "quantized_matmul", "index_select", "softmax"], ops
    table = rng.standard_normal((64, 8)).astype(np.float32)
    ids = np.array([3, 63, 0], np.int64)
    probs, rows = executable.run({"x": upload(session, x, "bf16"), "w": upload(session, packed, "u32"),
                                  "s": upload(session, s, "bf16"), "b": upload(session, b, "bf16"),
                                  "table": upload(session, table, "f32"), "ids": session.tensor(ids, "i64")})
    h = O.rms_norm(x)
    logits = O.quantized_matmul(h, packed, s, b, 4, 64)
    np.testing.assert_allclose(probs.numpy(), O.softmax(logits), rtol=2e-2, atol=1e-4)
    np.testing.assert_array_equal(rows.numpy(), table[ids])


def test_decode_op_validation(session):
    x = session.tensor(np.ones((2, 4), np.float32), "f32")
    with pytest.raises(TypeError, match="last axis"):
        A.softmax(x, 0)
    with pytest.raises(TypeError, match="epsilon"):
        A.rms_norm(x, 1, epsilon=-1.0)
    with pytest.raises(TypeError, match="i64"):
        A.index_select(x, 0, session.tensor([0, 1], "f32"))
    lib = _native.load()
    assert lib.affon_rocm_softmax(session._handle, x.data_ptr, 2, 2, 4, x.data_ptr) == _native.INVALID_SHAPE
    assert lib.affon_rocm_index_select(session._handle, x.data_ptr, 0, 2, 4, 2, x.data_ptr, 1,
                                       x.data_ptr) == _native.INVALID_SHAPE
    assert "axis" in _native.last_error()
