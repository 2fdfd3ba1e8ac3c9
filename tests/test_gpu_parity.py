"""GPU parity of every rocm quantized_matmul implementation, quantize and
dequantize against the CPU oracle and the reference's exact known answers.

Tolerances (stated per test): outputs that the reference pins exactly (its
known-answer tests use integer or dyadic values) must match exactly; seeded
random products must be within rtol 2e-3 / atol 1e-4 for f32 activations and
rtol 1e-2 / atol 1e-2*rms(expected) for bf16 activations (f32 accumulation in
both); packed words, scales, biases and dequantized weights must be bit-exact.
"""
import json
import pathlib

import numpy as np
import pytest

import affon_amd as A
from affon_amd import _native
from oracle import oracle as O
from tests.helpers import (assert_bf16_product_close, assert_close_rtol_atol, fixture_operands, oracle_columns,
                           near_tie_group, pack_codes, peak_tolerance, reference_f64, storage, tie_group,
                           unpack_bytes_le)
from tests.test_oracle import crossing_word_case, tile_edge_case

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
IMPLS = ["auto", "generic", "gemv", "gemv_mfma", "mfma"]


def upload(session, arr: np.ndarray, dtype: str) -> A.Tensor:
    """Uploads host storage (f32, uint16 bf16 bits, or uint32 words)."""
    spec = {"f32": A.TensorSpec.f32, "bf16": A.TensorSpec.bf16, "u32": A.TensorSpec.u32}[dtype](arr.shape)
    return session.from_bytes(np.ascontiguousarray(arr), spec)


def dtype_of(arr: np.ndarray) -> str:
    return "bf16" if arr.dtype == np.uint16 else ("u32" if arr.dtype == np.uint32 else "f32")


def run_all(session, x, w, s, b, bits, group, impls=IMPLS):
    """Runs every implementation that accepts the problem; returns {impl: output}."""
    results = {}
    for impl in impls:
        try:
            selected = A.selected_implementation(x, w, s, b, bits=bits, group_size=group, implementation=impl)
        except _native.NativeError as error:
            assert error.status == _native.UNSUPPORTED, str(error)
            continue
        out = session.empty("f32", (x.shape[0], w.shape[0]))
        A.quantized_matmul_into(out, x, w, s, b, bits=bits, group_size=group, implementation=impl)
        results[impl if impl != "auto" else "auto:" + selected] = out.numpy()
    assert any(k.startswith("auto") for k in results)
    return results


def test_known_answers_every_implementation(session, kats):
    for case in kats["cases"]:
        x = session.tensor(case["input"]["values"], dtype=case["input"]["dtype"])
        w = session.tensor(case["packed"], dtype="u32")
        s = session.tensor(case["scales"]["values"], dtype=case["scales"]["dtype"])
        b = session.tensor(case["biases"]["values"], dtype=case["biases"]["dtype"])
        y = A.quantized_matmul(x, w, s, b, {"bits": case["bits"], "group_size": case["group_size"]})
        assert y.shape == tuple(np.array(case["expected"]).shape) and y.dtype == "f32"
        assert y.to_array() == case["expected"], case["name"]
        for impl, out in run_all(session, x, w, s, b, case["bits"], case["group_size"]).items():
            assert out.tolist() == case["expected"], (case["name"], impl)


def test_views_with_byte_offsets(session, kats):
    case = kats["views"][0]
    base_x = session.tensor(case["base_input"]["values"])
    x = A.transpose(base_x, [1, 0])
    base_w = session.tensor(case["base_packed"], dtype="u32")
    w = A.slice(base_w, [{"start": 1, "stop": 2}, {"start": 1, "stop": 2}])
    base_s = session.tensor(case["base_scales"]["values"], dtype="bf16")
    base_b = session.tensor(case["base_biases"]["values"], dtype="bf16")
    s = A.slice(base_s, [{"start": 0, "stop": 1}, {"start": 1, "stop": 2}])
    b = A.slice(base_b, [{"start": 0, "stop": 1}, {"start": 1, "stop": 2}])
    y = A.quantized_matmul(x, w, s, b, bits=8, group_size=4)
    assert y.to_array() == case["expected"]


def test_groups_crossing_words_and_packed_unchanged(session):
    x, q, scales, biases, g, expected = crossing_word_case()
    packed = pack_codes(q, 4)
    for dtype in ("f32", "bf16"):
        xt, st, bt = (upload(session, storage(v, dtype), dtype) for v in (x, scales, biases))
        wt = upload(session, packed, "u32")
        for impl, out in run_all(session, xt, wt, st, bt, 4, g).items():
            assert out.tolist() == expected, impl
        np.testing.assert_array_equal(wt.numpy(), packed)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_tile_edges_exact(session, bits):
    """quantized-matmul.test.ts:123-148, including the transposed / sliced
    layouts the reference uses at M=17 and M=64."""
    for m in (1, 3, 4, 7, 16, 17, 33, 64, 128):
        x, q, scales, biases, g, expected = tile_edge_case(bits, m)
        packed = pack_codes(q, bits)
        if m in (17, 64):
            base_x = upload(session, storage(x.T, "bf16"), "bf16")
            xt = A.transpose(base_x, [1, 0])
            padded = np.concatenate([np.zeros((packed.shape[0], 1), np.uint32), packed], axis=1)
            wt = A.slice(upload(session, padded, "u32"), [{"start": 0, "stop": packed.shape[0]},
                                                          {"start": 1, "stop": packed.shape[1] + 1}])
        else:
            xt = upload(session, storage(x, "bf16"), "bf16")
            wt = upload(session, packed, "u32")
        st = upload(session, storage(scales, "bf16"), "bf16")
        bt = upload(session, storage(biases, "bf16"), "bf16")
        for impl, out in run_all(session, xt, wt, st, bt, bits, g).items():
            np.testing.assert_array_equal(out, expected.astype(np.float32), err_msg=f"{impl} m={m}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_group_specializations_closed_form(session, dtype):
    m, n, k = 8, 3, 128
    x = upload(session, storage(np.ones((m, k)), "bf16"), "bf16")
    w = upload(session, np.full((n, k // 4), 0x80808080, np.uint32), "u32")
    for group in (32, 64, 128):
        groups = k // group
        s = upload(session, storage([[(g + 1) / 128 for g in range(groups)]] * n, dtype), dtype)
        b = upload(session, storage(np.full((n, groups), -1.0), dtype), dtype)
        for impl, out in run_all(session, x, w, s, b, 8, group).items():
            assert (out == group * groups * (groups - 1) / 2).all(), (impl, group)


@pytest.mark.parametrize("group", [48, 64])
def test_groups_across_k_tiles(session, group):
    m, n = 64, 64
    k = 96 if group == 48 else 256
    r, c = np.arange(m)[:, None], np.arange(k)[None, :]
    o, blk = np.arange(n)[:, None], np.arange(k // group)[None, :]
    x = ((r + c) % 11 - 5) / 8
    q = (o + c) % 256
    scales = (o % 3 - 1) * (blk + 1) / 128
    biases = np.broadcast_to((blk % 3 - 1) / 4, (n, k // group))
    expected = reference_f64(x, q, scales, biases, group).astype(np.float32)
    for dtype in ("f32", "bf16"):
        xt, st, bt = (upload(session, storage(v, dtype), dtype) for v in (x, scales, biases))
        wt = upload(session, pack_codes(q, 8), "u32")
        for impl, out in run_all(session, xt, wt, st, bt, 8, group).items():
            np.testing.assert_array_equal(out, expected, err_msg=impl)


def _catalog_layout(session, case, x, packed, s, b):
    """Physical layouts of test/parity/workers/affon-quantized.ts:34-60."""
    rows, inner, outputs = case["shape"]
    per_word = 32 // case["bits"]
    dtype = case["dtype"]
    if "/transposed/" in case["id"]:
        xt = A.transpose(upload(session, np.ascontiguousarray(x.T), dtype), [1, 0])
        padded = np.concatenate([np.zeros((outputs, 1), np.uint32), packed], axis=1)
        wt = A.slice(upload(session, padded, "u32"), [{"start": 0, "stop": outputs}, {"start": 1, "stop": inner // per_word + 1}])
        return xt, wt, upload(session, s, dtype), upload(session, b, dtype)
    if "/offset_" in case["id"]:
        def pad(a, kind):
            p = np.zeros((a.shape[0] + 1, a.shape[1] + 1), a.dtype)
            p[1:, 1:] = a
            t = upload(session, p, kind)
            return A.slice(t, [{"start": 1, "stop": a.shape[0] + 1}, {"start": 1, "stop": a.shape[1] + 1}])
        return pad(x, dtype), pad(packed, "u32"), pad(s, dtype), pad(b, dtype)
    return upload(session, x, dtype), upload(session, packed, "u32"), upload(session, s, dtype), upload(session, b, dtype)


@pytest.mark.parametrize("catalog", ["metal-quantized-grid-128.json", "metal-quantized-views-128.json"])
def test_reference_parity_catalogs(session, catalog):
    """All 256 reference catalog cells with the fixture formula values, checked
    on every element with the catalog oracle's peak-scaled tolerance."""
    cases = json.loads((GOLDEN / catalog).read_text())["cases"]
    for case in cases:
        rows, inner, outputs = case["shape"]
        bits, group, dtype = case["bits"], case["group_size"], case["dtype"]
        xv, q, sv, bv = fixture_operands(rows, inner, outputs, bits, group)
        x, s, b = storage(xv, dtype), storage(sv, dtype), storage(bv, dtype)
        expected = O.quantized_matmul_f64(x, pack_codes(q, bits), s, b, bits, group)
        tol = peak_tolerance(expected, "f32")
        xt, wt, st, bt = _catalog_layout(session, case, x, pack_codes(q, bits), s, b)
        for impl, out in run_all(session, xt, wt, st, bt, bits, group).items():
            err = np.abs(out - expected).max()
            assert err <= tol, (case["id"], impl, err, tol)


def general_checker_cases():
    """The 192 random cases of test/parity/reference/check-cuda-quantized-general.py:34-59
    (seed 20261105), regenerated by tests/golden/make_general_cases.py."""
    data = np.load(GOLDEN / "general_checker_cases.npz", allow_pickle=False)
    result = []
    for i, entry in enumerate(data["ids"]):
        case_id, group = str(entry).split("|")
        bits, x_dtype, p_dtype, _, layout = case_id.split("/")
        result.append(dict(id=case_id, bits=int(bits[1:]), group=int(group), layout=layout, x=data[f"x{i}"],
                           q=data[f"q{i}"].astype(np.int64), s=data[f"s{i}"], b=data[f"b{i}"], x_dtype=x_dtype,
                           p_dtype=p_dtype))
    return result


def _physical(session, arr, kind, layout):
    """check-cuda-quantized-general.py:18-31 layouts."""
    rows, cols = arr.shape
    if layout == "transposed":
        return A.transpose(upload(session, np.ascontiguousarray(arr.T), kind), [1, 0])
    if layout in ("offset", "strided"):
        step = 2 if layout == "strided" else 1
        stored = np.zeros((rows * step + 2, cols * step + 2), arr.dtype)
        stored[1:1 + rows * step:step, 1:1 + cols * step:step] = arr
        t = upload(session, stored, kind)
        return A.slice(t, [{"start": 1, "stop": 1 + rows * step, "step": step},
                           {"start": 1, "stop": 1 + cols * step, "step": step}])
    return upload(session, arr, kind)


def test_reference_general_checker_cases(session):
    """The reference's random checker: 192 cases, torch f64 oracle after source
    dtype rounding, tolerance 2e-6 * max(1, peak) on every element
    (check-cuda-quantized-general.py:71-78,108-110)."""
    cases = general_checker_cases()
    assert len(cases) == 192
    for case in cases:
        bits, group = case["bits"], case["group"]
        x = storage(case["x"], case["x_dtype"])
        s = storage(case["s"], case["p_dtype"])
        b = storage(case["b"], case["p_dtype"])
        packed = pack_codes(case["q"], bits)
        expected = O.quantized_matmul_f64(x, packed, s, b, bits, group)
        tol = 2e-6 * max(1.0, float(np.abs(expected).max()))
        layout = case["layout"]
        xt = _physical(session, x, case["x_dtype"], layout)
        wt = _physical(session, packed, "u32", layout)
        st = _physical(session, s, case["p_dtype"], layout)
        bt = _physical(session, b, case["p_dtype"], layout)
        # exact-class and reassociated-class candidates only: the reference
        # checker's f32 tolerance does not cover bf16-rounded weights.
        for impl, out in run_all(session, xt, wt, st, bt, bits, group,
                                 impls=["auto", "generic", "gemv", "gemv_mfma"]).items():
            err = float(np.abs(out - expected).max())
            assert err <= tol, (case["id"], impl, err, tol)


def seeded_problem(M, N, K, bits, group, x_dtype, p_dtype, seed=1):
    """Affon generator inputs: x ~ N(0,1), W ~ N(0,0.02) quantized by the oracle."""
    xf, xb = O.randn(seed, M * K, 0.0, 1.0)
    wf, wb = O.randn(seed + 1, N * K, 0.0, 0.02)
    x = (xb if x_dtype == "bf16" else xf).reshape(M, K)
    w = (wb if p_dtype == "bf16" else wf).reshape(N, K)
    packed, s, b = O.quantize(w, bits, group, p_dtype)
    return x, packed, s, b


def check_against_oracle(out, x, packed, s, b, bits, group, bf16_input, n_range=None):
    expected = O.quantized_matmul(x, packed, s, b, bits, group, n_range=n_range)
    if n_range is not None:
        out, expected = out[:, n_range[0]:n_range[1]], expected[:, n_range[0]:n_range[1]]
    if bf16_input:
        rms = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
        assert_close_rtol_atol(out, expected, rtol=1e-2, atol=1e-2 * rms)
    else:
        assert_close_rtol_atol(out, expected, rtol=2e-3, atol=1e-4)


@pytest.mark.parametrize("bits,group", [(2, 64), (4, 64), (8, 64), (4, 32), (4, 128), (8, 32)])
@pytest.mark.parametrize("x_dtype,p_dtype", [("f32", "f32"), ("bf16", "bf16"), ("f32", "bf16"), ("bf16", "f32")])
def test_seeded_random_every_implementation(session, bits, group, x_dtype, p_dtype):
    for M, N, K in [(1, 300, 512), (3, 77, 256), (16, 128, 1024), (64, 192, 512)]:
        x, packed, s, b = seeded_problem(M, N, K, bits, group, x_dtype, p_dtype)
        xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
        for impl, out in run_all(session, xt, wt, st, bt, bits, group).items():
            check_against_oracle(out, x, packed, s, b, bits, group, x_dtype == "bf16")


@pytest.mark.parametrize("bits,group", [(4, 64), (8, 32), (2, 16), (4, 3)])
@pytest.mark.parametrize("x_dtype,p_dtype", [("f32", "f32"), ("bf16", "bf16")])
def test_generic_is_bit_identical_to_ordered_cpu_loop(session, bits, group, x_dtype, p_dtype):
    """The exact-class candidate (the only one exact_only admits) reproduces the
    ordered, separately rounded f32 loop bit for bit on non-dyadic data."""
    K = int(np.lcm(32 // bits, group)) * 16
    x, packed, s, b = seeded_problem(3, 50, K, bits, group, x_dtype, p_dtype, seed=4)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    out = session.empty("f32", (3, 50))
    A.quantized_matmul_into(out, xt, wt, st, bt, bits=bits, group_size=group, implementation="generic")
    np.testing.assert_array_equal(out.numpy(), O.quantized_matmul(x, packed, s, b, bits, group))
    exact = session.empty("f32", (3, 50))
    A.quantized_matmul_into(exact, xt, wt, st, bt, bits=bits, group_size=group, policy="exact_only")
    np.testing.assert_array_equal(exact.numpy(), out.numpy())


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("x_dtype,p_dtype", [("bf16", "bf16"), ("f32", "f32"), ("bf16", "f32")])
def test_decode_integer_products_exact(session, bits, x_dtype, p_dtype, rng):
    """Integer activations, every code value, power-of-two scales and integer
    biases make every product and partial sum exact in f32, so the decode
    kernels must match exactly (shapes chosen so the M=1 kernel accepts them:
    K a multiple of 128/bits, group a power-of-two number of 16-byte chunks)."""
    for M, N, K, group in [(1, 37, 512, 64), (1, 130, 4096, 128), (1, 9, 14336, 64), (3, 40, 1024, 64)]:
        q = rng.integers(0, 1 << bits, size=(N, K))
        x = rng.integers(-3, 4, size=(M, K)).astype(np.float64)
        s = 2.0 ** rng.integers(-2, 2, size=(N, K // group))
        b = rng.integers(-2, 3, size=(N, K // group)).astype(np.float64)
        expected = reference_f64(x, q, s, b, group)
        xt = upload(session, storage(x, x_dtype), x_dtype)
        wt = upload(session, pack_codes(q, bits), "u32")
        st, bt = upload(session, storage(s, p_dtype), p_dtype), upload(session, storage(b, p_dtype), p_dtype)
        for impl, out in run_all(session, xt, wt, st, bt, bits, group).items():
            np.testing.assert_array_equal(out, expected.astype(np.float32), err_msg=f"{impl} {M}x{N}x{K} g{group}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_decode_m1_parameter_layouts_exact(session, bits, group, rng):
    """The M=1 kernel loads group parameters once per lane group when a group
    spans at least 2 (4-bit) or 4 (8-bit) 16-byte chunks (g64, g128), and per
    lane otherwise (g32), with K-parts rounded up to the lane-group width
    (8-bit K=4160: 260 chunks in parts of 132 and 128). Integer data make the
    products exact."""
    for N, K in [(67, 4160), (40, 11008), (13, 4096)]:
        if K % group:
            continue
        q = rng.integers(0, 1 << bits, size=(N, K))
        x = rng.integers(-3, 4, size=(1, K)).astype(np.float64)
        s = 2.0 ** rng.integers(-2, 2, size=(N, K // group))
        b = rng.integers(-2, 3, size=(N, K // group)).astype(np.float64)
        expected = reference_f64(x, q, s, b, group).astype(np.float32)
        xt = upload(session, storage(x, "bf16"), "bf16")
        wt = upload(session, pack_codes(q, bits), "u32")
        st, bt = upload(session, storage(s, "bf16"), "bf16"), upload(session, storage(b, "bf16"), "bf16")
        assert A.selected_implementation(xt, wt, st, bt, bits=bits, group_size=group,
                                         implementation="gemv") == "rocm_quantized_matmul.gemv"
        out = session.empty("f32", (1, N))
        A.quantized_matmul_into(out, xt, wt, st, bt, bits=bits, group_size=group, implementation="gemv")
        np.testing.assert_array_equal(out.numpy(), expected, err_msg=f"{bits}-bit g{group} {N}x{K}")


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_decode_sweep_full_size(session, M):
    """8-bit group-64 decode sweep at 14336x4096, bf16 operands, full output."""
    x, packed, s, b = seeded_problem(M, 14336, 4096, 8, 64, "bf16", "bf16", seed=1)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    y = A.quantized_matmul(xt, wt, st, bt, bits=8, group_size=64)
    check_against_oracle(y.numpy(), x, packed, s, b, 8, 64, True)


def test_decode_headline_4bit_full_size(session):
    """4-bit group-64 decode at 14336x4096 (bf16), and the 4096x4096 f32 case."""
    x, packed, s, b = seeded_problem(1, 14336, 4096, 4, 64, "bf16", "bf16", seed=1)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    check_against_oracle(A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=64).numpy(), x, packed, s, b, 4, 64, True)
    x, packed, s, b = seeded_problem(1, 4096, 4096, 4, 64, "f32", "f32", seed=1)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    check_against_oracle(A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=64).numpy(), x, packed, s, b, 4, 64, False)


# ---- prefill GEMM (decoded weights rounded to bf16: numerical class "approximate") ----

def run_mfma(session, x, w, s, b, bits, group):
    out = session.empty("f32", (x.shape[0], w.shape[0]))
    A.quantized_matmul_into(out, x, w, s, b, bits=bits, group_size=group, implementation="mfma", policy="approximate")
    return out.numpy()


def test_prefill_selection_follows_policy(session):
    x, packed, s, b = seeded_problem(64, 128, 256, 4, 64, "bf16", "bf16")
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=64, policy="approximate") == \
        "rocm_quantized_matmul.mfma"
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=64) != "rocm_quantized_matmul.mfma"
    out = session.empty("f32", (64, 128))
    with pytest.raises(_native.NativeError, match="numerical policy"):
        A.quantized_matmul_into(out, xt, wt, st, bt, bits=4, group_size=64, implementation="mfma")
    # K not a multiple of 256: the prefill kernel declines, AUTO falls back.
    x, packed, s, b = seeded_problem(64, 128, 192, 4, 64, "bf16", "bf16")
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    impl = A.selected_implementation(xt, wt, st, bt, bits=4, group_size=64, policy="approximate")
    assert impl != "rocm_quantized_matmul.mfma"
    y = session.empty("f32", (64, 128))
    A.quantized_matmul_into(y, xt, wt, st, bt, bits=4, group_size=64, policy="approximate")
    check_against_oracle(y.numpy(), x, packed, s, b, 4, 64, True)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("p_dtype", ["bf16", "f32"])
def test_prefill_exact_integer_products(session, bits, p_dtype, rng):
    """Power-of-two scales and zero biases keep every decoded weight exact in
    bf16 and every partial sum exact in f32: the GEMM must match exactly,
    including partial M/N tiles and one or many K steps."""
    for M, N, K, group in [(64, 128, 256, 32), (100, 40, 512, 64), (300, 300, 1024, 128), (515, 129, 4096, 64),
                           (256, 256, 11008, 128)]:
        q = rng.integers(0, 1 << bits, size=(N, K))
        x = rng.integers(-3, 4, size=(M, K)).astype(np.float64)
        s = 2.0 ** rng.integers(-3, 1, size=(N, K // group))
        b = np.zeros((N, K // group))
        expected = reference_f64(x, q, s, b, group)
        xt = upload(session, storage(x, "bf16"), "bf16")
        wt = upload(session, pack_codes(q, bits), "u32")
        st, bt = upload(session, storage(s, p_dtype), p_dtype), upload(session, storage(b, p_dtype), p_dtype)
        if p_dtype == "f32" and group == 32:
            # f32 groups of 32 do not fit the kernel's parameter window: it
            # declines, and AUTO falls back to a path that is still exact here.
            with pytest.raises(_native.NativeError, match="cannot run this shape"):
                run_mfma(session, xt, wt, st, bt, bits, group)
            out = session.empty("f32", (M, N))
            A.quantized_matmul_into(out, xt, wt, st, bt, bits=bits, group_size=group, policy="approximate")
            np.testing.assert_array_equal(out.numpy(), expected.astype(np.float32))
            continue
        np.testing.assert_array_equal(run_mfma(session, xt, wt, st, bt, bits, group), expected.astype(np.float32),
                                      err_msg=f"{M}x{N}x{K} g{group}")


@pytest.mark.parametrize("bits,group", [(4, 64), (8, 64), (4, 32), (2, 128)])
def test_prefill_seeded_against_oracle(session, bits, group):
    """Seeded Affon-generator inputs, bf16 activations: rtol 1e-2 with atol
    1e-2 * rms(expected) (decoded weights carry bf16 rounding)."""
    for M, N, K in [(64, 256, 512), (512, 384, 4096), (200, 130, 2048)]:
        x, packed, s, b = seeded_problem(M, N, K, bits, group, "bf16", "bf16", seed=7)
        xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
        check_against_oracle(run_mfma(session, xt, wt, st, bt, bits, group), x, packed, s, b, bits, group, True)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("p_dtype", ["bf16", "f32"])
def test_gemv_mfma_exact_integer_products(session, bits, p_dtype, rng):
    """Small-M MFMA decode kernel: integer codes times integer activations with
    power-of-two scales and integer biases keep every step sum exact, so the
    output must equal the f64 reference exactly (partial column tiles, one or
    many K steps, split K)."""
    for M, N, K, group in [(1, 40, 256, 64), (2, 300, 1024, 128), (5, 129, 4096, 64), (16, 1000, 2048, 256),
                           (16, 4096, 14336, 64), (17, 200, 1024, 64), (32, 1100, 4096, 128)]:
        q = rng.integers(0, 1 << bits, size=(N, K))
        x = rng.integers(-3, 4, size=(M, K)).astype(np.float64)
        s = 2.0 ** rng.integers(-3, 1, size=(N, K // group))
        b = rng.integers(-2, 3, size=(N, K // group)).astype(np.float64)
        expected = reference_f64(x, q, s, b, group)
        xt = upload(session, storage(x, "bf16"), "bf16")
        wt = upload(session, pack_codes(q, bits), "u32")
        st, bt = upload(session, storage(s, p_dtype), p_dtype), upload(session, storage(b, p_dtype), p_dtype)
        out = session.empty("f32", (M, N))
        A.quantized_matmul_into(out, xt, wt, st, bt, bits=bits, group_size=group, implementation="gemv_mfma")
        np.testing.assert_array_equal(out.numpy(), expected.astype(np.float32), err_msg=f"{M}x{N}x{K} g{group}")


VROW_CASES = {  # (M, N, K, group); groups of 32 and 16 keep M = 3, 4 on the virtual-row kernels
    8: [(1, 77, 1024, 64), (2, 300, 512, 32), (2, 129, 2048, 16), (4, 1000, 2048, 64), (8, 64, 4096, 64),
        (6, 200, 1024, 64), (3, 200, 1024, 32), (4, 90, 2048, 16)],
    4: [(1, 77, 4096, 64), (2, 300, 1024, 128), (1, 129, 1024, 32), (4, 1000, 2048, 64), (8, 40, 8192, 128),
        (5, 50, 4096, 128), (4, 300, 1024, 32), (3, 129, 2048, 32)],
    2: [(1, 77, 2048, 64), (2, 300, 2048, 128), (4, 129, 4096, 128), (3, 50, 2048, 128), (2, 129, 4096, 64)],
}


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("p_dtype", ["bf16", "f32"])
def test_virtual_row_decode_exact_integer_products(session, bits, p_dtype, rng):
    """Small-M decode on the matrix cores (the 8-row virtual-row layout at 8
    bits and M <= 2, the 16-row layout up to M = 4, the LDS-tiled kernel for
    larger M and wherever it is the faster one: from M = 2 at 8 bits and
    M = 3 otherwise, for the groups it takes): integer codes and activations
    with power-of-two scales and integer biases make every partial sum exact,
    so the output must equal the f64 reference exactly. Partial row blocks,
    1-4 groups per MFMA span, and 1, 2 or 4 K-parts per row."""
    for M, N, K, group in VROW_CASES[bits]:
        q = rng.integers(0, 1 << bits, size=(N, K))
        x = rng.integers(-3, 4, size=(M, K)).astype(np.float64)
        s = 2.0 ** rng.integers(-3, 1, size=(N, K // group))
        b = rng.integers(-2, 3, size=(N, K // group)).astype(np.float64)
        expected = reference_f64(x, q, s, b, group)
        xt = upload(session, storage(x, "bf16"), "bf16")
        wt = upload(session, pack_codes(q, bits), "u32")
        st, bt = upload(session, storage(s, p_dtype), p_dtype), upload(session, storage(b, p_dtype), p_dtype)
        out = session.empty("f32", (M, N))
        A.quantized_matmul_into(out, xt, wt, st, bt, bits=bits, group_size=group, implementation="gemv_mfma")
        np.testing.assert_array_equal(out.numpy(), expected.astype(np.float32), err_msg=f"{M}x{N}x{K} g{group}")


@pytest.mark.parametrize("M", [2, 3, 4, 8])
def test_virtual_row_decode_against_oracle(session, M):
    """Seeded N(0,1) activations and quantized N(0,0.02) weights, 4-bit and
    8-bit group 64 at the decode sweep's row length: within the bf16
    tolerance of the oracle."""
    for bits in (4, 8):
        x, packed, s, b = seeded_problem(M, 1100, 4096, bits, 64, "bf16", "bf16", seed=13)
        xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
        assert A.selected_implementation(xt, wt, st, bt, bits=bits, group_size=64) == "rocm_quantized_matmul.gemv_mfma"
        y = A.quantized_matmul(xt, wt, st, bt, bits=bits, group_size=64)
        check_against_oracle(y.numpy(), x, packed, s, b, bits, 64, True)


@pytest.mark.parametrize("M", [24, 32])
def test_gemv_mfma_two_row_blocks_against_oracle(session, M):
    """M = 17..32 runs two blocks of 16 MFMA rows on shared decoded codes."""
    x, packed, s, b = seeded_problem(M, 1024, 4096, 4, 64, "bf16", "bf16", seed=5)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=64) == "rocm_quantized_matmul.gemv_mfma"
    y = A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=64)
    check_against_oracle(y.numpy(), x, packed, s, b, 4, 64, True)


@pytest.mark.parametrize("M", [33, 100, 512])
def test_row_tiled_mfma_decode_exact_and_selected(session, M, rng):
    """Beyond 32 activation rows the LDS-tiled gemv_mfma kernel runs row tiles
    of 32 (grid dimension y): the reassociated class's path for prefill, which
    the default policy selects. Integer activations and codes, power-of-two
    scales and integer biases make every sum exact, so the output must equal
    the f64 reference exactly (partial last row tile, split K for the small N)."""
    for bits, N, K, group in ((4, 200, 1024, 64), (8, 72, 2048, 128), (2, 130, 1024, 64)):
        q = rng.integers(0, 1 << bits, size=(N, K))
        x = rng.integers(-3, 4, size=(M, K)).astype(np.float64)
        s = 2.0 ** rng.integers(-3, 1, size=(N, K // group))
        b = rng.integers(-2, 3, size=(N, K // group)).astype(np.float64)
        xt = upload(session, storage(x, "bf16"), "bf16")
        wt = upload(session, pack_codes(q, bits), "u32")
        st, bt = upload(session, storage(s, "bf16"), "bf16"), upload(session, storage(b, "bf16"), "bf16")
        assert A.selected_implementation(xt, wt, st, bt, bits=bits, group_size=group) == \
            "rocm_quantized_matmul.gemv_mfma"
        out = A.quantized_matmul(xt, wt, st, bt, bits=bits, group_size=group).numpy()
        np.testing.assert_array_equal(out, reference_f64(x, q, s, b, group).astype(np.float32),
                                      err_msg=f"M={M} {bits}-bit")


def test_gemv_mfma_selected_for_decode_batches(session):
    x, packed, s, b = seeded_problem(8, 512, 1024, 4, 64, "bf16", "bf16")
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=64) == "rocm_quantized_matmul.gemv_mfma"
    x, packed, s, b = seeded_problem(1, 512, 1024, 4, 64, "bf16", "bf16")
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=64) == "rocm_quantized_matmul.gemv"


def test_prefill_split_k_deterministic(session):
    """Shapes with few tiles split K over workgroups (partials summed in range
    order by the reduction kernel): repeated runs are bit-identical, and match
    the reassociated decode kernel within the bf16 tolerance."""
    for M, N, K, bits, group in [(512, 4096, 14336, 4, 64), (64, 256, 4096, 8, 64), (300, 300, 1024, 2, 128)]:
        x, packed, s, b = seeded_problem(M, N, K, bits, group, "bf16", "bf16", seed=11)
        xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
        first = run_mfma(session, xt, wt, st, bt, bits, group)
        for _ in range(3):
            np.testing.assert_array_equal(run_mfma(session, xt, wt, st, bt, bits, group), first)
        ref = session.empty("f32", (M, N))
        A.quantized_matmul_into(ref, xt, wt, st, bt, bits=bits, group_size=group, implementation="gemv")
        ref = ref.numpy()
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        assert_close_rtol_atol(first, ref, rtol=1e-2, atol=1e-2 * rms)


@pytest.mark.parametrize("shape", [(512, 14336, 4096, 4, 64), (512, 4096, 14336, 4, 64)])
def test_prefill_full_size_against_oracle(session, shape):
    """Full prefill shapes, every implementation AUTO picks under each policy:
    1024 output columns spread across N (all 512 rows) directly against the
    oracle, computed on the host's cores. Tolerance: rtol 1e-2 with atol
    1e-2 * rms(expected) (bf16 activations, f32 accumulation). The two
    policies' outputs must also agree on every element within that tolerance."""
    M, N, K, bits, group = shape
    x, packed, s, b = seeded_problem(M, N, K, bits, group, "bf16", "bf16", seed=3)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    cols = np.unique(np.linspace(0, N - 1, 1024).astype(int))
    expected = oracle_columns(x, packed, s, b, bits, group, cols)
    outs = {}
    for policy in ("approximate", "backend_equivalent"):
        out = session.empty("f32", (M, N))
        A.quantized_matmul_into(out, xt, wt, st, bt, bits=bits, group_size=group, policy=policy)
        outs[policy] = out.numpy()
        assert_bf16_product_close(outs[policy][:, cols], expected)
    assert_bf16_product_close(outs["approximate"], outs["backend_equivalent"])


# ---- quantize / dequantize ----------------------------------------------------------

@pytest.mark.parametrize("bits,group", [(2, 32), (4, 64), (8, 64), (4, 32), (4, 128), (8, 16), (2, 8), (4, 48),
                                        (4, 3), (2, 64), (8, 256)])
@pytest.mark.parametrize("w_dtype,p_dtype", [("f32", "f32"), ("f32", "bf16"), ("bf16", "bf16")])
def test_quantize_bit_exact(session, bits, group, w_dtype, p_dtype):
    per_word = 32 // bits
    cols = int(np.lcm(per_word, group)) * 8
    rows = 37
    wf, wb = O.randn(9, rows * cols, 0.0, 0.02)
    w = (wb if w_dtype == "bf16" else wf).reshape(rows, cols)
    w[3, :group] = 0.125            # constant group
    if w_dtype == "f32":
        w[4, :group] = -0.0        # signed zeros
        w[4, 1:group:2] = 0.0
    # exact ties k + 1/2 for the stored scale and bias: rounding half to even is observable
    ties, tie_codes = tie_group(bits, group)
    w[5, group:2 * group] = O.bf16_from_f32(ties) if w_dtype == "bf16" else ties
    # quotients a few ulps from k + 1/2 for a scale that is not a power of two
    near = near_tie_group(bits, group, p_dtype)
    w[6, :group] = O.bf16_from_f32(near) if w_dtype == "bf16" else near
    # NaN as a group's first value, as the first value of a later word of a
    # group, and inside a word: the group's scale and codes follow the
    # comparison scan from the group's first value
    nan = O.bf16_from_f32(np.float32(np.nan)).reshape(-1)[0] if w_dtype == "bf16" else np.float32(np.nan)
    for c in [0, 2 * group + 1] + ([group + per_word] if group > per_word else []):
        w[7, c] = nan
    expected = O.quantize(w, bits, group, p_dtype)
    np.testing.assert_array_equal(unpack_bytes_le(expected[0], bits)[5, group:2 * group], tie_codes)
    packed, scales, biases = A.quantize(upload(session, w, w_dtype), bits=bits, group_size=group,
                                        param_dtype=p_dtype)
    np.testing.assert_array_equal(packed.storage(), expected[0])
    np.testing.assert_array_equal(scales.storage(), expected[1])
    np.testing.assert_array_equal(biases.storage(), expected[2])
    for out_dtype in ("f32", "bf16"):
        deq = A.dequantize(packed, scales, biases, bits=bits, group_size=group, dtype=out_dtype)
        np.testing.assert_array_equal(deq.storage(), O.dequantize(*expected, bits, group, out_dtype))


def test_quantize_full_size_stress_bit_exact(session):
    """f32 [28672, 8192] at 4-bit group 32 with bf16 parameters, and its
    dequantization back to f32 and to bf16."""
    rows, cols = 28672, 8192
    w, _ = O.randn(2, rows * cols, 0.0, 0.02)
    w = w.reshape(rows, cols)
    expected = O.quantize(w, 4, 32, "bf16")
    packed, scales, biases = A.quantize(upload(session, w, "f32"), bits=4, group_size=32, param_dtype="bf16")
    np.testing.assert_array_equal(packed.storage(), expected[0])
    np.testing.assert_array_equal(scales.storage(), expected[1])
    np.testing.assert_array_equal(biases.storage(), expected[2])
    del w
    for out_dtype in ("f32", "bf16"):
        deq = A.dequantize(packed, scales, biases, bits=4, group_size=32, dtype=out_dtype)
        np.testing.assert_array_equal(deq.storage(), O.dequantize(*expected, 4, 32, out_dtype))
        del deq


def test_prefill_stress_full_size_sampled(session):
    """Large prefill stress: x bf16 [2048, 8192], 4-bit group 32, bf16
    parameters, W [28672, 8192] and W [8192, 28672] (the same seeded values in
    both shapes), quantized on the GPU (bit-exactness of that quantize: the
    test above), under the approximate policy. Every activation row of 112
    sampled columns per orientation (the first and last 16, which lie in the
    first and last column tiles, and 80 spread over the rest) against the
    oracle, within the bf16-input tolerance. The default policy's run of the
    same shapes: tests/test_gpu_prefill_g32.py."""
    wf, _ = O.randn(2, 28672 * 8192, 0.0, 0.02)
    _, xb = O.randn(1, 2048 * 8192, 0.0, 1.0)
    x = xb.reshape(2048, 8192)
    for N, K in ((28672, 8192), (8192, 28672)):
        w = wf.reshape(N, K)
        packed, scales, biases = A.quantize(upload(session, w, "f32"), bits=4, group_size=32, param_dtype="bf16")
        # activations of the second orientation: the seeded rows repeated to K columns
        xk = x if K == 8192 else np.ascontiguousarray(np.tile(x, (1, -(-K // 8192)))[:, :K])
        xt = upload(session, xk, "bf16")
        y = run_mfma(session, xt, packed, scales, biases, 4, 32)
        cols = np.unique(np.concatenate([np.arange(16), np.linspace(0, N - 1, 80).astype(int), np.arange(N - 16, N)]))
        expected = oracle_columns(xt.storage(), packed.storage(), scales.storage(), biases.storage(), 4, 32, cols)
        assert_bf16_product_close(y[:, cols], expected)


def test_checkpoint_adapter_quantized_linears(session, tmp_path, rng):
    """MLX-affine checkpoint layers loaded onto the device: one shaped like the
    reference's checkpoint evidence (8-bit group 64, U32 [2048,256] with BF16
    [2048,16] scales/biases, docs/core/quantized-inference.md:89-96), one
    4-bit group 64 layer, one U32 tensor without parameters (not a layer).
    Loaded storage is bit-identical to the file, and each layer applied to the
    reference tool's activations ((c*7 + r*3) % 31 - 15)/16
    (tools/test-quantized-checkpoint.py:53) matches the oracle."""
    from affon_amd import checkpoint as C
    from tests.test_checkpoint import write_file
    layers = {"talker.lm_head.0": (8, 2048, 1024), "talker.proj": (4, 300, 512)}
    entries, arrays = [], {}
    for prefix, (bits, out, inp) in layers.items():
        q = rng.integers(0, 1 << bits, size=(out, inp))
        s = O.bf16_from_f32(rng.uniform(0.001, 0.01, size=(out, inp // 64)).astype(np.float32))
        b = O.bf16_from_f32(rng.uniform(-0.5, 0.5, size=(out, inp // 64)).astype(np.float32))
        arrays[prefix] = (pack_codes(q, bits), s, b)
        entries += [(prefix + ".weight", "U32", [out, inp * bits // 32], arrays[prefix][0].tobytes()),
                    (prefix + ".scales", "BF16", list(s.shape), s.tobytes()),
                    (prefix + ".biases", "BF16", list(b.shape), b.tobytes())]
    entries.append(("talker.codebook.weight", "U32", [16, 4], np.arange(64, dtype=np.uint32).tobytes()))
    path = str(write_file(tmp_path / "model.safetensors", entries, metadata={"format": "mlx"}))
    for prefix, (bits, out, inp) in layers.items():
        bound = C.quantized_linears(session, path, bits=bits, group_size=64, prefixes=[prefix])[prefix]
        assert (bound.out_features, bound.in_features) == (out, inp)
        for tensor, expected in zip((bound.packed, bound.scales, bound.biases), arrays[prefix]):
            np.testing.assert_array_equal(tensor.storage(), expected)
        x = np.array([[((c * 7 + r * 3) % 31 - 15) / 16 for c in range(inp)] for r in range(3)], np.float32)
        y = bound(session.tensor(x, "f32")).numpy()
        check_against_oracle(y, x, *arrays[prefix], bits, 64, False)
    with pytest.raises(C.CheckpointError, match="shapes do not match"):
        C.quantized_linears(session, path, bits=4, group_size=64)  # the 8-bit layer read as 4-bit
    t = C.load(session, path, ["talker.codebook.weight"])["talker.codebook.weight"]
    np.testing.assert_array_equal(t.storage(), np.arange(64, dtype=np.uint32).reshape(16, 4))


# ---- boundary behaviour -------------------------------------------------------------------

def test_drop_in_host_pointer_entry_point():
    """compute_core_cyna_smoke.zig:970-984 through the exact reference signature."""
    lib = _native.load()
    a = np.array([1, 2, 3, 4, 5, 6, 7, 8, 2, 3, 4, 5, 6, 7, 8, 9], np.float32)
    w = np.array([0x01010101] * 2 + [0x02020202] * 2 + [0x03030303] * 2, np.uint32)
    s, b = np.ones(6, np.float32), np.zeros(6, np.float32)
    out = np.full(6, -1.0, np.float32)
    args = (a.ctypes.data, 16, w.ctypes.data, 6, s.ctypes.data, 6, b.ctypes.data, 6, out.ctypes.data, 6)
    assert lib.compute_core_run_quantized_matmul_f32(*args, 2, 8, 3, 8, 4) == 0
    assert out.tolist() == [36, 72, 108, 44, 88, 132]
    out[:] = -1
    assert lib.compute_core_run_quantized_matmul_f32(*args, 2, 8, 3, 3, 4) == 1
    assert out.tolist() == [-1] * 6


def test_program_explain_and_policies(session):
    source = A.program("quantized_linear", lambda p: A.quantized_matmul(
        p.argument("x", A.TensorSpec.f32([1, 4])), p.argument("w", A.TensorSpec.u32([1, 1])),
        p.argument("s", A.TensorSpec.bf16([1, 1])), p.argument("b", A.TensorSpec.bf16([1, 1])),
        {"bits": 8, "group_size": 4}))
    executable = session.compile(source, explanationLevel="detailed")
    explanation = json.dumps(executable.explain())
    assert "rocm_quantized_matmul" in explanation and "rocm_host_" not in explanation
    exact = session.compile(source, numericalPolicy="exact_only")
    assert "rocm_quantized_matmul.generic" in json.dumps(exact.explain())
    x = session.tensor([[1, 2, 3, 4]])
    w = session.tensor([[0x04030201]], dtype="u32")
    s = session.tensor([[1]], dtype="bf16")
    b = session.tensor([[0]], dtype="bf16")
    assert executable.run({"x": x, "w": w, "s": s, "b": b}).to_array() == [[30]]
    assert exact.run({"x": x, "w": w, "s": s, "b": b}).to_array() == [[30]]


def test_cross_session_and_bits_rejected(session):
    other = A.Session("rocm")
    try:
        x = session.tensor([[1, 2, 3, 4]])
        w = session.tensor([[0xFFFFFFFF]], dtype="u32")
        s = session.tensor([[1]])
        b = other.tensor([[0]])
        with pytest.raises(TypeError, match="same Session"):
            A.quantized_matmul(x, w, s, b, bits=8, group_size=4)
        with pytest.raises(TypeError, match="bits"):
            A.quantized_matmul(x, w, s, session.tensor([[0]]), bits=3, group_size=4)
    finally:
        other.dispose()


def test_executable_reusable_after_rejected_run(session):
    """test/e2e/program/execution/recovery.test.ts:7-22."""
    source = A.program("q", lambda p: A.quantized_matmul(
        p.argument("x", A.TensorSpec.f32([1, 4])), p.argument("w", A.TensorSpec.u32([1, 1])),
        p.argument("s", A.TensorSpec.f32([1, 1])), p.argument("b", A.TensorSpec.f32([1, 1])), bits=8, group_size=4))
    executable = session.compile(source)
    good = dict(x=session.tensor([[1, 2, 3, 4]]), w=session.tensor([[0x04030201]], dtype="u32"),
                s=session.tensor([[1]]), b=session.tensor([[0]]))
    with pytest.raises(TypeError):
        executable.run({**good, "x": session.tensor([[1, 2, 3]])})
    assert executable.run(good).to_array() == [[30]]
