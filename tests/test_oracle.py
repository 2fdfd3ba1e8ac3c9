"""Pins the CPU oracle before it is trusted as the checker (runs without a GPU).

Each check is chosen so that a plausible mistake in the oracle (wrong lane
order, dropped bias, group index off by one, transposed operand, wrong
rounding) fails at least one of them.
"""
import math
import pathlib
import json

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import (fixture_operands, near_tie_group, pack_codes, reference_f64, storage, tie_group,
                           unpack_bytes_le, widened)


def _operands(case):
    x = storage(case["input"]["values"], case["input"]["dtype"])
    packed = np.array(case["packed"], dtype=np.uint32)
    s = storage(case["scales"]["values"], case["scales"]["dtype"])
    b = storage(case["biases"]["values"], case["biases"]["dtype"])
    return x, packed, s, b


def test_known_answers(kats):
    for case in kats["cases"]:
        x, packed, s, b = _operands(case)
        out = O.quantized_matmul(x, packed, s, b, case["bits"], case["group_size"])
        assert out.tolist() == case["expected"], case["name"]
        out64 = O.quantized_matmul_f64(x, packed, s, b, case["bits"], case["group_size"])
        assert out64.tolist() == case["expected"], case["name"]


def test_view_known_answer_materialized(kats):
    case = kats["views"][0]
    x = np.array(case["base_input"]["values"], dtype=np.float32).T.copy()
    (r0, r1), (c0, c1) = case["packed_view"]["slice"]
    packed = np.array(case["base_packed"], dtype=np.uint32)[r0:r1, c0:c1]
    (p0, p1), (q0, q1) = case["param_view"]["slice"]
    s = storage(case["base_scales"]["values"], "bf16")[p0:p1, q0:q1]
    b = storage(case["base_biases"]["values"], "bf16")[p0:p1, q0:q1]
    out = O.quantized_matmul(x, packed, s, b, case["bits"], case["group_size"])
    assert out.tolist() == case["expected"]


def crossing_word_case():
    """quantized-matmul.test.ts:95-122: K=24, N=3, M=2, g=3, 4-bit."""
    k, n, m, g = 24, 3, 2, 3
    q = np.array([[(row * 5 + col) % 16 for col in range(k)] for row in range(n)])
    x = np.array([[((row + col) % 7 - 3) / 8 for col in range(k)] for row in range(m)])
    scales = np.array([[(grp % 3 - 1) / 4 for grp in range(k // g)] for _ in range(n)])
    biases = np.array([[grp % 2 - 0.5 for grp in range(k // g)] for _ in range(n)])
    expected = [[sum(x[r][c] * (scales[o][c // g] * q[o][c] + biases[o][c // g]) for c in range(k))
                 for o in range(n)] for r in range(m)]
    return x, q, scales, biases, g, expected


def test_groups_crossing_words_zero_and_negative_scales():
    x, q, scales, biases, g, expected = crossing_word_case()
    packed = pack_codes(q, 4)
    for dtype in ("f32", "bf16"):
        out = O.quantized_matmul(storage(x, dtype), packed, storage(scales, dtype), storage(biases, dtype), 4, g)
        assert out.tolist() == expected


def tile_edge_case(bits, m):
    """quantized-matmul.test.ts:123-148."""
    n, k, g = (64, 96, 16) if m >= 64 else (19, 80, 16)
    mask = (1 << bits) - 1
    x = np.array([[((r + c) % 7 - 3) / 8 for c in range(k)] for r in range(m)])
    q = np.array([[(r * 5 + c) & mask for c in range(k)] for r in range(n)])
    scales = np.array([[(grp % 3 - 1) / 4 for grp in range(k // g)] for _ in range(n)])
    biases = np.array([[grp % 2 - 0.5 for grp in range(k // g)] for _ in range(n)])
    expected = reference_f64(x, q, scales, biases, g)
    return x, q, scales, biases, g, expected


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_tile_edges_exact(bits):
    for m in (1, 3, 4, 7, 16, 17, 33, 64, 128):
        x, q, scales, biases, g, expected = tile_edge_case(bits, m)
        out = O.quantized_matmul(storage(x, "bf16"), pack_codes(q, bits), storage(scales, "bf16"),
                                 storage(biases, "bf16"), bits, g)
        np.testing.assert_array_equal(out, expected.astype(np.float32))


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_group_specialization_closed_form(group, dtype):
    """quantized-matmul.test.ts:171-184: x=1, q=128, s=(g+1)/128, b=-1 gives g*G*(G-1)/2."""
    m, n, k = 8, 3, 128
    groups = k // group
    x = storage(np.ones((m, k)), "bf16")
    packed = np.full((n, k // 4), 0x80808080, dtype=np.uint32)
    s = storage([[(g + 1) / 128 for g in range(groups)] for _ in range(n)], dtype)
    b = storage(np.full((n, groups), -1.0), dtype)
    out = O.quantized_matmul(x, packed, s, b, 8, group)
    assert (out == group * groups * (groups - 1) / 2).all()


@pytest.mark.parametrize("group", [48, 64])
def test_groups_across_k_tiles(group):
    """quantized-matmul.test.ts:186-204."""
    m, n = 64, 64
    k = 96 if group == 48 else 256
    r = np.arange(m)[:, None]
    c = np.arange(k)[None, :]
    x = ((r + c) % 11 - 5) / 8
    o = np.arange(n)[:, None]
    q = (o + c) % 256
    blk = np.arange(k // group)[None, :]
    scales = (o % 3 - 1) * (blk + 1) / 128
    biases = np.broadcast_to((blk % 3 - 1) / 4, (n, k // group))
    expected = reference_f64(x, q, scales, biases, group)
    for dtype in ("f32", "bf16"):
        out = O.quantized_matmul(storage(x, dtype), pack_codes(q, 8), storage(scales, dtype), storage(biases, dtype),
                                 8, group)
        np.testing.assert_array_equal(out, expected.astype(np.float32))


def test_parity_fixture_formula():
    """quantized_fixture.py:36-45 restated in f64 against the oracle."""
    for rows, inner, outputs, bits, group in [(1, 32, 3, 8, 4), (2, 64, 17, 4, 16), (16, 128, 8, 2, 32)]:
        x, q, scales, biases = fixture_operands(rows, inner, outputs, bits, group)
        expected = reference_f64(x, q, scales, biases, group)
        out = O.quantized_matmul(storage(x, "f32"), pack_codes(q, bits), storage(scales, "f32"),
                                 storage(biases, "f32"), bits, group)
        np.testing.assert_allclose(out, expected, rtol=0, atol=2e-6 * max(1, np.abs(expected).max()))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_random_against_little_endian_byte_decode(bits, rng):
    """An f64 product that decodes codes from little-endian bytes (not u32 shifts)."""
    m, n, k, group = 3, 11, 256, 32
    packed = rng.integers(0, 2**32, size=(n, k * bits // 32), dtype=np.uint64).astype(np.uint32)
    x = storage(rng.standard_normal((m, k)), "bf16")
    s = storage(rng.random((n, k // group)) / (1 << bits), "f32")
    b = storage(rng.random((n, k // group)) - 0.5, "f32")
    q = unpack_bytes_le(packed, bits)
    expected = reference_f64(widened(x), q, widened(s), widened(b), group)
    out64 = O.quantized_matmul_f64(x, packed, s, b, bits, group)
    np.testing.assert_allclose(out64, expected, rtol=1e-12, atol=1e-12)
    out32 = O.quantized_matmul(x, packed, s, b, bits, group)
    # Ordered f32 accumulation: error bounded by K * eps * sum |x*w|.
    bound = k * 2**-23 * (np.abs(widened(x)) @ np.abs(q * np.repeat(widened(s), group, 1)
                                                     + np.repeat(widened(b), group, 1)).T)
    assert (np.abs(out32 - expected) <= bound + 1e-30).all()


def test_special_case_integer_matmul(rng):
    """bits=8, s=1, b=0 with integer activations is an integer matmul."""
    m, n, k = 4, 9, 64
    q = rng.integers(0, 256, size=(n, k))
    x = rng.integers(-8, 8, size=(m, k))
    out = O.quantized_matmul(x.astype(np.float32), pack_codes(q, 8), np.ones((n, 2), np.float32),
                             np.zeros((n, 2), np.float32), 8, 32)
    np.testing.assert_array_equal(out, (x @ q.T).astype(np.float32))


def test_special_case_single_group(rng):
    """g = K: y = s * (x . q) + b * sum(x)."""
    m, n, k, bits = 2, 5, 64, 4
    q = rng.integers(0, 16, size=(n, k))
    x = rng.standard_normal((m, k)).astype(np.float32)
    s = (rng.random((n, 1)) * 0.1).astype(np.float32)
    b = (rng.random((n, 1)) - 0.5).astype(np.float32)
    expected = (x.astype(np.float64) @ q.T) * s.T.astype(np.float64) + x.astype(np.float64).sum(1, keepdims=True) * b.T
    out = O.quantized_matmul(x, pack_codes(q, bits), s, b, bits, k)
    np.testing.assert_allclose(out, expected, rtol=1e-5, atol=1e-5)


def test_bias_and_scale_are_not_swapped():
    """A single code pins which parameter multiplies: q=3, s=2, b=5 -> 11 per unit x."""
    packed = np.array([[0x3]], dtype=np.uint32) | np.array([[0]], dtype=np.uint32)
    out = O.quantized_matmul(np.array([[1, 0, 0, 0]], np.float32), packed, np.array([[2]], np.float32),
                             np.array([[5]], np.float32), 8, 4)
    assert out.tolist() == [[11.0]]


# ---- bf16 rounding -----------------------------------------------------------

def _reference_formula(values: np.ndarray) -> np.ndarray:
    """probe-capabilities.py:112-115 restated on bit patterns."""
    bits = values.view(np.uint32).astype(np.uint64)
    return (((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000) >> 16).astype(np.uint16)


def test_bf16_structured_exhaustive():
    """Every upper half with the low halves that decide rounding (ties, both
    sides of ties, extremes), finite values only."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFE, 0x7FFF, 0x8000, 0x8001, 0xFFFE, 0xFFFF, 0x1234, 0xC000], dtype=np.uint32)
    patterns = (hi[:, None] | lows[None, :]).reshape(-1)
    values = patterns.view(np.float32)
    finite = np.isfinite(values)
    # Values that would round past the largest finite bf16 are excluded from
    # the formula comparison (the formula wraps into the exponent field as
    # IEEE rounding to infinity does, so they agree anyway).
    got = O.bf16_from_f32(values[finite])
    np.testing.assert_array_equal(got, _reference_formula(values[finite]))
    nan = O.bf16_from_f32(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_bf16_matches_torch_rounding(rng):
    """torch's float32 -> bfloat16 conversion is round-to-nearest-even."""
    torch = pytest.importorskip("torch")
    values = np.concatenate([rng.standard_normal(200_000).astype(np.float32),
                             (rng.standard_normal(50_000) * 1e-38).astype(np.float32),
                             rng.integers(0, 2**32, 50_000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    values = values[np.isfinite(values)]
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.bf16_from_f32(values), expected)


# ---- seeded generator ------------------------------------------------------------------

def _mulberry32_js(seed: int, count: int) -> list[float]:
    """program.ts:1385-1394 with JS int32 semantics spelled out (Math.imul,
    ToInt32 of the sum), an implementation independent of the C one."""
    def imul(a, b):
        return ((a & 0xFFFFFFFF) * (b & 0xFFFFFFFF)) & 0xFFFFFFFF

    def to_int32(v):
        v &= 0xFFFFFFFF
        return v - (1 << 32) if v >= (1 << 31) else v

    value = seed & 0xFFFFFFFF
    out = []
    for _ in range(count):
        value = (value + 0x6D2B79F5) & 0xFFFFFFFF
        nxt = to_int32(value)
        nxt = to_int32(imul(nxt ^ ((nxt & 0xFFFFFFFF) >> 15), nxt | 1))
        nxt = to_int32(nxt ^ (nxt + to_int32(imul(nxt ^ ((nxt & 0xFFFFFFFF) >> 7), nxt | 61))))
        out.append(((nxt ^ ((nxt & 0xFFFFFFFF) >> 14)) & 0xFFFFFFFF) / 4294967296)
    return out


def test_mulberry32_stream():
    for seed in (0, 1, 2, 3, 42, 20261105):
        assert O.uniforms(seed, 64).tolist() == _mulberry32_js(seed, 64)


def _generator_vectors():
    path = pathlib.Path(__file__).resolve().parent / "golden" / "generator_vectors.json"
    return json.loads(path.read_text())["cases"]


def _seed_value(text):
    return float(text) if "." in text else int(text)


def test_generator_matches_reference_js():
    """The reference's own seededRandom and normal() (program.ts:1385-1413),
    run under node by tests/golden/make_generator_vectors.py: uniforms exactly,
    and Tensor.randn's f32 values (mean + std * normal(), rounded to f32) for
    std 1 and 0.02, from the oracle's C generator and from the product's
    vectorized one. The seeds include JS's seed normalization cases: negative,
    past 2^32, not a safe integer (2^53), and fractional."""
    from affon_amd import generator as G
    for case in _generator_vectors():
        seed = _seed_value(case["seed"])
        uniforms = np.array([float(v) for v in case["uniforms"]])
        np.testing.assert_array_equal(O.uniforms(seed, 64), uniforms, err_msg=f"oracle uniforms, seed {seed}")
        np.testing.assert_array_equal(G.uniforms(seed, 0, 64), uniforms, err_msg=f"product uniforms, seed {seed}")
        for key, std in (("f32_std1", 1.0), ("f32_std002", 0.02)):
            want = np.array([float(v) for v in case[key]], dtype=np.float32)
            got, _ = O.randn(seed, 65, mean=0.0, std=std)
            np.testing.assert_array_equal(got, want, err_msg=f"oracle randn, seed {seed}, std {std}")
            np.testing.assert_array_equal(G.normal_f32(seed, 65, 0.0, std), want,
                                          err_msg=f"product randn, seed {seed}, std {std}")


def test_randn_box_muller_and_moments():
    u = _mulberry32_js(7, 4)
    radius = math.sqrt(-2 * math.log(max(u[0], 2.220446049250313e-16)))
    angle = 2 * math.pi * u[1]
    f32, bf16 = O.randn(7, 3, mean=0.0, std=1.0)
    assert f32[0] == np.float32(radius * math.cos(angle))
    assert f32[1] == np.float32(radius * math.sin(angle))
    np.testing.assert_array_equal(bf16, O.bf16_from_f32(f32))
    values, _ = O.randn(1, 1 << 20, mean=0.0, std=0.02)
    assert abs(values.mean()) < 1e-4 and abs(values.std() - 0.02) < 1e-4


# ---- quantize / dequantize -----------------------------------------------------------------

@pytest.mark.parametrize("bits,group", [(2, 8), (2, 32), (4, 3), (4, 32), (4, 64), (8, 16), (8, 256)])
@pytest.mark.parametrize("param_dtype", ["f32", "bf16"])
def test_quantize_rounds_exact_ties_to_even(bits, group, param_dtype):
    """Groups whose (w - b) / s is exactly k + 1/2 for the stored scale and
    bias (tests.helpers.tie_group): the codes are the even neighbours
    (rintf, round half to even), which rounding half away from zero would
    miss on every even k. The tie group sits in several group slots of a row
    among random groups, with the rows' other groups untouched."""
    per_word = 32 // bits
    cols = int(np.lcm(per_word, group)) * 4
    values, codes = tie_group(bits, group)
    w, _ = O.randn(5, 3 * cols, 0.0, 0.02)
    w = w.reshape(3, cols)
    slots = [0, cols // group - 1]
    for slot in slots:
        w[1, slot * group:(slot + 1) * group] = values
    packed, scales, biases = O.quantize(w, bits, group, param_dtype)
    q = unpack_bytes_le(packed, bits)
    for slot in slots:
        np.testing.assert_array_equal(q[1, slot * group:(slot + 1) * group], codes, err_msg=f"group slot {slot}")
        assert widened(scales[1:2, slot:slot + 1])[0, 0] == 0.125 and widened(biases[1:2, slot:slot + 1])[0, 0] == -1.5
    ties = codes[2:2 + max(0, min((1 << bits) - 1, group - 2, 128))]
    assert (ties != np.arange(1, ties.size + 1)).any(), "half-away rounding would give these codes"


@pytest.mark.parametrize("bits,group", [(2, 8), (2, 32), (4, 3), (4, 32), (4, 64), (8, 16), (8, 256)])
@pytest.mark.parametrize("param_dtype", ["f32", "bf16"])
def test_quantize_near_ties_follow_the_division(bits, group, param_dtype):
    """The near-tie group of tests.helpers.near_tie_group: the codes are
    rint((w - b) / s) with the division correctly rounded, and on some values
    of the group rint((w - b) * RN(1/s)) is another code, so a quantizer that
    skips the division there fails the GPU test that uses this group."""
    per_word = 32 // bits
    cols = int(np.lcm(per_word, group)) * 4
    values = near_tie_group(bits, group, param_dtype)
    w = np.zeros((1, cols), np.float32)
    w[0, :group] = values
    packed, scales, biases = O.quantize(w, bits, group, param_dtype)
    s, b = np.float32(widened(scales)[0, 0]), np.float32(widened(biases)[0, 0])
    assert b == 0.0 and s not in (0.125, 0.25, 0.5)
    levels = (1 << bits) - 1
    d = (values - b).astype(np.float32)
    codes = unpack_bytes_le(packed, bits)[0, :group]
    np.testing.assert_array_equal(codes, np.clip(np.rint((d / s).astype(np.float32)), 0, levels))
    by_reciprocal = np.clip(np.rint((d * np.float32(np.float32(1) / s)).astype(np.float32)), 0, levels)
    assert (by_reciprocal != codes).any()



@pytest.mark.parametrize("bits,group", [(2, 32), (4, 64), (8, 64), (4, 32), (4, 128), (8, 16), (2, 8), (4, 48)])
@pytest.mark.parametrize("param_dtype", ["f32", "bf16"])
def test_quantize_recovers_exact_affine_rows(bits, group, param_dtype, rng):
    """Rows built as b + s*q with dyadic s, b and both extreme codes in every
    group quantize back to exactly (q, s, b)."""
    n, k = 6, group * 4
    max_q = (1 << bits) - 1
    q = rng.integers(0, max_q + 1, size=(n, k))
    q[:, ::group] = 0
    q[:, 1::group] = max_q
    s = 2.0 ** rng.integers(-10, -2, size=(n, k // group))
    b = rng.integers(-64, 64, size=(n, k // group)) / 256
    w = (np.repeat(b, group, 1) + np.repeat(s, group, 1) * q).astype(np.float32)
    packed, scales, biases = O.quantize(w, bits, group, param_dtype)
    np.testing.assert_array_equal(unpack_bytes_le(packed, bits), q)
    np.testing.assert_array_equal(widened(scales), s)
    np.testing.assert_array_equal(widened(biases), b)


@pytest.mark.parametrize("bits,group", [(4, 64), (8, 64), (4, 32), (2, 64)])
@pytest.mark.parametrize("param_dtype", ["f32", "bf16"])
def test_quantize_invariants(bits, group, param_dtype):
    n, k = 64, 512
    w, _ = O.randn(11, n * k, 0.0, 0.02)
    w = w.reshape(n, k)
    max_q = (1 << bits) - 1
    packed, scales, biases = O.quantize(w, bits, group, param_dtype)
    q = unpack_bytes_le(packed, bits).reshape(n, k // group, group)
    wg = w.reshape(n, k // group, group).astype(np.float64)
    s, b = widened(scales), widened(biases)
    if param_dtype == "f32":
        # The stored bias is the group minimum and the stored scale spans the range.
        assert (q.min(axis=2) == 0).all() and (q.max(axis=2) == max_q).all()
        np.testing.assert_array_equal(np.argmin(wg, 2), np.argmin(np.where(q == 0, wg, np.inf), 2))
    else:
        # bf16 rounding moves the bias by up to |min| * 2^-9, which is a
        # fraction of a step for these weights: the extremes land within one code.
        assert (q.min(axis=2) <= 1).all() and (q.max(axis=2) >= max_q - 1).all()
    deq = s[..., None] * q + b[..., None]
    # f32 parameters: half a step plus rounding; bf16 parameters add the
    # parameter rounding carried over the whole code range.
    slack = 1e-6 if param_dtype == "f32" else (2**-8) * (np.abs(b) + max_q * s)[..., None]
    assert (np.abs(deq - wg) <= s[..., None] / 2 * (1 + 1e-5) + slack).all()
    exact_scale = (wg.max(2) - wg.min(2)) / max_q
    assert (np.abs(s - exact_scale) <= exact_scale * (2**-8 if param_dtype == "bf16" else 2**-22)).all()


def test_quantize_constant_and_signed_zero_groups():
    w = np.zeros((3, 64), dtype=np.float32)
    w[0, :] = 0.375
    w[1, :32] = -0.0
    w[2, ::2] = -0.0
    packed, scales, biases = O.quantize(w, 4, 32, "f32")
    assert (packed == 0).all()
    assert (scales.view(np.uint32) == 0).all()  # +0.0, never -0.0
    assert biases[0].tolist() == [0.375, 0.375]
    assert (biases[1:].view(np.uint32) == 0).all()
    np.testing.assert_array_equal(O.dequantize(packed, scales, biases, 4, 32), np.abs(w) * np.sign(w + 1))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_codes_are_idempotent(bits):
    n, k, group = 16, 256, 64
    w, _ = O.randn(5, n * k, 0.0, 0.02)
    packed, scales, biases = O.quantize(w.reshape(n, k), bits, group, "f32")
    again = O.quantize(O.dequantize(packed, scales, biases, bits, group), bits, group, "f32")
    np.testing.assert_array_equal(again[0], packed)


def test_dequantize_hand_built_words():
    packed = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    s = np.array([[0.5, 2.0]], np.float32)
    b = np.array([[-1.0, 3.0]], np.float32)
    out = O.dequantize(packed, s, b, 4, 8)
    expected = [[0.5 * i - 1 for i in range(8)] + [2.0 * i + 3 for i in range(8, 16)]]
    assert out.tolist() == expected
    bf = O.dequantize(packed, s, b, 4, 8, out_dtype="bf16")
    np.testing.assert_array_equal(bf, O.bf16_from_f32(np.array(expected, np.float32)))


def test_product_generator_matches_oracle_generator():
    """The vectorized Tensor.randn of the package against the sequential C
    restatement, bit for bit (odd count exercises the unused spare)."""
    from affon_amd.generator import normal_f32
    for seed, count, mean, std in [(1, 4097, 0.0, 1.0), (2, 10_001, 0.0, 0.02), (20261105, 3, 0.5, 2.0)]:
        expected, _ = O.randn(seed, count, mean, std)
        np.testing.assert_array_equal(normal_f32(seed, count, mean, std), expected)


# ---- element-wise epilogue ops (add of the output bias, silu gate) ----

def test_add_output_bias_exact_dyadic(rng):
    """Dyadic values with few significant bits add exactly in f32, so the sum
    is fixed; a zero bias is the identity; a bf16 bias is widened exactly."""
    y = rng.integers(-64, 64, size=(3, 10)) / 8.0
    bias = rng.integers(-16, 16, size=10) / 4.0
    got = O.add_output_bias(y.astype(np.float32), bias.astype(np.float32))
    np.testing.assert_array_equal(got, (y + bias[None, :]).astype(np.float32))
    np.testing.assert_array_equal(O.add_output_bias(y.astype(np.float32), O.bf16_from_f32(bias.astype(np.float32))),
                                  got)
    yr = rng.standard_normal((2, 5)).astype(np.float32)
    np.testing.assert_array_equal(O.add_output_bias(yr, np.zeros(5, np.float32)), yr)


def test_silu_closed_forms_and_identities(rng):
    """silu(0) = 0; silu(g) -> g for large g and -> 0 (from below) for very
    negative g; silu(g) - silu(-g) = g (the odd part of g * sigmoid(g));
    within 4 ulp of g * sigmoid(g) evaluated in f64 (exp, add and divide
    each round)."""
    assert O.silu(np.float32(0.0)) == 0.0
    big = np.array([30.0, 60.0, 88.0], np.float32)
    np.testing.assert_array_equal(O.silu(big), big)
    tiny = O.silu(np.array([-100.0, -200.0], np.float32))
    assert np.all(tiny <= 0) and np.all(tiny > -1e-30)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    odd = O.silu(g).astype(np.float64) - O.silu(-g).astype(np.float64)
    assert np.all(np.abs(odd - g) <= 2e-6 * np.maximum(1.0, np.abs(g)))
    exact = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(O.silu(g) - exact) <= 4 * ulp + 1e-45)
    up = rng.standard_normal(4096).astype(np.float32)
    np.testing.assert_array_equal(O.silu_gate(g, up), (O.silu(g) * up).astype(np.float32))


# ---- decode-step ops (rms_norm, softmax, index_select) ----

def test_rms_norm_closed_forms(rng):
    """A constant row c maps to c / sqrt(c^2 + eps); the result is invariant
    to scaling the row (up to eps); its mean square is ms / (ms + eps); bf16
    inputs are widened exactly and the result rounded once."""
    c = np.full((2, 64), 3.0, np.float32)
    np.testing.assert_allclose(O.rms_norm(c), 3.0 / np.sqrt(9.0 + 1e-5), rtol=1e-7)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    np.testing.assert_allclose(O.rms_norm(x * 8, 0.0), O.rms_norm(x, 0.0), rtol=2e-7)
    y = O.rms_norm(x).astype(np.float64)
    ms = (x.astype(np.float64) ** 2).mean(axis=1)
    np.testing.assert_allclose((y ** 2).mean(axis=1), ms / (ms + 1e-5), rtol=1e-6)
    xb = O.bf16_from_f32(x)
    assert O.rms_norm(xb).dtype == np.uint16
    np.testing.assert_array_equal(O.rms_norm(xb), O.bf16_from_f32(O.rms_norm(O.f32_from_bf16(xb))))


def test_softmax_closed_forms(rng):
    """Rows sum to 1; adding a constant changes nothing; a constant row is
    uniform; [0, ln 3] gives [1/4, 3/4]; inputs near 1000 do not overflow."""
    x = (rng.standard_normal((5, 320)) * 3).astype(np.float32)
    y = O.softmax(x).astype(np.float64)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(O.softmax(x + np.float32(5.0)), O.softmax(x), rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(O.softmax(np.zeros((1, 7), np.float32)), 1 / 7, rtol=1e-7)
    np.testing.assert_allclose(O.softmax(np.array([[0.0, np.log(3.0)]], np.float32)), [[0.25, 0.75]], rtol=1e-7)
    big = O.softmax(np.array([[1000.0, 1000.0, 999.0]], np.float32))
    assert np.all(np.isfinite(big)) and abs(float(big.sum()) - 1.0) < 1e-6


def test_index_select_permutations_and_zero_fill(rng):
    x = rng.standard_normal((6, 5)).astype(np.float32)
    np.testing.assert_array_equal(O.index_select(x, 0, np.arange(6)), x)
    np.testing.assert_array_equal(O.index_select(x, 0, np.arange(5, -1, -1)), x[::-1])
    picked = O.index_select(x, 0, np.array([2, 6, -1, 0]))
    np.testing.assert_array_equal(picked[[0, 3]], x[[2, 0]])
    assert not picked[[1, 2]].any()
    cols = np.array([4, 0, 9, 1])
    np.testing.assert_array_equal(O.index_select(x, 1, cols), O.index_select(np.ascontiguousarray(x.T), 0, cols).T)
    xb = O.bf16_from_f32(x)
    np.testing.assert_array_equal(O.index_select(xb, 1, cols)[:, 0], xb[:, 4])


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_cpu_baseline_loop_is_bit_identical_to_oracle(bits, rng):
    """The timed CPU baseline (specialised per bit width and dtype pair) runs
    the oracle's rounding sequence, so its outputs are the oracle's bit for
    bit: every dtype pair, power-of-two and odd groups, a group that crosses
    words, and an N sub-range."""
    per_word = 32 // bits
    for x_dtype in ("f32", "bf16"):
        for p_dtype in ("f32", "bf16"):
            for M, K, N, group in ((1, 256, 9, 64), (3, per_word * 12, 7, 3 * per_word), (2, per_word * 6, 5, 3)):
                if K % group:
                    continue
                x = storage(rng.standard_normal((M, K)), x_dtype)
                q = rng.integers(0, 1 << bits, size=(N, K))
                s = storage(rng.random((N, K // group)) / 16, p_dtype)
                b = storage(rng.random((N, K // group)) - 0.5, p_dtype)
                packed = pack_codes(q, bits)
                want = O.quantized_matmul(x, packed, s, b, bits, group)
                got = O.baseline_quantized_matmul(x, packed, s, b, bits, group)
                np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
                part = O.baseline_quantized_matmul(x, packed, s, b, bits, group, n_range=(2, 4))
                np.testing.assert_array_equal(part[:, 2:4].view(np.uint32), want[:, 2:4].view(np.uint32))
                assert not part[:, :2].any() and not part[:, 4:].any()
