"""The reassociated prefill GEMM (gemm_re.hip): what the default policy runs
for tall bf16 activations with 4-bit weights, bf16 scales and biases and
groups of 64 or 128 (implementation rocm_quantized_matmul.gemv_mfma).

Two kinds of check, both against f64 products computed here:
  * exact -- integer activations and codes, power-of-two scales and integer
    biases keep every partial sum exact in f32, so the output must equal the
    f64 product bit for bit: partial row and column tiles, one or several K
    ranges, K ranges whose group count is not a multiple of 16 (a partial
    chunk of the bias term), and a K range count raised because one range
    would hold more than 64 groups;
  * reassociated accuracy -- seeded random inputs, per element
    |y - y64| <= 2^-18 * sum_k |x_k * w_k| with w = s*q + b in f64: f32
    accumulation of unrounded products. Rounding the decoded weights to bf16
    (the approximate class) violates that bound; the test shows so on the
    approximate GEMM with the same inputs, so the bound separates the classes.
"""
import numpy as np
import pytest

import affon_amd as A
from tests.helpers import pack_codes, storage, unpack_bytes_le, widened
from tests.test_gpu_parity import dtype_of, seeded_problem, upload

pytestmark = pytest.mark.gpu

GEMV_MFMA = "rocm_quantized_matmul.gemv_mfma"


def exact_operands(rng, M, N, K, group):
    q = rng.integers(0, 16, size=(N, K))
    x = rng.integers(-3, 4, size=(M, K)).astype(np.float64)
    s = 2.0 ** rng.integers(-3, 1, size=(N, K // group))
    b = rng.integers(-2, 3, size=(N, K // group)).astype(np.float64)
    return x, q, s, b


def product_f64(x, q, s, b, group, cols):
    w = q[cols] * np.repeat(s[cols], group, axis=1) + np.repeat(b[cols], group, axis=1)
    return x @ w.T


# (M, N, K, group): a half row tile and a partial column tile over eight K
# ranges of 16 steps; partial tiles over eight ranges of 16 groups; seven
# ranges of 8 groups (half a bias-term chunk); the full-size down projection
# (four ranges of 56 groups); the full-size gate/up projection (one range of
# 64 groups); eight ranges of 32 and of 16 groups; two ranges where the tile
# count alone would take one range of 128 groups.
EXACT_SHAPES = [
    (128, 200, 8192, 64),
    (300, 130, 16384, 128),
    (200, 300, 7168, 128),
    (512, 4096, 14336, 64),
    (512, 14336, 4096, 64),
    (256, 384, 16384, 64),
    (256, 256, 16384, 128),
    (1024, 6144, 8192, 64),
]


@pytest.mark.parametrize("shape", EXACT_SHAPES, ids=lambda s: "m{}_n{}_k{}_g{}".format(*s))
def test_reassociated_prefill_exact(session, shape, rng):
    M, N, K, group = shape
    x, q, s, b = exact_operands(rng, M, N, K, group)
    xt = upload(session, storage(x, "bf16"), "bf16")
    wt = upload(session, pack_codes(q, 4), "u32")
    st, bt = upload(session, storage(s, "bf16"), "bf16"), upload(session, storage(b, "bf16"), "bf16")
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=group) == GEMV_MFMA
    out = A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=group).numpy()
    cols = np.unique(np.concatenate([np.arange(min(N, 160)), np.linspace(0, N - 1, 96).astype(int)]))
    np.testing.assert_array_equal(out[:, cols], product_f64(x, q, s, b, group, cols).astype(np.float32),
                                  err_msg=f"{shape}")


def accuracy_ratio(out, x, packed, s, b, group, cols):
    """max over elements of |out - y64| / sum_k |x_k w_k|."""
    xf = widened(x)
    q = unpack_bytes_le(packed, 4)[cols].astype(np.float64)
    w = q * np.repeat(widened(s)[cols], group, axis=1) + np.repeat(widened(b)[cols], group, axis=1)
    y64 = xf @ w.T
    mag = np.abs(xf) @ np.abs(w).T
    return float(np.max(np.abs(out[:, cols].astype(np.float64) - y64) / mag))


@pytest.mark.parametrize("M,N,K,group", [(512, 1024, 4096, 64), (300, 640, 8192, 128), (512, 4096, 14336, 64)])
def test_reassociated_prefill_accuracy(session, M, N, K, group):
    x, packed, s, b = seeded_problem(M, N, K, 4, group, "bf16", "bf16", seed=17)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=group) == GEMV_MFMA
    cols = np.unique(np.linspace(0, N - 1, 256).astype(int))
    out = A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=group).numpy()
    bound = 2.0 ** -18
    ratio = accuracy_ratio(out, x, packed, s, b, group, cols)
    assert ratio <= bound, f"reassociated: worst error {ratio:.3g} of sum|x*w| (bound {bound:.3g})"
    approx = session.empty("f32", (M, N))
    A.quantized_matmul_into(approx, xt, wt, st, bt, bits=4, group_size=group, implementation="mfma",
                            policy="approximate")
    assert accuracy_ratio(approx.numpy(), x, packed, s, b, group, cols) > bound, \
        "the bound does not separate the classes"


def test_reassociated_prefill_deterministic(session):
    """Repeated runs (one and several K ranges) are bit-identical."""
    for M, N, K in ((512, 14336, 4096), (512, 4096, 14336)):
        x, packed, s, b = seeded_problem(M, N, K, 4, 64, "bf16", "bf16", seed=19)
        xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
        first = A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=64).numpy()
        for _ in range(2):
            np.testing.assert_array_equal(A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=64).numpy(), first)


def test_reassociated_prefill_epilogues_one_range(session, rng):
    """Output bias (f32 and bf16) and the SiLU-gated product stored by the
    kernel itself (one K range: 192 tiles of 256 x 128): the fused outputs
    against the plain outputs with the epilogue applied here (the bias add is
    the same f32 add, so bit-exact; silu(g) * u within 6 ulp of its f64
    value), and the plain output against f64 on a column subset."""
    M, N, K, group = 256, 24576, 1024, 128
    x, gp, gs, gb = seeded_problem(M, N, K, 4, group, "bf16", "bf16", seed=23)
    _, upk, us, ub = seeded_problem(M, N, K, 4, group, "bf16", "bf16", seed=29)
    xt = upload(session, x, "bf16")
    gate = tuple(upload(session, a, dtype_of(a)) for a in (gp, gs, gb))
    up = tuple(upload(session, a, dtype_of(a)) for a in (upk, us, ub))
    assert A.selected_implementation(xt, *gate, bits=4, group_size=group) == GEMV_MFMA
    g = A.quantized_matmul(xt, *gate, bits=4, group_size=group).numpy()
    u = A.quantized_matmul(xt, *up, bits=4, group_size=group).numpy()
    cols = np.unique(np.linspace(0, N - 1, 256).astype(int))
    assert accuracy_ratio(g, x, gp, gs, gb, group, cols) <= 2.0 ** -18
    for bias_dtype in ("f32", "bf16"):
        bias_values = rng.standard_normal(N).astype(np.float32)
        bias = storage(bias_values, "bf16") if bias_dtype == "bf16" else bias_values
        fused = A.quantized_linear(xt, *gate, upload(session, bias, bias_dtype), bits=4, group_size=group).numpy()
        np.testing.assert_array_equal(fused, (g + widened(bias).astype(np.float32)).astype(np.float32),
                                      err_msg=bias_dtype)
    fused = A.quantized_silu_gate(xt, gate, up, bits=4, group_size=group).numpy()
    g64 = g.astype(np.float64)
    with np.errstate(over="ignore"):
        expected = g64 / (1.0 + np.exp(-g64)) * u.astype(np.float64)
    bound = 6 * np.spacing(np.abs(expected).astype(np.float32)).astype(np.float64) + 1e-30
    err = np.abs(fused.astype(np.float64) - expected)
    assert np.all(err <= bound), f"worst {float(err.max())}"


# ---- the same kernel in the approximate class (implementation "mfma") ----------------

MFMA = "rocm_quantized_matmul.mfma"


@pytest.mark.parametrize("shape", EXACT_SHAPES, ids=lambda s: "m{}_n{}_k{}_g{}".format(*s))
def test_rounded_prefill_exact(session, shape, rng):
    """Under the approximate policy the kernel rounds each decoded weight
    s*q + b to bf16. Power-of-two scales, integer biases in [-2, 2] and codes
    below 16 keep every decoded weight exact in bf16 (multiples of 1/8 below
    18), so with integer activations the output must equal the f64 product."""
    M, N, K, group = shape
    x, q, s, b = exact_operands(rng, M, N, K, group)
    xt = upload(session, storage(x, "bf16"), "bf16")
    wt = upload(session, pack_codes(q, 4), "u32")
    st, bt = upload(session, storage(s, "bf16"), "bf16"), upload(session, storage(b, "bf16"), "bf16")
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=group, policy="approximate") == MFMA
    out = session.empty("f32", (M, N))
    A.quantized_matmul_into(out, xt, wt, st, bt, bits=4, group_size=group, implementation="mfma",
                            policy="approximate")
    cols = np.unique(np.concatenate([np.arange(min(N, 160)), np.linspace(0, N - 1, 96).astype(int)]))
    np.testing.assert_array_equal(out.numpy()[:, cols], product_f64(x, q, s, b, group, cols).astype(np.float32),
                                  err_msg=f"{shape}")


@pytest.mark.parametrize("M,N,K,group", [(512, 1024, 4096, 64), (300, 640, 8192, 128)])
def test_rounded_prefill_against_oracle_and_default(session, M, N, K, group):
    """Seeded inputs: the approximate policy's output within the bf16-product
    tolerance of the oracle (rtol 1e-2, atol 1e-2 * rms) and of the default
    policy's output on every element."""
    from tests.helpers import assert_bf16_product_close, oracle_columns
    x, packed, s, b = seeded_problem(M, N, K, 4, group, "bf16", "bf16", seed=31)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    approx = session.empty("f32", (M, N))
    A.quantized_matmul_into(approx, xt, wt, st, bt, bits=4, group_size=group, policy="approximate")
    default = A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=group).numpy()
    cols = np.unique(np.linspace(0, N - 1, 256).astype(int))
    assert_bf16_product_close(approx.numpy()[:, cols], oracle_columns(x, packed, s, b, 4, group, cols))
    assert_bf16_product_close(approx.numpy(), default)
