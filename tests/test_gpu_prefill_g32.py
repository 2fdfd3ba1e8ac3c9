"""The reassociated prefill GEMM for groups of 32 (gemm_re32.hip): what the
default policy runs for tall bf16 activations with 4-bit weights, bf16 scales
and biases and groups of 32 (implementation rocm_quantized_matmul.gemv_mfma).

Checks against f64 products computed here:
  * exact -- integer activations in {-1, 0, 1}, codes below 16, scales with
    full 8-bit bf16 significands (m / 64, m in [128, 255], so s * sum(x*q)
    needs up to 17 significant bits) and integer biases: every partial sum is
    a multiple of 2^-6 below 2^17, exact in f32, so the output must equal the
    f64 product bit for bit. Shapes cover partial row and column tiles, one
    and several K ranges, bias-term rounds of 64 groups (one partial, several
    with a partial last one) and K = 2 mod 4 steps (a last packed-word run of
    two steps);
  * reassociated accuracy -- seeded random inputs, per element
    |y - y64| <= 2^-18 * sum_k |x_k * w_k| with w = s*q + b in f64; the
    approximate GEMM on the same inputs violates the bound;
  * the fused output-bias and SiLU-gate epilogues, repeat determinism, and
    both orientations of the 2048-row stress shape on sampled columns
    including the first and last column tiles, against f64;
  * the same kernel's approximate form (decoded weights rounded to bf16,
    the approximate policy's path past 128 rows): bit-exact where every
    decoded weight is exact in bf16, within the bf16-product tolerance of
    the oracle and of the default policy on seeded inputs, repeat
    determinism, and its output-bias and SiLU-gate epilogues;
  * both forms captured into a HIP graph and replayed, bit-identical to the
    eager results.
"""
import numpy as np
import pytest

import affon_amd as A
from oracle import oracle as O
from tests.helpers import pack_codes, storage, widened
from tests.test_gpu_parity import dtype_of, seeded_problem, upload
from tests.test_gpu_prefill_reassociated import accuracy_ratio, product_f64

pytestmark = pytest.mark.gpu

GEMV_MFMA = "rocm_quantized_matmul.gemv_mfma"


def exact_operands(rng, M, N, K, group=32):
    q = rng.integers(0, 16, size=(N, K))
    x = rng.integers(-1, 2, size=(M, K)).astype(np.float64)
    s = rng.integers(128, 256, size=(N, K // group)) / 64.0 * rng.choice([-1.0, 1.0], size=(N, K // group))
    b = rng.integers(-2, 3, size=(N, K // group)).astype(np.float64)
    return x, q, s, b


def run_default(session, x, q, s, b, group=32):
    xt = upload(session, storage(x, "bf16"), "bf16")
    wt = upload(session, pack_codes(q, 4), "u32")
    st, bt = upload(session, storage(s, "bf16"), "bf16"), upload(session, storage(b, "bf16"), "bf16")
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=group) == GEMV_MFMA
    return A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=group).numpy()


# (M, N, K): one row tile and 16 column tiles (four K ranges); partial row
# and column tiles (eight K ranges); 5 row tiles (the last partial) x 2
# column tiles over one range of 24 groups (a partial bias-term round); short
# batches past the virtual-row kernels (M = 5, 64) with a partial column tile;
# K = 1152 and 4224 (18 and 66 steps: one range whose last packed-word run
# holds two steps; 36 and 132 groups: one and three bias-term rounds, the
# last partial).
EXACT_SHAPES = [(256, 2048, 2048), (300, 200, 4096), (1100, 256, 768), (5, 384, 2048), (64, 130, 2048),
                (130, 200, 1152), (600, 300, 4224)]


@pytest.mark.parametrize("shape", EXACT_SHAPES, ids=lambda s: "m{}_n{}_k{}".format(*s))
def test_g32_prefill_exact(session, shape, rng):
    M, N, K = shape
    x, q, s, b = exact_operands(rng, M, N, K)
    out = run_default(session, x, q, s, b)
    cols = np.unique(np.concatenate([np.arange(min(N, 160)), np.linspace(0, N - 1, 96).astype(int)]))
    np.testing.assert_array_equal(out[:, cols], product_f64(x, q, s, b, 32, cols).astype(np.float32),
                                  err_msg=f"{shape}")


def test_g32_single_products_are_exact(session, rng):
    """One nonzero activation per row picks single products x * s * q: each
    output equals s*q exactly (biases zero), which fails if the code or the
    scale of the picked k's group is wrong or s*q is rounded to bf16."""
    M, N, K = 256, 256, 1024
    _, q, s, b = exact_operands(rng, M, N, K)
    b[:] = 0.0
    x = np.zeros((M, K))
    picks = rng.integers(0, K, size=M)
    x[np.arange(M), picks] = 1.0
    out = run_default(session, x, q, s, b)
    expected = (q[:, picks] * s[:, picks // 32]).T.astype(np.float32)
    np.testing.assert_array_equal(out, expected)
    # the products need more than bf16's 8 significant bits
    assert (widened(storage(expected, "bf16")) != expected).any()


@pytest.mark.parametrize("M,N,K", [(512, 1024, 4096), (300, 640, 8192)])
def test_g32_prefill_accuracy(session, M, N, K):
    x, packed, s, b = seeded_problem(M, N, K, 4, 32, "bf16", "bf16", seed=37)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=32) == GEMV_MFMA
    cols = np.unique(np.linspace(0, N - 1, 256).astype(int))
    out = A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=32).numpy()
    bound = 2.0 ** -18
    ratio = accuracy_ratio(out, x, packed, s, b, 32, cols)
    assert ratio <= bound, f"reassociated: worst error {ratio:.3g} of sum|x*w| (bound {bound:.3g})"
    approx = session.empty("f32", (M, N))
    A.quantized_matmul_into(approx, xt, wt, st, bt, bits=4, group_size=32, implementation="mfma",
                            policy="approximate")
    assert accuracy_ratio(approx.numpy(), x, packed, s, b, 32, cols) > bound, "the bound does not separate the classes"


def test_g32_prefill_deterministic(session):
    """Repeated runs (one and several K ranges) are bit-identical."""
    for M, N, K in ((512, 2048, 2048), (512, 256, 8192)):
        x, packed, s, b = seeded_problem(M, N, K, 4, 32, "bf16", "bf16", seed=41)
        xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
        first = A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=32).numpy()
        for _ in range(2):
            np.testing.assert_array_equal(A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=32).numpy(), first)


def test_g32_prefill_epilogues(session, rng):
    """Output bias (f32, bf16) and the SiLU-gated product stored by the kernel
    (one K range): bias bit-exact against plain + the same f32 add, the gate
    within 6 ulp of silu(g) * u in f64."""
    M, N, K = 256, 8192, 1024
    x, gp, gs, gb = seeded_problem(M, N, K, 4, 32, "bf16", "bf16", seed=43)
    _, upk, us, ub = seeded_problem(M, N, K, 4, 32, "bf16", "bf16", seed=47)
    xt = upload(session, x, "bf16")
    gate = tuple(upload(session, a, dtype_of(a)) for a in (gp, gs, gb))
    up = tuple(upload(session, a, dtype_of(a)) for a in (upk, us, ub))
    g = A.quantized_matmul(xt, *gate, bits=4, group_size=32).numpy()
    u = A.quantized_matmul(xt, *up, bits=4, group_size=32).numpy()
    for bias_dtype in ("f32", "bf16"):
        bias_values = rng.standard_normal(N).astype(np.float32)
        bias = storage(bias_values, "bf16") if bias_dtype == "bf16" else bias_values
        fused = A.quantized_linear(xt, *gate, upload(session, bias, bias_dtype), bits=4, group_size=32).numpy()
        np.testing.assert_array_equal(fused, (g + widened(bias).astype(np.float32)).astype(np.float32),
                                      err_msg=bias_dtype)
    fused = A.quantized_silu_gate(xt, gate, up, bits=4, group_size=32).numpy()
    g64 = g.astype(np.float64)
    with np.errstate(over="ignore"):
        expected = g64 / (1.0 + np.exp(-g64)) * u.astype(np.float64)
    bound = 6 * np.spacing(np.abs(expected).astype(np.float32)).astype(np.float64) + 1e-30
    err = np.abs(fused.astype(np.float64) - expected)
    assert np.all(err <= bound), f"worst {float(err.max())}"


def test_g32_prefill_stress_full_size(session):
    """The 2048-row stress configuration under the default policy, both
    orientations: W f32 [28672, 8192] N(0, 0.02) (the same values reshaped to
    [8192, 28672] for the second) quantized on the GPU at 4 bits, group 32,
    bf16 parameters; x bf16 [2048, 8192] N(0, 1), its rows repeated to 28672
    columns for the second orientation. Every row of 112 sampled columns (the
    first and last column tiles among them) against f64 within the
    reassociated bound."""
    M = 2048
    wf, _ = O.randn(2, 28672 * 8192, 0.0, 0.02)
    _, xb = O.randn(1, M * 8192, 0.0, 1.0)
    x8 = xb.reshape(M, 8192)
    for N, K in ((28672, 8192), (8192, 28672)):
        packed, scales, biases = A.quantize(upload(session, wf.reshape(N, K), "f32"), bits=4, group_size=32,
                                            param_dtype="bf16")
        x = x8 if K == 8192 else np.ascontiguousarray(np.tile(x8, (1, -(-K // 8192)))[:, :K])
        xt = upload(session, x, "bf16")
        assert A.selected_implementation(xt, packed, scales, biases, bits=4, group_size=32) == GEMV_MFMA
        out = A.quantized_matmul(xt, packed, scales, biases, bits=4, group_size=32).numpy()
        cols = np.unique(np.concatenate([np.arange(16), np.linspace(0, N - 1, 80).astype(int), np.arange(N - 16, N)]))
        ratio = accuracy_ratio(out, xt.storage(), packed.storage(), scales.storage(), biases.storage(), 32, cols)
        assert ratio <= 2.0 ** -18, f"{N}x{K}: worst error {ratio:.3g} of sum|x*w|"
        del packed, scales, biases, xt, out

# ---- the same kernel in the approximate class (implementation "mfma", past 128 rows) ----

MFMA = "rocm_quantized_matmul.mfma"

# (M, N, K): one row tile, 16 column tiles, four K ranges; partial row and
# column tiles, eight K ranges; 5 row tiles over one range; one range of 68
# steps (17 packed-word runs). The approximate candidate takes K in whole
# multiples of 256, so no last run of two steps occurs here.
ROUNDED_SHAPES = [(256, 2048, 2048), (300, 200, 4096), (1100, 256, 768), (600, 300, 4352)]


@pytest.mark.parametrize("shape", ROUNDED_SHAPES, ids=lambda s: "m{}_n{}_k{}".format(*s))
def test_g32_rounded_prefill_exact(session, shape, rng):
    """Under the approximate policy the kernel rounds each decoded weight
    s*q + b to bf16 (per group of 32). Power-of-two scales, integer biases in
    [-2, 2] and codes below 16 keep every decoded weight exact in bf16
    (multiples of 1/8 below 18), so with integer activations in [-3, 3] every
    partial sum is a multiple of 1/8 below 2^18 and the output must equal the
    f64 product bit for bit."""
    from tests.test_gpu_prefill_reassociated import exact_operands as rounded_operands
    M, N, K = shape
    x, q, s, b = rounded_operands(rng, M, N, K, 32)
    xt = upload(session, storage(x, "bf16"), "bf16")
    wt = upload(session, pack_codes(q, 4), "u32")
    st, bt = upload(session, storage(s, "bf16"), "bf16"), upload(session, storage(b, "bf16"), "bf16")
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=32, policy="approximate") == MFMA
    out = session.empty("f32", (M, N))
    A.quantized_matmul_into(out, xt, wt, st, bt, bits=4, group_size=32, implementation="mfma",
                            policy="approximate")
    cols = np.unique(np.concatenate([np.arange(min(N, 160)), np.linspace(0, N - 1, 96).astype(int)]))
    np.testing.assert_array_equal(out.numpy()[:, cols], product_f64(x, q, s, b, 32, cols).astype(np.float32),
                                  err_msg=f"{shape}")


@pytest.mark.parametrize("M,N,K", [(512, 1024, 4096), (300, 640, 8192)])
def test_g32_rounded_prefill_against_oracle_and_default(session, M, N, K):
    """Seeded inputs: the approximate policy's output within the bf16-product
    tolerance of the oracle (rtol 1e-2, atol 1e-2 * rms) and of the default
    policy's output on every element; a second run is bit-identical."""
    from tests.helpers import assert_bf16_product_close, oracle_columns
    x, packed, s, b = seeded_problem(M, N, K, 4, 32, "bf16", "bf16", seed=53)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    assert A.selected_implementation(xt, wt, st, bt, bits=4, group_size=32, policy="approximate") == MFMA
    approx = session.empty("f32", (M, N))
    A.quantized_matmul_into(approx, xt, wt, st, bt, bits=4, group_size=32, policy="approximate")
    again = session.empty("f32", (M, N))
    A.quantized_matmul_into(again, xt, wt, st, bt, bits=4, group_size=32, policy="approximate")
    np.testing.assert_array_equal(again.numpy(), approx.numpy())
    default = A.quantized_matmul(xt, wt, st, bt, bits=4, group_size=32).numpy()
    cols = np.unique(np.linspace(0, N - 1, 256).astype(int))
    assert_bf16_product_close(approx.numpy()[:, cols], oracle_columns(x, packed, s, b, 4, 32, cols))
    assert_bf16_product_close(approx.numpy(), default)


def test_g32_rounded_prefill_epilogues(session, rng):
    """The rounded form's output bias (f32, bf16) and SiLU-gated product under
    the approximate policy, eight K ranges (the reduction applies them): the
    bias bit-exact against the plain product plus the same f32 add, the gate
    within 6 ulp of silu(g) * u in f64."""
    M, N, K = 512, 1024, 4096
    x, gp, gs, gb = seeded_problem(M, N, K, 4, 32, "bf16", "bf16", seed=59)
    _, upk, us, ub = seeded_problem(M, N, K, 4, 32, "bf16", "bf16", seed=61)
    xt = upload(session, x, "bf16")
    gate = tuple(upload(session, a, dtype_of(a)) for a in (gp, gs, gb))
    up = tuple(upload(session, a, dtype_of(a)) for a in (upk, us, ub))
    assert A.selected_implementation(xt, *gate, bits=4, group_size=32, policy="approximate") == MFMA
    g = session.empty("f32", (M, N))
    A.quantized_matmul_into(g, xt, *gate, bits=4, group_size=32, policy="approximate")
    u = session.empty("f32", (M, N))
    A.quantized_matmul_into(u, xt, *up, bits=4, group_size=32, policy="approximate")
    g, u = g.numpy(), u.numpy()
    for bias_dtype in ("f32", "bf16"):
        bias_values = rng.standard_normal(N).astype(np.float32)
        bias = storage(bias_values, "bf16") if bias_dtype == "bf16" else bias_values
        fused = A.quantized_linear(xt, *gate, upload(session, bias, bias_dtype), bits=4, group_size=32,
                                   policy="approximate").numpy()
        np.testing.assert_array_equal(fused, (g + widened(bias).astype(np.float32)).astype(np.float32),
                                      err_msg=bias_dtype)
    fused = A.quantized_silu_gate(xt, gate, up, bits=4, group_size=32, policy="approximate").numpy()
    g64 = g.astype(np.float64)
    with np.errstate(over="ignore"):
        expected = g64 / (1.0 + np.exp(-g64)) * u.astype(np.float64)
    bound = 6 * np.spacing(np.abs(expected).astype(np.float32)).astype(np.float64) + 1e-30
    err = np.abs(fused.astype(np.float64) - expected)
    assert np.all(err <= bound), f"worst {float(err.max())}"


def test_g32_graph_replay(session):
    """Both forms of the group-32 GEMM (the default policy's exact codes with
    its group-sum pre-pass, the approximate policy's rounded weights, each
    over eight K ranges and the reduction) captured into one HIP graph on
    the session stream, after eager calls sized the workspace, and replayed
    three times. Between replays an eager call of another shape leaves other
    contents in the workspace and the outputs are cleared; every replay
    reproduces the eager results bit for bit."""
    import ctypes

    from affon_amd import _native, ops
    from tests.helpers import HipRuntime
    hip = HipRuntime()
    lib = _native.load()
    # Each descriptor holds raw device pointers: its operands stay referenced
    # here for as long as the descriptor (and the graph) is used.
    calls = []
    for (M, N, K), policy in (((512, 1024, 4096), "backend_equivalent"), ((300, 640, 8192), "approximate")):
        x, packed, s, b = seeded_problem(M, N, K, 4, 32, "bf16", "bf16", seed=M + 3)
        operands = tuple(upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
        out = session.tensor(np.full((M, N), 7.0, np.float32))
        desc = ops._descriptor(*operands, 4, 32, out, "auto", policy)
        calls.append((desc, out, operands))
    eager = []
    for desc, out, _ in calls:
        assert lib.affon_rocm_quantized_matmul(session._handle, ctypes.byref(desc)) == 0, _native.last_error()
        session.synchronize()
        eager.append(out.numpy().copy())

    def enqueue():
        for desc, _, _ in calls:
            assert lib.affon_rocm_quantized_matmul(session._handle, ctypes.byref(desc)) == 0, _native.last_error()

    graph = hip.capture(session.stream, enqueue)
    try:
        ox, op, osc, ob = seeded_problem(256, 512, 4096, 4, 32, "bf16", "bf16", seed=71)
        other = tuple(upload(session, a, dtype_of(a)) for a in (ox, op, osc, ob))
        for i in range(3):
            A.quantized_matmul(*other, bits=4, group_size=32)
            for _, out, _ in calls:
                zeros = np.zeros(out.shape, np.float32)
                _native.check(lib.affon_rocm_memcpy_h2d(session._handle, out.data_ptr, zeros.ctypes.data,
                                                        zeros.nbytes), "clear")
            session.synchronize()
            hip.replay(session.stream, graph)
            for (_, out, _), want in zip(calls, eager):
                np.testing.assert_array_equal(out.numpy().view(np.uint32), want.view(np.uint32),
                                              err_msg=f"replay {i}, output {out.shape}")
    finally:
        hip.destroy(graph)
