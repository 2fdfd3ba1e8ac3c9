"""GPU parity of the fused output epilogues (the output-bias add and the
SiLU-gated product of two projections, applied by the kernel that stores the
output) and of grouped projections of one input, against the same kernels'
plain outputs and the CPU oracle.

Tolerances (stated per test): the bias epilogue must be bit-identical to the
plain kernel's output followed by one f32 add; the two-launch SiLU gate must be
within 4 ulp of f32 silu(gate) * up formed on the host from the plain kernels'
outputs (the device and host exponentials may differ in the last place); the
bias output must be within the matmul tolerance of the oracle (rtol 2e-3 /
atol 1e-4 for f32 activations, rtol 1e-2 / atol 1e-2*rms for bf16). For the
SiLU gate that tolerance t_g, t_u of each projection (the oracle's gate and up
are its ordered quantized_matmul loops) is carried through the product:
|error| <= 1.1*t_g*|u| + |silu(g)|*t_u + 1.1*t_g*t_u + 4 ulp, with
1.1 >= max |silu'|.
"""
import ctypes

import numpy as np
import pytest

import affon_amd as A
from affon_amd import _native
from oracle import oracle as O
from tests.helpers import assert_close_rtol_atol
from tests.test_gpu_parity import IMPLS, dtype_of, seeded_problem, upload

pytestmark = pytest.mark.gpu

# (M, N, K, bits, group, x_dtype, p_dtype): decode (M=1 kernel, virtual-row
# and LDS-tiled decode kernels, the general VALU kernel), prefill (one K range
# and split K), and an f32 case.
CASES = [
    (1, 300, 512, 4, 64, "bf16", "bf16"),
    (1, 96, 4096, 8, 64, "f32", "f32"),
    (1, 200, 1024, 8, 32, "bf16", "bf16"),  # M=1 kernel, parameters loaded per lane (groups of 2 chunks)
    (1, 136, 2048, 4, 32, "bf16", "bf16"),  # M=1 kernel, one chunk per group
    (2, 136, 1024, 8, 64, "bf16", "bf16"),
    (4, 72, 512, 4, 32, "bf16", "f32"),
    (16, 128, 1024, 4, 64, "bf16", "bf16"),
    (8, 200, 2048, 4, 64, "bf16", "bf16"),  # LDS-tiled kernel with twin column tiles (split K)
    (6, 136, 4096, 8, 128, "bf16", "f32"),  # the same, 8-bit codes and f32 parameters
    (3, 77, 256, 2, 64, "f32", "bf16"),
    (64, 192, 512, 4, 64, "bf16", "bf16"),
    (96, 64, 4096, 8, 128, "bf16", "bf16"),
    (200, 136, 8192, 4, 64, "bf16", "bf16"),  # reassociated prefill GEMM, K split (epilogue in the reduction)
]


def accepted(x, w, s, b, bits, group):
    """Implementations (with the auto pick) that accept a problem, with the
    policy each needs."""
    out = []
    for impl in IMPLS:
        policy = "approximate" if impl == "mfma" else "backend_equivalent"
        try:
            A.selected_implementation(x, w, s, b, bits=bits, group_size=group, implementation=impl, policy=policy)
        except _native.NativeError as error:
            assert error.status == _native.UNSUPPORTED, str(error)
            continue
        out.append((impl, policy))
    return out


def plain(session, x, w, s, b, bits, group, impl, policy):
    out = session.empty("f32", (x.shape[0], w.shape[0]))
    A.quantized_matmul_into(out, x, w, s, b, bits=bits, group_size=group, implementation=impl, policy=policy)
    return out.numpy()


def oracle_close(actual, expected, bf16_input):
    if bf16_input:
        rms = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
        assert_close_rtol_atol(actual, expected, rtol=1e-2, atol=1e-2 * rms)
    else:
        assert_close_rtol_atol(actual, expected, rtol=2e-3, atol=1e-4)


def silu_gate_close(actual, g, u, bf16_input):
    """The matmul tolerance of gate and up, propagated through silu(g) * u."""
    g = g.astype(np.float64)
    u = u.astype(np.float64)
    if bf16_input:
        rtol, atol_g, atol_u = 1e-2, 1e-2 * np.sqrt(np.mean(g ** 2)), 1e-2 * np.sqrt(np.mean(u ** 2))
    else:
        rtol, atol_g, atol_u = 2e-3, 1e-4, 1e-4
    tg = atol_g + rtol * np.abs(g)
    tu = atol_u + rtol * np.abs(u)
    expected = O.silu_gate(g.astype(np.float32), u.astype(np.float32)).astype(np.float64)
    sg = np.abs(O.silu(g.astype(np.float32))).astype(np.float64)
    bound = 1.1 * tg * np.abs(u) + sg * tu + 1.1 * tg * tu + 4 * np.spacing(np.abs(expected).astype(np.float32))
    err = np.abs(actual.astype(np.float64) - expected)
    bad = err > bound
    assert not bad.any(), (f"{int(bad.sum())} of {err.size} out of tolerance; worst at "
                           f"{np.unravel_index(np.argmax(err - bound), err.shape)}")


def within_ulps(actual, expected, ulps):
    expected = np.asarray(expected, dtype=np.float64)
    bound = ulps * np.spacing(np.abs(expected).astype(np.float32)).astype(np.float64) + 1e-30
    err = np.abs(actual.astype(np.float64) - expected)
    assert np.all(err <= bound), f"worst {float(err.max())} at {np.unravel_index(np.argmax(err - bound), err.shape)}"


def silu_gate_f64(g, u):
    """silu(g) * u evaluated in f64 from the f32 projections: the fused
    epilogue's f32 steps (e^-g, 1 + e^-g, the division, the product) each
    round once, so it lies within a few f32 ulps of this."""
    g = g.astype(np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "m{}_n{}_k{}_b{}_g{}_{}_{}".format(*c))
@pytest.mark.parametrize("bias_dtype", ["f32", "bf16"])
def test_bias_epilogue_every_implementation(session, case, bias_dtype, rng):
    M, N, K, bits, group, x_dtype, p_dtype = case
    x, packed, s, b = seeded_problem(M, N, K, bits, group, x_dtype, p_dtype, seed=11)
    xt, wt, st, bt = (upload(session, a, dtype_of(a)) for a in (x, packed, s, b))
    bias_values = rng.standard_normal(N).astype(np.float32)
    bias = O.bf16_from_f32(bias_values) if bias_dtype == "bf16" else bias_values
    bias_t = upload(session, bias, bias_dtype)
    oracle = O.add_output_bias(O.quantized_matmul(x, packed, s, b, bits, group), bias)
    for impl, policy in accepted(xt, wt, st, bt, bits, group):
        plan = A.fused_plan(xt, wt, st, bt, bits=bits, group_size=group, output_bias=bias_t, implementation=impl,
                            policy=policy)
        assert plan.endswith("[bias]") and ";" not in plan, plan
        fused = A.quantized_linear(xt, wt, st, bt, bias_t, bits=bits, group_size=group, implementation=impl,
                                   policy=policy).numpy()
        expected = O.add_output_bias(plain(session, xt, wt, st, bt, bits, group, impl, policy), bias)
        np.testing.assert_array_equal(fused, expected, err_msg=f"{impl} {case}")
        oracle_close(fused, oracle, x_dtype == "bf16")


@pytest.mark.parametrize("case", CASES, ids=lambda c: "m{}_n{}_k{}_b{}_g{}_{}_{}".format(*c))
def test_silu_gate_epilogue_every_implementation(session, case):
    M, N, K, bits, group, x_dtype, p_dtype = case
    x, gp, gs, gb = seeded_problem(M, N, K, bits, group, x_dtype, p_dtype, seed=21)
    _, upk, us, ub = seeded_problem(M, N, K, bits, group, x_dtype, p_dtype, seed=31)
    xt = upload(session, x, dtype_of(x))
    gate = tuple(upload(session, a, dtype_of(a)) for a in (gp, gs, gb))
    up = tuple(upload(session, a, dtype_of(a)) for a in (upk, us, ub))
    g_oracle = O.quantized_matmul(x, gp, gs, gb, bits, group)
    u_oracle = O.quantized_matmul(x, upk, us, ub, bits, group)
    for impl, policy in accepted(xt, *gate, bits, group):
        plan = A.fused_plan(xt, *gate, bits=bits, group_size=group, up=up, implementation=impl, policy=policy)
        fused = A.quantized_silu_gate(xt, gate, up, bits=bits, group_size=group, implementation=impl,
                                      policy=policy).numpy()
        if plan.endswith("[silu_gate]"):
            # One launch computing both projections (rows paired in one wave):
            # the sums may be ordered differently from the plain kernel's.
            assert M == 1 and plan.startswith("rocm_quantized_matmul.gemv[") and ";" not in plan, plan
        else:
            assert plan.count(";") == 1 and plan.endswith("[gate_mul]"), plan
            g = plain(session, xt, *gate, bits, group, impl, policy)
            u = plain(session, xt, *up, bits, group, impl, policy)
            within_ulps(fused, silu_gate_f64(g, u), 6)
        silu_gate_close(fused, g_oracle, u_oracle, x_dtype == "bf16")


def test_silu_gate_single_launch_at_decode(session):
    """At M = 1 the auto pick pairs gate and up rows in one launch."""
    x, gp, gs, gb = seeded_problem(1, 256, 1024, 4, 64, "bf16", "bf16", seed=5)
    _, upk, us, ub = seeded_problem(1, 256, 1024, 4, 64, "bf16", "bf16", seed=6)
    xt = upload(session, x, "bf16")
    gate = tuple(upload(session, a, dtype_of(a)) for a in (gp, gs, gb))
    up = tuple(upload(session, a, dtype_of(a)) for a in (upk, us, ub))
    assert A.fused_plan(xt, *gate, bits=4, group_size=64, up=up) == "rocm_quantized_matmul.gemv[silu_gate]"
    # Strided up operands (a column slice of wider tensors) take two launches.
    wide = upload(session, np.concatenate([upk, upk], axis=1), "u32")
    up_view = (A.slice(wide, [{"start": 0, "stop": 256}, {"start": 0, "stop": upk.shape[1]}]), *up[1:])
    plan = A.fused_plan(xt, *gate, bits=4, group_size=64, up=up_view)
    assert plan == "rocm_quantized_matmul.gemv;rocm_quantized_matmul.gemv[gate_mul]", plan
    fused = A.quantized_silu_gate(xt, gate, up_view, bits=4, group_size=64).numpy()
    silu_gate_close(fused, O.quantized_matmul(x, gp, gs, gb, 4, 64), O.quantized_matmul(x, upk, us, ub, 4, 64), True)


@pytest.mark.parametrize("bits", [4, 8])
def test_silu_gate_llama_feed_forward_full_size(session, bits):
    """Llama-8B gate/up (14336x4096, group 64, bf16) at M = 1 (one paired
    launch) and M = 4 (two launches) against the oracle."""
    for M in (1, 4):
        x, gp, gs, gb = seeded_problem(M, 14336, 4096, bits, 64, "bf16", "bf16", seed=41)
        _, upk, us, ub = seeded_problem(M, 14336, 4096, bits, 64, "bf16", "bf16", seed=43)
        xt = upload(session, x, "bf16")
        gate = tuple(upload(session, a, dtype_of(a)) for a in (gp, gs, gb))
        up = tuple(upload(session, a, dtype_of(a)) for a in (upk, us, ub))
        fused = A.quantized_silu_gate(xt, gate, up, bits=bits, group_size=64).numpy()
        silu_gate_close(fused, O.quantized_matmul(x, gp, gs, gb, bits, 64), O.quantized_matmul(x, upk, us, ub, bits, 64),
                        True)


def test_epilogue_validation_leaves_output_untouched(session):
    """Malformed epilogues are rejected before any launch (status 1) and the
    output keeps its contents."""
    x, gp, gs, gb = seeded_problem(1, 64, 256, 4, 64, "bf16", "bf16", seed=7)
    xt = upload(session, x, "bf16")
    gate = [upload(session, a, dtype_of(a)) for a in (gp, gs, gb)]
    out = session.tensor(np.full((1, 64), 7.0, np.float32), dtype="f32")
    desc = A.ops._descriptor(xt, *gate, 4, 64, out, "auto", "backend_equivalent")
    lib = _native.load()

    def run(epi):
        return lib.affon_rocm_quantized_matmul_fused(session._handle, ctypes.byref(desc), ctypes.byref(epi))

    short_bias = upload(session, np.zeros(63, np.float32), "f32")
    epi = A.ops._epilogue(output_bias=short_bias)
    assert run(epi) == _native.INVALID_SHAPE and "bias" in _native.last_error()
    epi = A.ops._epilogue(up=(gate[0], gate[1], upload(session, np.zeros((64, 4), np.float32), "f32")))
    assert run(epi) == _native.INVALID_SHAPE and "up biases" in _native.last_error()
    epi = A.ops._epilogue()
    epi.kind = 9
    assert run(epi) == _native.INVALID_SHAPE and "epilogue" in _native.last_error()
    assert lib.affon_rocm_quantized_matmul_fused(session._handle, ctypes.byref(desc), None) == _native.INVALID_SHAPE
    session.synchronize()
    np.testing.assert_array_equal(out.numpy(), np.full((1, 64), 7.0, np.float32))


@pytest.mark.parametrize("x_dtype,p_dtype,bits,group", [("bf16", "bf16", 4, 64), ("f32", "f32", 8, 64),
                                                        ("bf16", "f32", 2, 64), ("bf16", "bf16", 4, 32),
                                                        ("bf16", "bf16", 8, 32)])
@pytest.mark.parametrize("sizes", [(4096, 1024, 1024), (300, 77, 13, 8)], ids=["qkv", "ragged"])
def test_grouped_projections_against_oracle(session, x_dtype, p_dtype, bits, group, sizes, rng):
    """Projections of one input in one launch (M = 1: the gemv kernel; M = 8
    and 16 with bf16 activations: the LDS-tiled gemv_mfma kernel, at 8 rows
    with twin column tiles, whose split-K partials span all projections) or
    in sequence (M = 2 on the virtual-row kernels; groups of 32 past M = 4 on
    the group-32 GEMM), with output biases on some of them; ragged sizes
    exercise the padding between projections. Group 32 at 4 and 8 bits takes
    the M=1 kernel's per-lane parameter loads."""
    K = 1024
    for M in (1, 2, 8, 16):
        projections, host = [], []
        x = seeded_problem(M, 8, K, bits, group, x_dtype, p_dtype, seed=59)[0]
        for i, n in enumerate(sizes):
            _, packed, s, b = seeded_problem(M, n, K, bits, group, x_dtype, p_dtype, seed=60 + 2 * i)
            parts = [upload(session, a, dtype_of(a)) for a in (packed, s, b)]
            bias = None
            if i % 2 == 0:
                bias = O.bf16_from_f32(rng.standard_normal(n).astype(np.float32))
                parts.append(upload(session, bias, "bf16"))
            projections.append(tuple(parts))
            host.append((packed, s, b, bias))
        xt = upload(session, x, dtype_of(x))
        plan = A.grouped_plan(xt, projections, bits=bits, group_size=group)
        # The tiled kernel (K steps of 64) takes M = 8, 16 and, for 8-bit codes, M = 2.
        tiled_m = (2, 8, 16) if bits == 8 else (8, 16)
        one_launch = M == 1 or (M in tiled_m and x_dtype == "bf16" and group % 64 == 0)
        if one_launch:
            kernel = "gemv" if M == 1 else "gemv_mfma"
            assert plan == f"rocm_quantized_matmul.{kernel}[grouped:{len(sizes)},bias]", plan
        else:
            assert plan.count(";") == len(sizes) - 1, plan
        outs = A.quantized_matmul_grouped(xt, projections, bits=bits, group_size=group)
        for out, (packed, s, b, bias), parts in zip(outs, host, projections):
            expected = O.quantized_matmul(x, packed, s, b, bits, group)
            single = A.quantized_matmul(xt, *parts[:3], bits=bits, group_size=group).numpy()
            if bias is not None:
                expected = O.add_output_bias(expected, bias)
                single = O.add_output_bias(single, bias)
            oracle_close(out.numpy(), expected, x_dtype == "bf16")
            if not one_launch:  # the same kernels one by one: identical results
                np.testing.assert_array_equal(out.numpy(), single)


def test_grouped_validation(session):
    x, packed, s, b = seeded_problem(1, 64, 256, 4, 64, "bf16", "bf16", seed=3)
    xt, x2 = upload(session, x, "bf16"), upload(session, x, "bf16")
    w = tuple(upload(session, a, dtype_of(a)) for a in (packed, s, b))
    descs = (_native.QmmDesc * 2)()
    descs[0] = A.ops._descriptor(xt, *w, 4, 64, session.empty("f32", (1, 64)), "auto", "backend_equivalent")
    descs[1] = A.ops._descriptor(x2, *w, 4, 64, session.empty("f32", (1, 64)), "auto", "backend_equivalent")
    lib = _native.load()
    assert lib.affon_rocm_quantized_matmul_grouped(session._handle, descs, None, 2) == _native.INVALID_SHAPE
    assert "share the input" in _native.last_error()
    assert lib.affon_rocm_quantized_matmul_grouped(session._handle, descs, None, 0) == _native.INVALID_SHAPE
    epis = (_native.Epilogue * 1)()
    epis[0] = A.ops._epilogue(up=w)
    assert lib.affon_rocm_quantized_matmul_grouped(session._handle, descs, epis, 1) == _native.INVALID_SHAPE
    assert "output bias" in _native.last_error()
