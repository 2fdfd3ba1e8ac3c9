"""Size-independent properties of every quantized_matmul implementation at the
workloads' full sizes, where the CPU oracle would take minutes.

All checks are bit-exact, because each follows from arithmetic that is exact
in f32 and bf16:
* doubling the activations doubles every product and every partial sum, so
  the output doubles exactly (bf16 and f32 scale by 2 without rounding);
* doubling the scales and the biases doubles every decoded weight (also when
  the prefill kernel rounds decoded weights to bf16), so again the output
  doubles;
* permuting the activation rows permutes the output rows: each output row's
  arithmetic does not depend on where the row sits in a tile;
* two runs of the same call give the same bits (ordered reductions, split-K
  included).
"""
import numpy as np
import pytest

import affon_amd as A
from affon_amd import _native
from oracle import oracle as O
from tests.test_gpu_parity import IMPLS, upload

pytestmark = pytest.mark.gpu

# (name, M, N, K, bits, group): the decode sweep, the north-star decode row,
# the prefill GEMM (both orientations) and the large prefill stress shape.
SHAPES = [
    ("decode_8bit_m1", 1, 14336, 4096, 8, 64),
    ("decode_8bit_m4", 4, 14336, 4096, 8, 64),
    ("decode_8bit_m16", 16, 14336, 4096, 8, 64),
    ("decode_4bit_m1", 1, 14336, 4096, 4, 64),
    ("decode_4bit_m32_down", 32, 4096, 14336, 4, 64),
    ("prefill_512x14336x4096", 512, 14336, 4096, 4, 64),
    ("prefill_512x4096x14336", 512, 4096, 14336, 4, 64),
    ("prefill_2048x28672x8192_g32", 2048, 28672, 8192, 4, 32),
]


def quantized(session, N, K, bits, group, seed):
    w = session.randn((N, K), seed=seed, std=0.02, dtype="bf16")
    return A.quantize(w, bits=bits, group_size=group, param_dtype="bf16")


def doubled(session, t: A.Tensor) -> A.Tensor:
    """2*t for a bf16 tensor, exactly (one more exponent step)."""
    values = O.f32_from_bf16(t.storage()).astype(np.float32) * np.float32(2.0)
    return upload(session, O.bf16_from_f32(values), "bf16")


def candidates(x, w, s, b, bits, group, M):
    out = []
    for impl in IMPLS[1:]:
        if impl == "generic" and M * w.shape[0] > 4 * 14336:
            continue  # one thread per output with a K-long loop: minutes at these sizes
        policy = "approximate" if impl == "mfma" else "backend_equivalent"
        try:
            A.selected_implementation(x, w, s, b, bits=bits, group_size=group, implementation=impl, policy=policy)
        except _native.NativeError as error:
            assert error.status == _native.UNSUPPORTED, str(error)
            continue
        out.append((impl, policy))
    return out


def run(session, x, w, s, b, bits, group, impl, policy):
    out = session.empty("f32", (x.shape[0], w.shape[0]))
    A.quantized_matmul_into(out, x, w, s, b, bits=bits, group_size=group, implementation=impl, policy=policy)
    return out.numpy()


@pytest.mark.parametrize("name,M,N,K,bits,group", SHAPES, ids=[s[0] for s in SHAPES])
def test_exact_homogeneity_permutation_and_determinism(session, name, M, N, K, bits, group):
    x = session.randn((M, K), seed=1, dtype="bf16")
    w, s, b = quantized(session, N, K, bits, group, seed=2)
    x2, s2, b2 = doubled(session, x), doubled(session, s), doubled(session, b)
    perm = np.random.default_rng(M).permutation(M)
    xp = upload(session, np.ascontiguousarray(x.storage()[perm]), "bf16")
    impls = candidates(x, w, s, b, bits, group, M)
    assert impls, name
    for impl, policy in impls:
        y = run(session, x, w, s, b, bits, group, impl, policy)
        assert np.isfinite(y).all(), (name, impl)
        np.testing.assert_array_equal(run(session, x, w, s, b, bits, group, impl, policy), y, err_msg=f"{impl} rerun")
        np.testing.assert_array_equal(run(session, x2, w, s, b, bits, group, impl, policy), 2 * y,
                                      err_msg=f"{impl} 2x")
        np.testing.assert_array_equal(run(session, x, w, s2, b2, bits, group, impl, policy), 2 * y,
                                      err_msg=f"{impl} 2(s, b)")
        if M > 1:
            np.testing.assert_array_equal(run(session, xp, w, s, b, bits, group, impl, policy), y[perm],
                                          err_msg=f"{impl} row permutation")
