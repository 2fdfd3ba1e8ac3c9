"""GPU parity at the Llama-8B decoder shapes the bench times
(packages/@affon/models/src/llama/model.ts:75-87: q/o [4096,4096], k/v
[1024,4096], gate/up [14336,4096], down [4096,14336], LM head [128256,4096]),
4-bit group 64, bf16 activations, scales and biases, at M = 1 and M = 32.

Each projection runs through the same calls as the bench's fused layer
sequence (query/key/value grouped in one call, gate and up as one SiLU-gated
call, o, down and the LM head alone) and is checked against the oracle on
512 output columns spread across N (all rows), computed on the host's cores.
Tolerance: rtol 1e-2 with atol 1e-2 * rms(expected) for the products
(f32 accumulation of bf16 activations); for silu(gate) * up the same
tolerance carried through the product.

The weights are random packed words (every code equally likely) with
scales and biases of the magnitude a N(0, 0.02) row quantizes to; the
quantize kernel is checked bit-exactly elsewhere.
"""
import numpy as np
import pytest

import affon_amd as A
from oracle import oracle as O
from tests.helpers import assert_bf16_product_close, oracle_columns
from tests.test_gpu_epilogue import silu_gate_close

pytestmark = pytest.mark.gpu

BITS, GROUP = 4, 64
LAYER = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096), "gate": (14336, 4096),
         "up": (14336, 4096), "down": (4096, 14336)}
SAMPLED = 512


def random_projection(rng, N, K):
    packed = rng.integers(0, 1 << 32, size=(N, K * BITS // 32), dtype=np.uint64).astype(np.uint32)
    scales = O.bf16_from_f32((0.008 + 0.004 * rng.random((N, K // GROUP))).astype(np.float32))
    biases = O.bf16_from_f32((-0.06 + 0.02 * rng.random((N, K // GROUP))).astype(np.float32))
    return packed, scales, biases


def upload(session, arr):
    dtype = "u32" if arr.dtype == np.uint32 else "bf16"
    spec = A.TensorSpec.u32(arr.shape) if dtype == "u32" else A.TensorSpec.bf16(arr.shape)
    return session.from_bytes(np.ascontiguousarray(arr), spec)


def sampled(N):
    return np.unique(np.linspace(0, N - 1, min(N, SAMPLED)).astype(int))


def check(out, x, host, cols=None):
    cols = sampled(host[0].shape[0]) if cols is None else cols
    expected = oracle_columns(x, *host, BITS, GROUP, cols)
    assert_bf16_product_close(out[:, cols], expected)


@pytest.mark.parametrize("M", [1, 32])
def test_llama8b_layer_sequence_against_oracle(session, M):
    rng = np.random.default_rng(8000 + M)
    host, dev = {}, {}
    for name, (N, K) in LAYER.items():
        host[name] = random_projection(rng, N, K)
        dev[name] = tuple(upload(session, a) for a in host[name])
    x = O.bf16_from_f32(rng.standard_normal((M, 4096)).astype(np.float32))
    h = O.bf16_from_f32(rng.standard_normal((M, 14336)).astype(np.float32))
    xt, ht = upload(session, x), upload(session, h)

    plan = A.grouped_plan(xt, [dev["q"], dev["k"], dev["v"]], bits=BITS, group_size=GROUP)
    q, k, v = A.quantized_matmul_grouped(xt, [dev["q"], dev["k"], dev["v"]], bits=BITS, group_size=GROUP)
    for name, out in zip("qkv", (q, k, v)):
        assert out.shape == (M, LAYER[name][0])
        check(out.numpy(), x, host[name])
    o = A.quantized_matmul(xt, *dev["o"], bits=BITS, group_size=GROUP)
    check(o.numpy(), x, host["o"])

    gated = A.quantized_silu_gate(xt, dev["gate"], dev["up"], bits=BITS, group_size=GROUP).numpy()
    cols = sampled(14336)
    g = oracle_columns(x, *host["gate"], BITS, GROUP, cols)
    u = oracle_columns(x, *host["up"], BITS, GROUP, cols)
    silu_gate_close(gated[:, cols], g, u, True)

    down = A.quantized_matmul(ht, *dev["down"], bits=BITS, group_size=GROUP)
    check(down.numpy(), h, host["down"])
    impl = A.selected_implementation(ht, *dev["down"], bits=BITS, group_size=GROUP)
    assert impl.startswith("rocm_quantized_matmul."), impl
    assert "rocm_quantized_matmul" in plan and "host_" not in plan


@pytest.mark.parametrize("M", [1, 32])
def test_llama8b_lm_head_against_oracle(session, M):
    rng = np.random.default_rng(9000 + M)
    host = random_projection(rng, 128256, 4096)
    dev = tuple(upload(session, a) for a in host)
    x = O.bf16_from_f32(rng.standard_normal((M, 4096)).astype(np.float32))
    xt = upload(session, x)
    out = A.quantized_matmul(xt, *dev, bits=BITS, group_size=GROUP).numpy()
    cols = np.concatenate([sampled(128256), np.arange(128256 - 64, 128256)])  # and the last row tile
    check(out, x, host, np.unique(cols))
    assert np.isfinite(out).all()
