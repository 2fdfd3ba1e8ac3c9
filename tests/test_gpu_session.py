"""Session resource rules on the GPU: scratch memory that a captured graph
still uses survives the session's later growth, and disposing a Session
frees the device memory of tensors that are still alive."""
import numpy as np
import pytest

import affon_amd as A
from affon_amd import _native
from oracle import oracle as O
from tests.helpers import HipRuntime, assert_close_rtol_atol

pytestmark = pytest.mark.gpu


def quantized(session, N, K, bits, group, seed):
    w = session.randn((N, K), seed=seed, std=0.02, dtype="bf16")
    return A.quantize(w, bits=bits, group_size=group, param_dtype="bf16")


def test_workspace_growth_keeps_captured_graph_valid():
    """A split-K decode-batch launch is captured into a graph; a later, larger
    split-K prefill grows the session's workspace. Replays of the graph (with
    eager work between them) must still give the eager result bit for bit:
    the grown workspace retires the captured buffer instead of freeing it.
    Tolerance: bit-exact against the eager run (split-K sums are added in a
    fixed order), and rtol 1e-2 / atol 1e-2*rms against the oracle."""
    hip = HipRuntime()
    with A.Session("rocm") as session:
        M, N, K, bits, group = 8, 2048, 4096, 4, 64
        x = session.randn((M, K), seed=1, dtype="bf16")
        packed, scales, biases = quantized(session, N, K, bits, group, seed=2)
        assert A.selected_implementation(x, packed, scales, biases, bits=bits, group_size=group) == \
            "rocm_quantized_matmul.gemv_mfma"
        out = session.empty("f32", (M, N))
        run = lambda: A.quantized_matmul_into(out, x, packed, scales, biases, bits=bits, group_size=group)
        run()
        eager = out.numpy().copy()
        ref = O.quantized_matmul(x.storage(), packed.storage(), scales.storage(), biases.storage(), bits, group)
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        assert_close_rtol_atol(eager, ref, 1e-2, 1e-2 * rms)

        graph = hip.capture(session.stream, run)
        try:
            # A prefill needing a much larger split-K workspace (4 ranges of [512, 4096] f32).
            x2 = session.randn((512, 14336), seed=3, dtype="bf16")
            w2 = quantized(session, 4096, 14336, 4, 64, seed=4)
            big = session.empty("f32", (512, 4096))
            A.quantized_matmul_into(big, x2, *w2, bits=4, group_size=64, policy="approximate")
            zeros = np.zeros((M, N), np.float32)
            for i in range(3):
                # Eager work between replays: a new allocation, and the output cleared.
                session.tensor(zeros)
                _native.check(_native.load().affon_rocm_memcpy_h2d(session._handle, out.data_ptr,
                                                                   zeros.ctypes.data, zeros.nbytes), "clear")
                hip.replay(session.stream, graph)
                np.testing.assert_array_equal(out.numpy(), eager, err_msg=f"replay {i}")
            assert big.shape == (512, 4096)
        finally:
            hip.destroy(graph)


def test_dispose_frees_live_tensors():
    """Tensors that outlive their Session: disposing the Session returns
    their device memory and the tensors report that they are disposed."""
    hip = HipRuntime()
    session = A.Session("rocm")
    session.synchronize()
    before = hip.free_bytes()
    held = [session.empty("u32", (64 << 20,)) for _ in range(4)]  # 4 x 256 MiB
    assert before - hip.free_bytes() >= 0.9 * 4 * (256 << 20)  # the runtime's figure has some slack
    session.dispose()
    assert hip.free_bytes() >= before - (16 << 20)
    with pytest.raises(RuntimeError, match="disposed"):
        held[0].numpy()
    del held  # releasing after dispose frees nothing twice
