"""affon_rocm_quantized_matmul_noalloc through the C ABI: the same kernels
with split-K partial sums in the library's static scratch array instead of
the session workspace. Each call is checked against affon_rocm_quantized_matmul
on the same operands. The bar is bit-identical outputs: the same plan runs
and the split-K sums are added in a fixed order. Two calls run in a row, the
second on a smaller problem, so the second reuses the array the first left
behind. A shape whose plan needs more than the array holds must be rejected
before anything is launched, leaving its output untouched."""
import ctypes

import numpy as np
import pytest

import affon_amd as A
from affon_amd import _native, ops
from tests.helpers import HipRuntime

pytestmark = pytest.mark.gpu


def problem(session, M, N, K, seed, group=64):
    rng = np.random.default_rng(seed)
    x = session.from_bytes(A.core.bf16_bits(rng.standard_normal((M, K)).astype(np.float32)), A.TensorSpec.bf16((M, K)))
    w = session.from_bytes(rng.integers(0, 1 << 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32),
                           A.TensorSpec.u32((N, K // 8)))
    s = session.from_bytes(A.core.bf16_bits((0.008 + 0.004 * rng.random((N, K // group))).astype(np.float32)),
                           A.TensorSpec.bf16((N, K // group)))
    b = session.from_bytes(A.core.bf16_bits((-0.06 + 0.02 * rng.random((N, K // group))).astype(np.float32)),
                           A.TensorSpec.bf16((N, K // group)))
    return x, w, s, b


def run(session, entry, operands, policy, group=64):
    x, w, s, b = operands
    out = session.tensor(np.full((x.shape[0], w.shape[0]), 7.0, np.float32))
    desc = ops._descriptor(x, w, s, b, 4, group, out, "auto", policy)
    status = getattr(_native.load(), entry)(session._handle, ctypes.byref(desc))
    message = _native.last_error()  # before the synchronize clears it
    session.synchronize()
    return status, out.numpy(), message


def test_noalloc_matches_allocating_entry_point():
    with A.Session("rocm") as session:
        lib = _native.load()
        cases = [
            # prefill whose four K ranges fill the whole array: 4 x 512 x 4096 f32 = 32 MiB
            ((512, 4096, 14336), "approximate", "rocm_quantized_matmul.mfma"),
            # the same shape under the default policy: the reassociated GEMM's four K ranges of partial
            # sums (32 MiB) plus its per-group activation sums (768 KiB)
            ((512, 4096, 14336), "backend_equivalent", "rocm_quantized_matmul.gemv_mfma"),
            # a smaller decode batch with split K, reusing what the first call left in the array
            ((16, 4096, 4096), "backend_equivalent", "rocm_quantized_matmul.gemv_mfma", 64),
            # groups of 32 on the group-32 GEMM, eight K ranges: exact codes with their per-group
            # activation sums (16 MiB + 1.5 MiB), then rounded weights (16 MiB)
            ((512, 1024, 4096), "backend_equivalent", "rocm_quantized_matmul.gemv_mfma", 32),
            ((512, 1024, 4096), "approximate", "rocm_quantized_matmul.mfma", 32),
        ]
        for (M, N, K), policy, impl, *grp in cases:
            group = grp[0] if grp else 64
            operands = problem(session, M, N, K, seed=M + N, group=group)
            assert A.selected_implementation(*operands, bits=4, group_size=group, policy=policy) == impl
            want_status, want, _ = run(session, "affon_rocm_quantized_matmul", operands, policy, group)
            got_status, got, message = run(session, "affon_rocm_quantized_matmul_noalloc", operands, policy, group)
            assert want_status == 0 and got_status == 0, message
            assert np.isfinite(got).all()
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"{M}x{N}x{K}")
        # 1280 x 4096 prefill: two K ranges of 1280 x 4096 f32 partial sums (42 MB) exceed the array.
        operands = problem(session, 1280, 4096, 4096, seed=3)
        status, out, message = run(session, "affon_rocm_quantized_matmul_noalloc", operands, "approximate")
        assert status == _native.UNSUPPORTED
        assert "no-allocation" in message and "scratch" in message, message
        np.testing.assert_array_equal(out, np.full(out.shape, 7.0, np.float32))
        # The allocating entry point runs it.
        status, out, message = run(session, "affon_rocm_quantized_matmul", operands, "approximate")
        assert status == 0 and np.isfinite(out).all(), message


def test_noalloc_under_graph_capture():
    """The use the entry point is for: calls captured into a HIP graph on the
    session stream and replayed. Both captured plans keep scratch in the
    static array (the default-policy prefill: split-K partial sums and
    per-group activation sums; a decode batch with split K). Between replays
    the program runs eager no-allocation calls of other shapes, which leave
    other contents in the array, and clears the outputs; every replay must
    reproduce the eager results bit for bit."""
    hip = HipRuntime()
    lib = _native.load()
    with A.Session("rocm") as session:
        shapes = [((512, 4096, 14336), "backend_equivalent"), ((16, 4096, 4096), "backend_equivalent")]
        # Each descriptor holds raw device pointers: its operand tensors stay
        # referenced here for as long as the descriptor (and the graph) is used.
        calls = []
        for (M, N, K), policy in shapes:
            operands = problem(session, M, N, K, seed=M + 7)
            out = session.tensor(np.full((M, N), 7.0, np.float32))
            desc = ops._descriptor(*operands, 4, 64, out, "auto", policy)
            calls.append((desc, out, operands))
        eager = []
        for desc, out, _ in calls:  # eager first: the first call on the device looks the array up
            assert lib.affon_rocm_quantized_matmul_noalloc(session._handle, ctypes.byref(desc)) == 0, \
                _native.last_error()
            session.synchronize()
            eager.append(out.numpy().copy())

        def enqueue():
            for desc, _, _ in calls:
                status = lib.affon_rocm_quantized_matmul_noalloc(session._handle, ctypes.byref(desc))
                assert status == 0, _native.last_error()

        graph = hip.capture(session.stream, enqueue)
        try:
            other = problem(session, 64, 2048, 8192, seed=11)
            for i in range(3):
                status, _, message = run(session, "affon_rocm_quantized_matmul_noalloc", other, "backend_equivalent")
                assert status == 0, message
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
