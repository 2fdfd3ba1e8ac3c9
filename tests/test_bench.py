"""CPU checks of the benchmark's contract: the one-GPU refusal, the
algorithmic byte counts its roofline figures divide by, and the restated CPU
kernel it times beside the GPU lines."""
import subprocess
import sys
import types

import numpy as np
import pytest

import bench
from oracle import oracle as O
from tests.helpers import pack_codes, storage


def test_more_than_one_gpu_is_refused_before_any_device_work():
    result = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True,
                            cwd=str(bench.ROOT), timeout=120)
    assert result.returncode == 2
    assert "one GPU only" in result.stderr
    assert result.stdout == ""


@pytest.mark.parametrize("shape,expected", [
    # (M, N, K, bits, group, x bytes, param bytes): the per-launch byte counts of the benchmark's workloads
    ((1, 14336, 4096, 4, 64, 2, 2), 33_095_680),        # headline decode, 4-bit g64 M=1
    ((1, 4096, 4096, 4, 64, 4, 4), 10_518_528),         # f32 decode 4096 x 4096
    ((1, 14336, 4096, 8, 64, 2, 2), 62_455_808),        # 8-bit decode M=1
    ((16, 14336, 4096, 8, 64, 2, 2), 63_438_848),       # 8-bit decode M=16
    ((512, 14336, 4096, 4, 64, 2, 2), 66_584_576),      # prefill 512 x 14336 x 4096
    ((512, 4096, 14336, 4, 64, 2, 2), 56_098_816),      # prefill 512 x 4096 x 14336
    ((2048, 28672, 8192, 4, 32, 2, 2), 415_236_096),    # stress GEMM 2048 x 28672 x 8192
    ((2048, 8192, 28672, 4, 32, 2, 2), 331_350_016),    # stress GEMM 2048 x 8192 x 28672
])
def test_algorithmic_bytes_match_the_per_unit_formula(shape, expected):
    """N*K*bits/8 + 2*N*(K/g)*param + M*K*x + M*N*4, against the byte counts
    stated for each configuration independently of this code."""
    assert bench.algorithmic_bytes(*shape) == expected


def _workload(M, N, K, bits, group, rng):
    x = storage(rng.standard_normal((M, K)), "bf16")
    codes = rng.integers(0, 1 << bits, (N, K))
    packed = pack_codes(codes, bits)
    scales = storage(rng.uniform(0.01, 0.02, (N, K // group)), "bf16")
    biases = storage(rng.uniform(-0.1, 0.0, (N, K // group)), "bf16")
    work = types.SimpleNamespace(M=M, N=N, K=K, bits=bits, group=group, x_dtype="bf16", p_dtype="bf16")
    work.host_operands = lambda: (x, packed, scales, biases)
    return work, (x, packed, scales, biases)


@pytest.mark.parametrize("unit", ["GB/s", "TFLOP/s"])
def test_cpu_baseline_reports_a_checked_sample(unit, rng):
    """The sample's output equals the oracle's bit for bit (so its error
    against an output that equals the oracle is zero), and the record names
    what was timed."""
    work, (x, packed, scales, biases) = _workload(3, 96, 256, 4, 64, rng)
    expected = O.quantized_matmul(x, packed, scales, biases, 4, 64)
    record = bench.cpu_baseline(work, expected, seconds=0.05, unit=unit, check_rows=96)
    assert record["unit"] == unit and record["cores"] == 1 and record["kind"] == "port"
    assert record["value"] > 0 and record["max_abs_err_vs_gpu"] == 0.0
    assert "oracle/cpu_baseline.c" in record["sample"] and "1 thread" in record["sample"]


def test_cpu_baseline_reports_the_distance_from_the_gpu_output(rng):
    work, (x, packed, scales, biases) = _workload(2, 64, 128, 8, 32, rng)
    shifted = O.quantized_matmul(x, packed, scales, biases, 8, 32) + np.float32(0.25)
    record = bench.cpu_baseline(work, shifted, seconds=0.05, threads=2)
    assert record["cores"] == 2
    assert abs(record["max_abs_err_vs_gpu"] - 0.25) < 1e-3
