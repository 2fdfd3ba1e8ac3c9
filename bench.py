#!/usr/bin/env python3
"""Benchmark of the rocm weight-quantized linear path on one MI355X.

A step is one quantized_matmul launch over one batch of synthetic input with
the inputs already resident in HBM. The reported workload (`value`,
`roofline`) is the 4-bit group-64 decode GEMV: W [14336, 4096] packed u32
(8 codes per word) with bf16 scales/biases, x bf16 [1, 4096], f32 out, from
Affon's seeded generator (x: seed 1 N(0,1); W: seed 2 N(0,0.02), quantized on
the GPU). `roofline_prefill` is the M=512 prefill of the same weight format
(x bf16 [512, 4096], W [14336, 4096]) as its configuration describes it
(decoded weights rounded to bf16 and fed to bf16 MFMA: the approximate
policy) against the bf16 MFMA peak, with the reference's CPU kernel timed on
a sample of its output columns beside it; the default policy's unrounded
GEMM is timed beside it. The same run measures, as extra fields, the 8-bit
decode sweep M in {1,2,4,8,16}, 4-bit M=16, both prefill orientations
(approximate and default policies), the 2048-row group-32 stress shapes
(approximate and default policies), the Llama-8B-shaped layer sequences at
M=1 and M=32, and the f32 4096x4096 4-bit case.

Timing: the K timed steps are captured once into a HIP graph on the session's
stream; after about 0.1 s of untimed replays (the clock settles under the
load), one untimed replay and then REPLAYS timed replays are enqueued back to
back, with a HIP event on that stream between consecutive replays. The median
interval over K gives the per-step time: the GPU's back-to-back launch
period, without host overhead (the graph's launch latency falls in the
untimed replay). Weight sets are rotated (>= 9 sets, > 600 MB in total) so that the
256 MB Infinity Cache cannot hold the working set.

Prints one JSON line. --gpus N with N > 1 exits: this path runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import pathlib
import platform
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "quant matmul GB/s (M=1) & TFLOP/s (M=512); % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
ROTATION_BYTES = 600e6
REPLAYS = 5


class Hip:
    """The few HIP runtime calls the benchmark needs (events and graphs)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        sig = {
            "hipEventCreate": [pvp], "hipEventRecord": [vp, vp], "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp], "hipEventDestroy": [vp],
            "hipStreamBeginCapture": [vp, ctypes.c_int], "hipStreamEndCapture": [vp, pvp],
            "hipGraphInstantiate": [pvp, vp, vp, ctypes.c_char_p, ctypes.c_size_t], "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp], "hipGraphDestroy": [vp], "hipStreamSynchronize": [vp],
        }
        for name, args in sig.items():
            fn = getattr(self.lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int

    def check(self, status: int, what: str) -> None:
        if status != 0:
            raise RuntimeError(f"{what} failed with HIP status {status}")

    def event(self) -> ctypes.c_void_p:
        ev = ctypes.c_void_p()
        self.check(self.lib.hipEventCreate(ctypes.byref(ev)), "hipEventCreate")
        return ev


def algorithmic_bytes(M, N, K, bits, group, xbytes, pbytes):
    """N*K*bits/8 + 2*N*(K/g)*sizeof(param) + M*K*sizeof(x) + M*N*4."""
    return N * K * bits // 8 + 2 * N * (K // group) * pbytes + M * K * xbytes + M * N * 4


SETTLE_S = 0.1


def settle(hip: Hip, session, replay) -> None:
    """Untimed replays until about SETTLE_S seconds of GPU time have passed,
    so that the timed replays run at the clock the GPU settles to under this
    load (matrix-core work lowers it within tens of milliseconds)."""
    stream = ctypes.c_void_p(session.stream)
    start, stop = hip.event(), hip.event()
    hip.check(hip.lib.hipEventRecord(start, stream), "hipEventRecord")
    replay()
    hip.check(hip.lib.hipEventRecord(stop, stream), "hipEventRecord")
    hip.check(hip.lib.hipEventSynchronize(stop), "hipEventSynchronize")
    ms = ctypes.c_float()
    hip.check(hip.lib.hipEventElapsedTime(ctypes.byref(ms), start, stop), "hipEventElapsedTime")
    for _ in range(min(1000, int(SETTLE_S * 1e3 / max(ms.value, 1e-3)))):
        replay()
    session.synchronize()
    hip.lib.hipEventDestroy(start)
    hip.lib.hipEventDestroy(stop)


class Workload:
    def __init__(self, session, name, M, N, K, bits, group, x_dtype="bf16", p_dtype="bf16", policy="backend_equivalent",
                 w_dtype=None, seed_x=1, seed_w=2):
        import affon_amd as A
        from affon_amd import ops
        self.session, self.name = session, name
        self.M, self.N, self.K, self.bits, self.group = M, N, K, bits, group
        self.x_dtype, self.p_dtype, self.policy = x_dtype, p_dtype, policy
        xbytes = 2 if x_dtype == "bf16" else 4
        pbytes = 2 if p_dtype == "bf16" else 4
        self.bytes = algorithmic_bytes(M, N, K, bits, group, xbytes, pbytes)
        self.flops = 2 * M * N * K
        set_bytes = N * K * bits // 8 + 2 * N * (K // group) * pbytes
        self.sets = max(9, math.ceil(ROTATION_BYTES / set_bytes))
        self.x = session.randn((M, K), seed=seed_x, dtype=x_dtype)
        w = session.randn((N, K), seed=seed_w, std=0.02, dtype=w_dtype or p_dtype)
        packed, scales, biases = A.quantize(w, bits=bits, group_size=group, param_dtype=p_dtype)
        del w
        self.weights = [(packed, scales, biases)]
        for _ in range(self.sets - 1):
            copies = []
            for t in (packed, scales, biases):
                c = session.empty(t.dtype, t.shape)
                ops._native.check(ops._native.load().affon_rocm_memcpy_d2d(
                    session._handle, c.data_ptr, t.data_ptr, c._buffer.nbytes), "copy")
                copies.append(c)
            self.weights.append(tuple(copies))
        self.out = session.empty("f32", (M, N))
        self.implementation = A.selected_implementation(self.x, packed, scales, biases, bits=bits, group_size=group,
                                                        policy=policy)
        self.descs = [ops._descriptor(self.x, w_, s_, b_, bits, group, self.out, "auto", policy)
                      for (w_, s_, b_) in self.weights]
        self.lib = ops._native.load()

    def launch(self, i: int) -> None:
        status = self.lib.affon_rocm_quantized_matmul(self.session._handle, ctypes.byref(self.descs[i % self.sets]))
        if status != 0:
            from affon_amd import _native
            raise RuntimeError(_native.last_error())

    def time(self, hip: Hip, steps: int, warmup: int, use_graph: bool = True) -> float:
        """Milliseconds per step: the median over REPLAYS timed runs of `steps`
        back-to-back launches (graph replays, or direct launches with
        --launch stream). Every run's figure is kept in self.replay_ms."""
        if use_graph:
            self.replay_ms = time_graph(hip, self.session, self.launch, steps, warmup)
            return median(self.replay_ms)
        stream = ctypes.c_void_p(self.session.stream)
        for i in range(warmup):
            self.launch(i)
        self.session.synchronize()
        start, stop = hip.event(), hip.event()
        runs = []
        for _ in range(REPLAYS):
            hip.check(hip.lib.hipEventRecord(start, stream), "hipEventRecord")
            for i in range(steps):
                self.launch(i)
            hip.check(hip.lib.hipEventRecord(stop, stream), "hipEventRecord")
            hip.check(hip.lib.hipEventSynchronize(stop), "hipEventSynchronize")
            ms = ctypes.c_float()
            hip.check(hip.lib.hipEventElapsedTime(ctypes.byref(ms), start, stop), "hipEventElapsedTime")
            runs.append(ms.value / steps)
        self.session.synchronize()
        hip.lib.hipEventDestroy(start)
        hip.lib.hipEventDestroy(stop)
        self.replay_ms = runs
        return median(runs)

    def time_read_floor(self, hip: Hip, steps: int, warmup: int) -> float:
        """Milliseconds per launch of affon_rocm_read_floor over the same
        rotated weight sets (packed words, scales, biases): the median of
        REPLAYS graph replays of `steps` launches, as for the workload."""
        sink = self.session.empty("u32", (4,))
        calls = []
        for packed, scales, biases in self.weights:
            ptrs = (ctypes.c_void_p * 3)(packed.data_ptr, scales.data_ptr, biases.data_ptr)
            sizes = (ctypes.c_uint64 * 3)(packed._buffer.nbytes, scales._buffer.nbytes, biases._buffer.nbytes)
            calls.append((ptrs, sizes))

        def launch(i):
            ptrs, sizes = calls[i % len(calls)]
            if self.lib.affon_rocm_read_floor(self.session._handle, ptrs, sizes, 3, sink.data_ptr) != 0:
                from affon_amd import _native
                raise RuntimeError(_native.last_error())

        return median(time_graph(hip, self.session, launch, steps, warmup))

    def host_operands(self):
        packed, scales, biases = self.weights[0]
        return self.x.storage(), packed.storage(), scales.storage(), biases.storage()

    def release(self) -> None:
        self.weights.clear()
        self.descs.clear()


def _cpu_name() -> str:
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(line.split(":", 1)[1].strip() for line in f if line.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return cpu


def _host_cores() -> int:
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(16, cores))  # the GPU box's CPU share is 16 cores


def cpu_baseline(work: Workload, gpu_out: np.ndarray, seconds: float = 10.0, threads: int = 1,
                 unit: str = "GB/s", check_rows: int = 512) -> dict:
    """The reference's scalar CPU kernel as restated in oracle/cpu_baseline.c
    (one specialised loop per bit width and dtype pair, ordered f32, decode
    inside the dot product), timed on this host over a bounded sample of
    about `seconds`: repeated whole passes of the workload, or a prefix of
    output rows when one pass takes longer. With threads > 1 the output rows
    are split over that many threads (the C call releases the interpreter
    lock). Checks its output against the GPU's and, on its first
    `check_rows` output rows, bit for bit against the oracle's."""
    from concurrent.futures import ThreadPoolExecutor
    from oracle import oracle as O
    x, packed, scales, biases = work.host_operands()
    M, N, K = work.M, work.N, work.K
    out = np.zeros((M, N), dtype=np.float32)

    def run(rows, pool):
        bounds = [(rows * i // threads, rows * (i + 1) // threads) for i in range(threads)]
        call = lambda r: O.baseline_quantized_matmul(x, packed, scales, biases, work.bits, work.group,
                                                     n_range=r, out=out)
        if pool is None:
            call((0, rows))
        else:
            list(pool.map(call, bounds))

    with ThreadPoolExecutor(threads) if threads > 1 else _NullPool() as pool:
        probe = min(N, 256 * threads, max(threads, 4_000_000_000 // (2 * M * K)))  # a few seconds at most
        t0 = time.perf_counter()
        run(probe, pool if threads > 1 else None)
        per_row = (time.perf_counter() - t0) / probe
        rows = int(min(N, max(probe, seconds / max(per_row, 1e-12))))
        passes = max(1, int(seconds / max(per_row * N, 1e-12))) if rows == N else 1
        t0 = time.perf_counter()
        for _ in range(passes):
            run(rows, pool if threads > 1 else None)
        elapsed = time.perf_counter() - t0
    xbytes = 2 if work.x_dtype == "bf16" else 4
    pbytes = 2 if work.p_dtype == "bf16" else 4
    sample_bytes = passes * algorithmic_bytes(M, rows, K, work.bits, work.group, xbytes, pbytes)
    sample_flops = passes * 2 * M * rows * K
    check = min(rows, check_rows)
    ref = O.quantized_matmul(x, packed, scales, biases, work.bits, work.group, n_range=(0, check))
    if not np.array_equal(out[:, :check].view(np.uint32), ref[:, :check].view(np.uint32)):
        raise AssertionError("CPU baseline loop differs from the oracle")
    err = float(np.abs(gpu_out[:, :rows].astype(np.float64) - out[:, :rows]).max())
    value = sample_bytes / elapsed / 1e9 if unit == "GB/s" else sample_flops / elapsed / 1e12
    return {"value": round(value, 6), "unit": unit, "cores": threads, "kind": "port",
            "sample": (f"reference CPU kernel restated (oracle/cpu_baseline.c: scalar, specialised per bits and "
                       f"dtype pair, ordered f32) over the timed workload, "
                       + (f"{passes} whole passes" if rows == N else f"rows 0..{rows} of {N} ({rows / N:.1%})")
                       + f", {elapsed:.1f} s on {threads} thread{'s' if threads > 1 else ''}; host {_cpu_name()}, "
                         f"nproc {os.cpu_count()}"),
            "max_abs_err_vs_gpu": err}


class _NullPool:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


def host_entry(work: Workload, calls: int = 50, warmup: int = 5) -> dict:
    """The drop-in host entry compute_core_run_quantized_matmul_f32 (the
    reference's Cyna C ABI, f32 operands in host memory) over the workload's
    own operands: each call allocates the device buffers, copies every
    operand in from pageable host memory, launches, copies the output back and
    frees. Wall-clock per synchronous call from this Python caller; the
    median over `calls`. The PCIe-inclusive rate, never the headline."""
    from affon_amd import _native
    x, packed, scales, biases = work.host_operands()
    out = np.empty((work.M, work.N), dtype=np.float32)
    lib = _native.load()
    args = (x.ctypes.data, x.size, packed.ctypes.data, packed.size, scales.ctypes.data, scales.size,
            biases.ctypes.data, biases.size, out.ctypes.data, out.size, work.M, work.K, work.N, work.bits, work.group)
    times = []
    for i in range(warmup + calls):
        t0 = time.perf_counter()
        status = lib.compute_core_run_quantized_matmul_f32(*args)
        if status != 0:
            raise RuntimeError(f"compute_core_run_quantized_matmul_f32 returned {status}: {_native.last_error()}")
        if i >= warmup:
            times.append(time.perf_counter() - t0)
    t = median(times)
    gpu = work.out.numpy()
    if not np.array_equal(out.view(np.uint32), gpu.view(np.uint32)):
        raise AssertionError("host entry output differs from the device launch")
    return {"us_per_call": round(t * 1e6, 1), "GB/s": round(work.bytes / t / 1e9, 2), "calls": calls,
            "includes": "device allocation of the five buffers, host-to-device copies of every operand from pageable "
                        "host memory, the launch, the device-to-host copy of the output and the frees; synchronous, "
                        "Python caller"}


def end_to_end(work: Workload, calls: int = 200) -> dict:
    """One call as the reference's benchmark times it: launch, then read the
    output back to the host (the host read synchronises), per call, from
    this Python caller."""
    out_ptr = ctypes.c_void_p(work.out.data_ptr)
    host = np.empty(work.M * work.N, dtype=np.float32)
    nbytes = host.nbytes

    def call(i):
        work.launch(i)
        status = work.lib.affon_rocm_memcpy_d2h(work.session._handle, host.ctypes.data, out_ptr, nbytes)
        if status != 0:
            raise RuntimeError("readback failed")

    for i in range(10):
        call(i)
    t0 = time.perf_counter()
    for i in range(calls):
        call(i)
    us = (time.perf_counter() - t0) / calls * 1e6
    return {"us_per_call": round(us, 2), "GB/s": round(work.bytes / (us * 1e-6) / 1e9, 1), "calls": calls,
            "includes": "launch + device-to-host copy of the output, synchronous, Python caller"}


def roofline_gemv(work: Workload, ms: float, traffic) -> dict:
    achieved = work.bytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}


def roofline_gemm(work: Workload, ms: float, traffic) -> dict:
    achieved = work.flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / BF16_MFMA_PEAK_TFLOPS, 4), "traffic": traffic,
            "workload": work.name, "implementation": work.implementation, "policy": work.policy}


def load_traffic(name: str):
    """HBM bytes per launch of the workload's kernel: FETCH_SIZE + WRITE_SIZE
    from counter runs, each scaled by the same counter's reading for a copy of
    known size (profiles/traffic.json, written from those runs)."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get(name)
    return None if entry is None else entry["traffic_bytes"]


LLAMA8B_LAYER = (("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                 ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336), ("lm_head", 128256, 4096))


def layer_sequence(session, hip: Hip, M: int, steps: int, warmup: int, fused: bool = False, sets: int = 2) -> dict:
    """The Llama-8B-shaped projections at 4-bit group 64 (bf16 x, scales and
    biases; one weight seed per projection), run back to back on one stream:
    a step is the whole sequence. One set of the eight weight tensors holds
    418.9 MB of packed words, scales and biases, more than the 256 MB MALL,
    and steps alternate between `sets` such sets (838 MB for two), so a
    step's weights were last touched 838 MB of traffic earlier and come from
    HBM. With ``fused`` the query, key and value projections run as one
    grouped call and the gate and up projections as one SiLU-gated call
    (silu(gate) * up written once)."""
    import affon_amd as A
    from affon_amd import ops
    lib = ops._native.load()
    tensors = []

    def build(copy: int):
        calls, impls, nbytes, flops = [], {}, 0, 0
        by_name = {}
        for i, (name, N, K) in enumerate(LLAMA8B_LAYER):
            x = session.randn((M, K), seed=1, dtype="bf16")
            w = session.randn((N, K), seed=3 + i + 100 * copy, std=0.02, dtype="bf16")
            packed, scales, biases = A.quantize(w, bits=4, group_size=64, param_dtype="bf16")
            del w
            by_name[name] = (x, packed, scales, biases)
            nbytes += algorithmic_bytes(M, N, K, 4, 64, 2, 2)
            flops += 2 * M * N * K
            if fused and name in ("k", "v"):
                # Grouped with q: rebuild the grouped call with every member so far.
                members = [n for n in ("q", "k", "v") if n in by_name]
                qx = by_name["q"][0]
                projections = [by_name[n][1:] for n in members]
                outs = [session.empty("f32", (M, by_name[n][1].shape[0])) for n in members]
                descs, epis = ops._grouped_arrays(qx, projections, 4, 64, outs, "auto", "backend_equivalent")
                calls[0] = (lib.affon_rocm_quantized_matmul_grouped, descs, (epis, len(members)))
                impls.pop("q", None)
                impls.pop("q+k", None)
                impls["+".join(members)] = A.grouped_plan(qx, projections, bits=4, group_size=64)
                tensors.append((x, packed, scales, biases, outs, descs, epis))
                continue
            if fused and name == "up":
                gx, gp, gs, gb = by_name["gate"]
                epi = ops._epilogue(up=(packed, scales, biases))
                calls[-1] = (lib.affon_rocm_quantized_matmul_fused, calls[-1][1], epi)
                impls["gate+up"] = A.fused_plan(gx, gp, gs, gb, bits=4, group_size=64, up=(packed, scales, biases))
                del impls["gate"]
                nbytes -= M * N * 4  # one [M, N] output instead of two
                tensors.append((x, packed, scales, biases, epi))
                continue
            out = session.empty("f32", (M, N))
            calls.append((lib.affon_rocm_quantized_matmul,
                          ops._descriptor(x, packed, scales, biases, 4, 64, out, "auto", "backend_equivalent"), None))
            impls[name] = A.selected_implementation(x, packed, scales, biases, bits=4, group_size=64)
            tensors.append((x, packed, scales, biases, out))
        return calls, impls, nbytes, flops

    built = [build(c) for c in range(sets)]
    impls, nbytes, flops = built[0][1], built[0][2], built[0][3]

    def launch_all(step: int):
        for fn, desc, epi in built[step % sets][0]:
            if epi is None:
                status = fn(session._handle, ctypes.byref(desc))
            elif isinstance(epi, tuple):  # grouped: arrays of descriptors and epilogues
                status = fn(session._handle, desc, epi[0], epi[1])
            else:
                status = fn(session._handle, ctypes.byref(desc), ctypes.byref(epi))
            if status != 0:
                from affon_amd import _native
                raise RuntimeError(_native.last_error())

    times = time_graph(hip, session, launch_all, steps, warmup)
    t = sorted(times)[len(times) // 2]
    tensors.clear()
    built.clear()
    return {"implementations": impls, "us_per_layer": round(t * 1e3, 2),
            "us_per_layer_replays": [round(v * 1e3, 2) for v in times],
            "GB/s": round(nbytes / (t * 1e-3) / 1e9, 1), "hbm_frac": round(nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "TFLOP/s": round(flops / (t * 1e-3) / 1e12, 3), "algorithmic_bytes": nbytes, "weight_sets": sets}


def quantize_stress(session, hip: Hip, steps: int, warmup: int) -> dict:
    """Quantize of the 2048-row stress shape's first weight matrix: f32 W
    [28672, 8192] (seed 2, N(0, 0.02)) to 4-bit codes with bf16 scales and
    biases in groups of 32, through affon_rocm_quantize into preallocated
    outputs. Algorithmic bytes: the f32 read, the packed codes and both
    parameter planes (1,086,324,736). W (940 MB) exceeds the 256 MB MALL, so
    every launch reads it from HBM."""
    from affon_amd import _native
    N, K, bits, group = 28672, 8192, 4, 32
    w = session.randn((N, K), seed=2, std=0.02, dtype="f32")
    packed = session.empty("u32", (N, K * bits // 32))
    scales = session.empty("bf16", (N, K // group))
    biases = session.empty("bf16", (N, K // group))
    lib = _native.load()

    def launch(i):
        _native.check(lib.affon_rocm_quantize(session._handle, w.data_ptr, _native.F32, N, K, bits, group,
                                              packed.data_ptr, scales.data_ptr, biases.data_ptr, _native.BF16),
                      "quantize")

    times = time_graph(hip, session, launch, steps, warmup)
    t = median(times)
    nbytes = N * K * 4 + N * K * bits // 8 + 2 * N * (K // group) * 2
    return {"us_per_step": round(t * 1e3, 3), "us_per_step_replays": [round(v * 1e3, 3) for v in times],
            "GB/s": round(nbytes / (t * 1e-3) / 1e9, 1), "hbm_frac": round(nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": nbytes, "shape": [N, K], "bits": bits, "group_size": group,
            "weight_dtype": "f32", "param_dtype": "bf16"}


def dequantize_stress(session, hip: Hip, steps: int, warmup: int) -> dict:
    """Dequantize of the same matrix back to f32: the packed 4-bit codes and
    bf16 scales and biases of f32 W [28672, 8192] (seed 2, N(0, 0.02), group
    32, quantized once beforehand) through affon_rocm_dequantize into a
    preallocated f32 [28672, 8192]. Algorithmic bytes: the codes, both
    parameter planes and the f32 write (1,086,324,736)."""
    import affon_amd as A
    from affon_amd import _native
    N, K, bits, group = 28672, 8192, 4, 32
    w = session.randn((N, K), seed=2, std=0.02, dtype="f32")
    packed, scales, biases = A.quantize(w, bits=bits, group_size=group, param_dtype="bf16")
    out = session.empty("f32", (N, K))
    lib = _native.load()

    def launch(i):
        _native.check(lib.affon_rocm_dequantize(session._handle, packed.data_ptr, scales.data_ptr, biases.data_ptr,
                                                _native.BF16, N, K, bits, group, out.data_ptr, _native.F32),
                      "dequantize")

    times = time_graph(hip, session, launch, steps, warmup)
    t = median(times)
    nbytes = N * K * bits // 8 + 2 * N * (K // group) * 2 + N * K * 4
    return {"us_per_step": round(t * 1e3, 3), "us_per_step_replays": [round(v * 1e3, 3) for v in times],
            "GB/s": round(nbytes / (t * 1e-3) / 1e9, 1), "hbm_frac": round(nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": nbytes, "shape": [N, K], "bits": bits, "group_size": group,
            "param_dtype": "bf16", "out_dtype": "f32"}


def reference_workload(session, hip: Hip, steps: int, warmup: int) -> dict:
    """The workload of the reference's own published timings
    (docs/core/quantized-inference.md:315-320, Apple M4): 8-bit codes,
    N = 2048, K = 1024, group 64, f32 activations, bf16 scales and biases,
    f32 output, M = 1, 8, 32 and 128, seeded as the other lines. Per M: the
    graph-replay period of the launch on resident operands, and one call with
    full readback (launch, then the synchronous copy of the output to the
    host), the kind of figure those timings are (0.400 / 1.033 / 2.500 /
    8.667 ms for Affon's Metal path there)."""
    result = {}
    for M in (1, 8, 32, 128):
        work = Workload(session, f"reference_8bit_g64_n2048_k1024_m{M}", M, 2048, 1024, 8, 64, x_dtype="f32",
                        p_dtype="bf16")
        t = work.time(hip, steps, warmup, True)
        e2e = end_to_end(work)
        result[f"m{M}"] = {"implementation": work.implementation, "us_per_step": round(t * 1e3, 3),
                           "us_per_step_replays": [round(v * 1e3, 3) for v in work.replay_ms],
                           "GB/s": round(work.bytes / (t * 1e-3) / 1e9, 1),
                           "full_readback_us_per_call": e2e["us_per_call"]}
        work.release()
    return result


def time_graph(hip: Hip, session, launch, steps: int, warmup: int) -> list:
    """Per-launch milliseconds of `steps` launches captured in one HIP graph
    on the session stream, for each of REPLAYS replays (after `warmup`
    direct launches and about 0.1 s of untimed replays). launch(i) enqueues
    launch i. All replays are enqueued back to back behind one untimed lead-in
    replay, with an event between consecutive replays: each timed interval is
    one replay's launches, and the graph's launch latency falls in the
    lead-in."""
    stream = ctypes.c_void_p(session.stream)
    for i in range(warmup):
        launch(i)
    session.synchronize()
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    hip.check(hip.lib.hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")  # relaxed
    for i in range(steps):
        launch(i)
    hip.check(hip.lib.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
    hip.check(hip.lib.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
    replay = lambda: hip.check(hip.lib.hipGraphLaunch(exe, stream), "hipGraphLaunch")
    settle(hip, session, replay)
    events = [hip.event() for _ in range(REPLAYS + 1)]
    replay()  # lead-in
    for e in range(REPLAYS + 1):
        hip.check(hip.lib.hipEventRecord(events[e], stream), "hipEventRecord")
        if e < REPLAYS:
            replay()
    hip.check(hip.lib.hipEventSynchronize(events[-1]), "hipEventSynchronize")
    runs = []
    for e in range(REPLAYS):
        ms = ctypes.c_float()
        hip.check(hip.lib.hipEventElapsedTime(ctypes.byref(ms), events[e], events[e + 1]), "hipEventElapsedTime")
        runs.append(ms.value / steps)
    hip.lib.hipGraphExecDestroy(exe)
    hip.lib.hipGraphDestroy(graph)
    for e in events:
        hip.lib.hipEventDestroy(e)
    return runs


def median(values):
    return sorted(values)[len(values) // 2]


def floor_sweep(session, hip: Hip, steps: int, warmup: int) -> dict:
    """What a decode launch's graph-replay period is made of, measured with
    the library's diagnostic kernels over rotated random data (never a MALL
    hit): the period of an empty launch; pure reads of the 4-bit 14336 x 4096
    weight set (33,095,680 bytes) by read geometry (KiB per wave, workgroup
    size); the same reads plus output stores (by how many waves store) and
    plus vector arithmetic per wave (the M = 1 decode's packed-word
    arithmetic alone is 88 instructions per 2 KiB); pure reads by size (a
    stream rate plus a fixed cost); and the decode kernel itself against the
    number of weight rows, fitted the same way."""
    from affon_amd import _native
    lib = _native.load()
    progress = lambda m: print(f"floor-sweep: {m}", file=sys.stderr, flush=True)  # noqa: E731
    pool_bytes = 1200 << 20
    pool = session.empty("u32", (pool_bytes // 4,))
    rng = np.random.default_rng(7)
    piece = rng.integers(0, 2**32, size=(64 << 20) // 4, dtype=np.uint32)
    for off in range(0, pool_bytes, piece.nbytes):
        piece ^= np.uint32(0x9E3779B9)
        _native.check(lib.affon_rocm_memcpy_h2d(session._handle, pool.data_ptr + off, piece.ctypes.data,
                                                min(piece.nbytes, pool_bytes - off)), "upload")
    sink = session.empty("u32", (1 << 20,))
    headline = 33095680
    out = {"headline_bytes": headline, "pool_bytes": pool_bytes, "steps": steps}

    def offsets(nbytes):
        stride = (nbytes + 4095) // 4096 * 4096
        return [pool.data_ptr + k * stride for k in range(pool_bytes // stride)]

    def read(nbytes, kib=2, threads=256, valu=0, store_every=0):
        ptrs = offsets(nbytes)
        g = _native.FloorGeometry(kib, threads, valu, store_every)

        def launch(i):
            _native.check(lib.affon_rocm_read_floor_geometry(session._handle, ptrs[i % len(ptrs)], nbytes,
                                                             sink.data_ptr, sink._buffer.nbytes, ctypes.byref(g)),
                          "read_floor_geometry")
        return round(median(time_graph(hip, session, launch, steps, warmup)) * 1e3, 3)

    def empty(blocks, threads):
        def launch(i):
            _native.check(lib.affon_rocm_empty_launch(session._handle, blocks, threads), "empty_launch")
        return round(median(time_graph(hip, session, launch, steps, warmup)) * 1e3, 3)

    out["empty_launch_us"] = {"1x64": empty(1, 64), "1792x256": empty(1792, 256), "7168x256": empty(7168, 256)}
    progress(f"empty launch {out['empty_launch_us']}")
    geometry = {}
    for kib in (1, 2, 4, 8):
        for threads in (64, 128, 256, 512, 1024):
            geometry[f"{kib}KiB_per_wave_T{threads}"] = read(headline, kib, threads)
    out["read_us_by_geometry"] = geometry
    best = min(geometry, key=geometry.get)
    out["best_read"] = {"geometry": best, "us": geometry[best],
                        "GB/s": round(headline / (geometry[best] * 1e-6) / 1e9, 1)}
    progress(f"best read geometry {out['best_read']}")
    out["read_us_by_store_every"] = {str(e): read(headline, 2, 256, 0, e) for e in (0, 1, 4, 16, 64)}
    out["read_us_by_valu_per_wave"] = {str(v): read(headline, 2, 256, v) for v in (0, 32, 64, 88, 128, 176, 256, 352)}
    progress(f"stores {out['read_us_by_store_every']}; arithmetic {out['read_us_by_valu_per_wave']}")
    sizes = {}
    for mb in (4, 8, 16, 32, 64, 128, 296):
        nbytes = mb << 20
        sizes[str(nbytes)] = read(nbytes, 2, 256)
    out["read_us_by_bytes"] = sizes
    xs = np.array([float(b) for b in sizes]), np.array(list(sizes.values()))
    slope, fixed = np.polyfit(xs[0], xs[1], 1)
    out["read_fit"] = {"fixed_us": round(float(fixed), 3), "stream_GB/s": round(1e-3 / float(slope), 1)}
    progress(f"read fit {out['read_fit']}")
    pool.dispose()
    pool = None  # the allocation is freed with its last reference
    decode = {}
    for N in (1792, 3584, 7168, 14336, 28672, 57344, 128256):
        work = Workload(session, f"decode_4bit_g64_m1_n{N}", 1, N, 4096, 4, 64)
        decode[str(N)] = {"bytes": work.bytes, "us": round(work.time(hip, steps, warmup) * 1e3, 3),
                          "implementation": work.implementation}
        work.release()
        progress(f"decode N={N}: {decode[str(N)]['us']} us")
    out["decode_us_by_rows"] = decode
    xs = np.array([v["bytes"] for v in decode.values()], dtype=float), np.array([v["us"] for v in decode.values()])
    slope, fixed = np.polyfit(xs[0], xs[1], 1)
    out["decode_fit"] = {"fixed_us": round(float(fixed), 3), "stream_GB/s": round(1e-3 / float(slope), 1)}
    return out


def copy_calibration(session) -> int:
    """Copies of a known size, profiled with the same byte counters as the
    kernels, give the factor from counter units to bytes."""
    from affon_amd import _native
    lib = _native.load()
    nbytes = 256 << 20
    src, dst = session.empty("u32", (nbytes // 4,)), session.empty("u32", (nbytes // 4,))
    for _ in range(8):
        _native.check(lib.affon_rocm_memcpy_d2d(session._handle, dst.data_ptr, src.data_ptr, nbytes), "copy")
    session.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 8}), flush=True)
    session.dispose()
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--launch", choices=["graph", "stream"], default="graph")
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--only", default="", help="comma-separated subset of extra workloads to run ('none': no extras)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run 8 device-to-device copies of 256 MiB (for scaling hardware byte counters)")
    parser.add_argument("--floor-sweep", action="store_true",
                        help="only measure what an M = 1 decode launch's period is made of (prints one JSON line)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the quantized linear path has no multi-GPU execution "
              f"(requested --gpus {args.gpus})", file=sys.stderr)
        return 2

    import affon_amd as A
    hip = Hip()
    session = A.Session("rocm")
    use_graph = args.launch == "graph"
    if args.copy_calibration:
        return copy_calibration(session)
    if args.floor_sweep:
        print(json.dumps({"floor_sweep": floor_sweep(session, hip, args.steps, args.warmup)}), flush=True)
        session.dispose()
        return 0

    def progress(message: str) -> None:
        print(f"bench: {message}", file=sys.stderr, flush=True)

    only = set(filter(None, args.only.split(",")))

    def want(name):
        return not only or name in only

    # The reported workload: 4-bit group-64 decode GEMV, 14336 x 4096, M = 1.
    main_work = Workload(session, "decode_4bit_g64_m1", 1, 14336, 4096, 4, 64)
    ms = main_work.time(hip, args.steps, args.warmup, use_graph)
    main_replays = main_work.replay_ms
    gpu_out = main_work.out.numpy()
    value = main_work.bytes / (ms * 1e-3) / 1e9
    roofline = roofline_gemv(main_work, ms, load_traffic(main_work.name))
    roofline["kernel_us_replays"] = [round(v * 1e3, 3) for v in main_replays]
    impl = main_work.implementation
    sets = main_work.sets
    # The floor of a launch that only reads the same weight bytes (no decode,
    # no activations, no output): the decode's distance from it is its overhead.
    floor_ms = main_work.time_read_floor(hip, args.steps, args.warmup)
    weight_bytes = main_work.bytes - main_work.M * main_work.K * 2 - main_work.M * main_work.N * 4
    roofline["read_floor"] = {"us": round(floor_ms * 1e3, 3), "weight_bytes": weight_bytes,
                              "GB/s": round(weight_bytes / (floor_ms * 1e-3) / 1e9, 1),
                              "frac_of_peak": round(weight_bytes / (floor_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              "decode_over_floor": round(ms / floor_ms, 4),
                              "kernel": "affon_rocm_read_floor (read_kernel: reads the packed words, scales and "
                                        "biases once, same rotation and graph replays)"}
    progress(f"{main_work.name}: {ms * 1e3:.3f} us per step ({roofline['frac']:.1%} of HBM peak); "
             f"read floor {floor_ms * 1e3:.3f} us")
    baseline = None
    extras = {"decode_4bit_g64_m1_end_to_end": end_to_end(main_work)}
    if args.cpu_seconds > 0:
        baseline = cpu_baseline(main_work, gpu_out, args.cpu_seconds)
        extras["cpu_baseline_all_cores"] = cpu_baseline(main_work, gpu_out, args.cpu_seconds / 2,
                                                        threads=_host_cores())
        progress(f"CPU baseline: {baseline['value']} GB/s on 1 thread, "
                 f"{extras['cpu_baseline_all_cores']['value']} GB/s on {extras['cpu_baseline_all_cores']['cores']}")
    main_work.release()

    def record(name, work, bound="hbm", keep=False):
        t = work.time(hip, args.steps, args.warmup, use_graph)
        entry = {"implementation": work.implementation, "us_per_step": round(t * 1e3, 3),
                 "us_per_step_replays": [round(v * 1e3, 3) for v in work.replay_ms],
                 "GB/s": round(work.bytes / (t * 1e-3) / 1e9, 1),
                 "TFLOP/s": round(work.flops / (t * 1e-3) / 1e12, 3)}
        if bound == "hbm":
            entry["hbm_frac"] = round(entry["GB/s"] / HBM_PEAK_GBS, 4)
        else:
            entry["mfma_frac"] = round(entry["TFLOP/s"] / BF16_MFMA_PEAK_TFLOPS, 4)
        extras[name] = entry
        progress(f"{name}: {entry['us_per_step']} us per step ({work.implementation})")
        if not keep:
            work.release()
        return t

    def with_cpu_baseline(name, work, unit, check_rows=512):
        """The restated CPU kernel beside a recorded line: one thread, about
        half the headline's sample time."""
        if args.cpu_seconds > 0:
            extras[name]["cpu_baseline"] = cpu_baseline(work, work.out.numpy(), args.cpu_seconds / 2, unit=unit,
                                                        check_rows=check_rows)
            progress(f"{name} CPU baseline: {extras[name]['cpu_baseline']['value']} {unit} on 1 thread")
        work.release()

    for M in (1, 2, 4, 8, 16):
        if want(f"decode_8bit_g64_m{M}"):
            work = Workload(session, f"decode_8bit_g64_m{M}", M, 14336, 4096, 8, 64)
            record(f"decode_8bit_g64_m{M}", work, keep=M == 1)
            if M == 1:
                with_cpu_baseline(f"decode_8bit_g64_m{M}", work, "GB/s")
    roofline_prefill = None
    for name, N, K in (("prefill_4bit_g64_m512_n14336_k4096", 14336, 4096),
                       ("prefill_4bit_g64_m512_n4096_k14336", 4096, 14336)):
        if want(name):
            work = Workload(session, name, 512, N, K, 4, 64, policy="approximate")
            t = record(name, work, bound="mfma", keep=True)
            extras[name]["numerical_policy"] = "approximate"
            if roofline_prefill is None:
                roofline_prefill = roofline_gemm(work, t, load_traffic(name))
                roofline_prefill["kernel_us_replays"] = extras[name]["us_per_step_replays"]
                if args.cpu_seconds > 0:
                    # The reference's CPU kernel on a sample of output columns (every activation row).
                    roofline_prefill["cpu_baseline"] = cpu_baseline(work, work.out.numpy(), args.cpu_seconds,
                                                                    unit="TFLOP/s")
                    progress(f"prefill CPU baseline: {roofline_prefill['cpu_baseline']['value']} TFLOP/s on 1 thread")
            work.release()
    # The same prefills under the default policy (backend_equivalent: no rounding of decoded weights).
    for name, N, K in (("prefill_4bit_g64_m512_n14336_k4096_backend_equivalent", 14336, 4096),
                       ("prefill_4bit_g64_m512_n4096_k14336_backend_equivalent", 4096, 14336)):
        if want(name):
            record(name, Workload(session, name, 512, N, K, 4, 64), bound="mfma")
            extras[name]["numerical_policy"] = "backend_equivalent"
    # Large prefill stress: 4-bit group 32, 2048 activation rows, both weight orientations.
    for name, N, K in (("prefill_4bit_g32_m2048_n28672_k8192", 28672, 8192),
                       ("prefill_4bit_g32_m2048_n8192_k28672", 8192, 28672)):
        if want(name):
            work = Workload(session, name, 2048, N, K, 4, 32, policy="approximate")
            record(name, work, bound="mfma", keep=True)
            extras[name]["numerical_policy"] = "approximate"
            if N == 28672:  # the CPU kernel on a prefix of the output columns (every activation row)
                with_cpu_baseline(name, work, "TFLOP/s", check_rows=16)
            else:
                work.release()
    # The same stress shapes under the default policy (the group-32 reassociated GEMM).
    for name, N, K in (("prefill_4bit_g32_m2048_n28672_k8192_backend_equivalent", 28672, 8192),
                       ("prefill_4bit_g32_m2048_n8192_k28672_backend_equivalent", 8192, 28672)):
        if want(name):
            record(name, Workload(session, name, 2048, N, K, 4, 32), bound="mfma")
            extras[name]["numerical_policy"] = "backend_equivalent"
    if want("decode_4bit_g64_m16"):
        record("decode_4bit_g64_m16", Workload(session, "decode_4bit_g64_m16", 16, 14336, 4096, 4, 64))
    for M in (1, 32):
        for fused in (False, True):
            name = f"llama8b_layer_4bit_g64_m{M}" + ("_fused" if fused else "")
            if want(name):
                extras[name] = layer_sequence(session, hip, M, args.steps // 10 or 1, args.warmup, fused=fused)
                progress(f"{name}: {extras[name]['us_per_layer']} us per layer")
    if want("decode_4bit_g64_f32_4096"):
        work = Workload(session, "decode_4bit_g64_f32_4096", 1, 4096, 4096, 4, 64, x_dtype="f32", p_dtype="f32")
        record("decode_4bit_g64_f32_4096", work, keep=True)
        extras["decode_4bit_g64_f32_4096"]["host_entry"] = host_entry(work)
        progress(f"decode_4bit_g64_f32_4096 through the host entry: "
                 f"{extras['decode_4bit_g64_f32_4096']['host_entry']['us_per_call']} us per call")
        with_cpu_baseline("decode_4bit_g64_f32_4096", work, "GB/s")
    if want("quantize_4bit_g32_28672x8192"):
        extras["quantize_4bit_g32_28672x8192"] = quantize_stress(session, hip, args.steps // 10 or 1, args.warmup)
        progress(f"quantize_4bit_g32_28672x8192: {extras['quantize_4bit_g32_28672x8192']['us_per_step']} us per step")
    if want("reference_8bit_g64_n2048_k1024"):
        extras["reference_8bit_g64_n2048_k1024"] = reference_workload(session, hip, args.steps, args.warmup)
        progress("reference_8bit_g64_n2048_k1024: " + ", ".join(
            f"{m}: {v['us_per_step']} us, {v['full_readback_us_per_call']} us with readback"
            for m, v in extras["reference_8bit_g64_n2048_k1024"].items()))
    if want("dequantize_4bit_g32_28672x8192"):
        extras["dequantize_4bit_g32_28672x8192"] = dequantize_stress(session, hip, args.steps // 10 or 1, args.warmup)
        progress(f"dequantize_4bit_g32_28672x8192: {extras['dequantize_4bit_g32_28672x8192']['us_per_step']} us per step")

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (Affon seeded generator: x seed 1 N(0,1) bf16, W seed 2 N(0,0.02) quantized on GPU)",
        "config": {"workload": "decode GEMV 4-bit group 64, W[14336,4096] u32-packed with bf16 scales/biases, "
                               "x bf16 [1,4096], f32 out", "M": 1, "N": 14336, "K": 4096, "bits": 4,
                   "group_size": 64, "implementation": impl, "launch": args.launch,
                   "weight_sets_rotated": sets, "replays": REPLAYS, "timing": "median of the replays"},
        "roofline": roofline,
        "roofline_prefill": roofline_prefill,
        "cpu_baseline": baseline,
        "extra": extras,
    }
    print(json.dumps(result), flush=True)
    session.dispose()
    return 0


if __name__ == "__main__":
    sys.exit(main())
