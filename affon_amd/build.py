"""Build recipe for the native library and the CPU oracle.

``build()`` compiles every HIP source under ``affon_amd/csrc`` for gfx950 into
``affon_amd/libaffon_rocm.so`` with one hipcc invocation per translation unit
(run in parallel) and a final link. It always rebuilds; loaders never build.
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess

ROOT = pathlib.Path(__file__).resolve().parent
REPO = ROOT.parent
CSRC = ROOT / "csrc"
LIBRARY = ROOT / "libaffon_rocm.so"
BUILD_DIR = REPO / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed FP32 instructions are disabled for all device code.
COMMON_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


# Files whose results must be bit-identical to the CPU oracle: no contraction
# of a*b+c into a fused multiply-add.
EXACT_FLAGS = {"quantize.hip": ["-ffp-contract=off"], "generic.hip": ["-ffp-contract=off"]}
# Decode-batch kernels whose MFMA results feed VALU scaling every step: the
# MFMAs write ordinary VGPRs, so no accumulator-register read
# (v_accvgpr_read) sits between each MFMA and its scaling. No kernel in
# these files needs scratch memory with it.
VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
UNIT_FLAGS = {**EXACT_FLAGS, **{f: VGPR_MFMA for f in ("gemv_mfma.hip", "vrow_b2.hip", "vrow_b4.hip", "vrow_b8.hip")}}


def _sources() -> list[pathlib.Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(source: pathlib.Path) -> pathlib.Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *UNIT_FLAGS.get(source.name, []), "-c", "-x", "hip", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")
    return obj


def build_library(verbose: bool = False) -> pathlib.Path:
    if shutil.which(HIPCC) is None and not pathlib.Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD_DIR.mkdir(exist_ok=True)
    sources = _sources()
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


def build_oracle(verbose: bool = False) -> pathlib.Path:
    oracle = REPO / "oracle"
    result = subprocess.run(["make", "-B", "-C", str(oracle)], capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{result.stdout}\n{result.stderr}")
    if verbose:
        print(f"built {oracle / 'liboracle.so'}")
    return oracle / "liboracle.so"


if __name__ == "__main__":
    build_library(verbose=True)
    build_oracle(verbose=True)
