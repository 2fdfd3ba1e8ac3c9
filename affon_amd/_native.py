"""ctypes binding of ``libaffon_rocm.so`` (declared in include/affon_rocm.h).

Loading never builds and never falls back: if the library is missing the
caller gets a RuntimeError naming the build step.
"""
from __future__ import annotations

import ctypes
import pathlib

LIBRARY_PATH = pathlib.Path(__file__).resolve().with_name("libaffon_rocm.so")

OK, INVALID_SHAPE, CORE_FAILURE, UNSUPPORTED, HIP_ERROR = 0, 1, 2, 3, 4
F32, BF16, U32 = 0, 1, 2
IMPL_AUTO, IMPL_GENERIC, IMPL_GEMV, IMPL_GEMV_MFMA, IMPL_MFMA = 0, 1, 2, 3, 4
BACKEND_EQUIVALENT, EXACT_ONLY, APPROXIMATE = 0, 1, 2

# Every entry point the header declares, with its ctypes signature.
c_size_t, c_int, c_int32, c_int64, c_uint32, c_void_p, c_char_p = (
    ctypes.c_size_t, ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_void_p,
    ctypes.c_char_p)


class View(ctypes.Structure):
    _fields_ = [
        ("data", c_void_p),
        ("buffer_bytes", c_size_t),
        ("byte_offset", c_size_t),
        ("shape", c_int64 * 2),
        ("stride", c_int64 * 2),
        ("dtype", c_int32),
    ]


class QmmDesc(ctypes.Structure):
    _fields_ = [
        ("input", View),
        ("packed", View),
        ("scales", View),
        ("biases", View),
        ("output", c_void_p),
        ("output_bytes", c_size_t),
        ("bits", c_uint32),
        ("group_size", c_uint32),
        ("implementation", c_int32),
        ("numerical_policy", c_int32),
    ]


EPILOGUE_NONE, EPILOGUE_BIAS, EPILOGUE_SILU_GATE = 0, 1, 2


class Epilogue(ctypes.Structure):
    _fields_ = [
        ("kind", c_int32),
        ("bias", c_void_p),
        ("bias_bytes", c_size_t),
        ("bias_dtype", c_int32),
        ("up_packed", View),
        ("up_scales", View),
        ("up_biases", View),
    ]


class FloorGeometry(ctypes.Structure):
    """affon_rocm_floor_geometry: one read-floor launch shape."""
    _fields_ = [
        ("kib_per_wave", c_int32),
        ("threads", c_int32),
        ("valu_per_wave", c_int32),
        ("store_every", c_int32),
    ]


SIGNATURES = {
    "affon_rocm_device_count": (c_int, [ctypes.POINTER(c_int)]),
    "affon_rocm_session_create": (c_int, [c_int, ctypes.POINTER(c_void_p)]),
    "affon_rocm_session_destroy": (c_int, [c_void_p]),
    "affon_rocm_session_stream": (c_void_p, [c_void_p]),
    "affon_rocm_alloc": (c_int, [c_void_p, c_size_t, ctypes.POINTER(c_void_p)]),
    "affon_rocm_free": (c_int, [c_void_p, c_void_p]),
    "affon_rocm_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
    "affon_rocm_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
    "affon_rocm_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
    "affon_rocm_synchronize": (c_int, [c_void_p]),
    "affon_rocm_last_error": (c_char_p, []),
    "affon_rocm_quantized_matmul": (c_int, [c_void_p, ctypes.POINTER(QmmDesc)]),
    "affon_rocm_quantized_matmul_noalloc": (c_int, [c_void_p, ctypes.POINTER(QmmDesc)]),
    "affon_rocm_read_floor": (c_int, [c_void_p, ctypes.POINTER(c_void_p), ctypes.POINTER(ctypes.c_uint64), c_int,
                                      c_void_p]),
    "affon_rocm_read_floor_geometry": (c_int, [c_void_p, c_void_p, ctypes.c_uint64, c_void_p, ctypes.c_uint64,
                                               ctypes.POINTER(FloorGeometry)]),
    "affon_rocm_empty_launch": (c_int, [c_void_p, c_uint32, c_uint32]),
    "affon_rocm_kernel_supports": (c_int, [ctypes.POINTER(QmmDesc), c_char_p, ctypes.POINTER(c_int)]),
    "affon_rocm_quantized_matmul_select": (c_int, [ctypes.POINTER(QmmDesc), c_char_p, c_size_t]),
    "affon_rocm_quantized_matmul_fused": (c_int, [c_void_p, ctypes.POINTER(QmmDesc), ctypes.POINTER(Epilogue)]),
    "affon_rocm_quantized_matmul_fused_select": (c_int, [ctypes.POINTER(QmmDesc), ctypes.POINTER(Epilogue), c_char_p,
                                                         c_size_t]),
    "affon_rocm_quantized_matmul_grouped": (c_int, [c_void_p, ctypes.POINTER(QmmDesc), ctypes.POINTER(Epilogue),
                                                    c_size_t]),
    "affon_rocm_quantized_matmul_grouped_select": (c_int, [ctypes.POINTER(QmmDesc), ctypes.POINTER(Epilogue), c_size_t,
                                                           c_char_p, c_size_t]),
    "affon_rocm_quantized_matmul_capabilities": (c_char_p, []),
    "compute_core_run_quantized_matmul_f32": (c_int, [
        c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t,
        c_size_t, c_size_t, c_size_t, c_size_t, c_size_t]),
    "affon_rocm_quantize": (c_int, [c_void_p, c_void_p, c_int32, c_int64, c_int64, c_uint32, c_uint32,
                                    c_void_p, c_void_p, c_void_p, c_int32]),
    "affon_rocm_dequantize": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int64,
                                      c_uint32, c_uint32, c_void_p, c_int32]),
    "affon_rocm_rms_norm": (c_int, [c_void_p, c_void_p, c_int32, c_int64, c_int64, ctypes.c_float, c_void_p]),
    "affon_rocm_softmax": (c_int, [c_void_p, c_void_p, c_int32, c_int64, c_int64, c_void_p]),
    "affon_rocm_index_select": (c_int, [c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int32, c_void_p, c_int64,
                                        c_void_p]),
}

_LIB: ctypes.CDLL | None = None


class NativeError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def load() -> ctypes.CDLL:
    """Returns the loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"{LIBRARY_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the rocm backend has no CPU fallback)")
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


def last_error() -> str:
    raw = load().affon_rocm_last_error()
    return raw.decode() if raw else ""


def check(status: int, what: str = "") -> None:
    if status != OK:
        message = last_error() or f"status {status}"
        raise NativeError(status, f"{what}: {message}" if what else message)
