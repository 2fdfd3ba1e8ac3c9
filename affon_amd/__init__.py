"""MI355X (gfx950) backend for Affon's affine group-wise weight-quantized linear path.

The product is the native library ``libaffon_rocm.so`` (C ABI in
``include/affon_rocm.h``); this package is the host-side mirror of the
reference's ``affon:ops`` / Session surface over that ABI.
"""
from .core import Executable, FormalTensor, Program, Session, Tensor, TensorSpec, program
from .ops import (add, dequantize, fused_plan, grouped_plan, index_select, mul, quantize, quantized_linear,
                  quantized_matmul, quantized_matmul_grouped, quantized_matmul_into, quantized_silu_gate, rms_norm,
                  selected_implementation, silu, slice, softmax, transpose)

__all__ = [
    "Executable", "FormalTensor", "Program", "Session", "Tensor", "TensorSpec", "program",
    "add", "dequantize", "fused_plan", "grouped_plan", "index_select", "mul", "quantize", "quantized_linear",
    "quantized_matmul", "quantized_matmul_grouped", "quantized_matmul_into", "quantized_silu_gate", "rms_norm",
    "selected_implementation", "silu", "slice", "softmax", "transpose",
]
