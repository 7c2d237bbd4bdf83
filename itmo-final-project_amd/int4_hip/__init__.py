"""int4_hip: MI355X-native W4A16 (int4 weights, bf16/fp16 activations) backend.

Drop-in for the reference package ``int4_triton`` (same public names,
arguments, storage layout and assertions; the submodules ``quantize``,
``gemm`` and ``qlinear`` hold what the reference's submodules of those names
hold), running hand-written gfx950 HIP kernels through the C-ABI library
``libint4_hip.so``.
"""
from . import quantize  # callable: quantize(w, group_size) == quantize_int4(w, group_size)
from .quantize import (dequantize_int4, dequantize_int4_ref, quantize_int4, quantize_int4_grouped,
                       quantize_int4_ref, unpack_int4_ref)
from .gemm import w4a16_matmul, w4a16_matmul_grouped, w16a16_matmul
from .qlinear import Int4Linear, quantize_model_linears

__all__ = [
    "quantize_int4",
    "quantize_int4_ref",
    "dequantize_int4_ref",
    "w4a16_matmul",
    "w16a16_matmul",
    "Int4Linear",
    "quantize_model_linears",
    # additions of this backend
    "quantize",
    "dequantize_int4",
    "unpack_int4_ref",
    "w4a16_matmul_grouped",
    "quantize_int4_grouped",
]
