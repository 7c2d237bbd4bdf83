"""Group-wise asymmetric int4 quantization of a 2-D weight W[N, K] on gfx950.

Same API, storage layout and error behaviour as the reference
(int4_triton/quantize.py:1-96):

    scale = (max - min) / 15 rounded to fp16 (1 for an all-zero group),
    zero  = clamp(floor(-min / scale + 0.5), 0, 15),
    q     = clamp(floor(w / scale + 0.5) + zero, 0, 15);
    qweight int32 [K/8, N] (nibble i of word k8 = row 8*k8 + i),
    scales, zeros fp16 [K/G, N].

``quantize_int4`` runs the HIP kernel (bit-exact with the reference's torch
implementation); ``dequantize_int4`` runs the HIP dequantize kernel.  The
``*_ref`` functions live in :mod:`int4_hip.reference`.
"""
from __future__ import annotations

import torch

from . import _lib

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16, torch.float32: _lib.DTYPE_FP32}


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def quantize_int4(w: torch.Tensor, group_size: int = 128):
    """Quantize W[N, K] (fp16 or bf16, on the GPU) -> (qweight int32 [K/8, N],
    scales fp16 [K/G, N], zeros fp16 [K/G, N]).

    Mirrors int4_triton/quantize.py:67-96, including its assertions.
    """
    assert w.dim() == 2 and w.is_cuda
    assert w.dtype in (torch.float16, torch.bfloat16)
    N, K = w.shape
    if group_size == -1:
        group_size = K
    assert K % group_size == 0 and group_size % 8 == 0
    assert group_size > 0 and (group_size & (group_size - 1)) == 0, "group_size must be a power of 2"

    qweight = torch.empty((K // 8, N), dtype=torch.int32, device=w.device)
    scales = torch.empty((K // group_size, N), dtype=torch.float16, device=w.device)
    zeros = torch.empty_like(scales)
    lib = _lib.load()
    with torch.cuda.device(w.device):
        rc = lib.w4_quantize(w.data_ptr(), _DT[w.dtype], N, K, w.stride(0), w.stride(1), group_size,
                             qweight.data_ptr(), scales.data_ptr(), zeros.data_ptr(), _stream_ptr(w.device))
    _lib.check(rc, "w4_quantize")
    return qweight, scales, zeros


def dequantize_int4(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                    dtype=torch.float16) -> torch.Tensor:
    """W_hat[N, K] = round_once_to_dtype((q - z) * s) on the GPU.

    Same result as int4_triton/quantize.py:128-135 (``dequantize_int4_ref``).
    """
    assert qweight.is_cuda and scales.is_cuda and zeros.is_cuda
    assert qweight.dtype == torch.int32 and scales.dtype == torch.float16 and zeros.dtype == torch.float16
    assert dtype in _DT, dtype
    K8, N = qweight.shape
    K = K8 * 8
    assert scales.shape == zeros.shape and scales.shape[1] == N and K % scales.shape[0] == 0
    G = K // scales.shape[0]
    qweight, scales, zeros = qweight.contiguous(), scales.contiguous(), zeros.contiguous()
    out = torch.empty((N, K), dtype=dtype, device=qweight.device)
    lib = _lib.load()
    with torch.cuda.device(qweight.device):
        rc = lib.w4_dequantize(qweight.data_ptr(), scales.data_ptr(), zeros.data_ptr(), N, K, G, _DT[dtype],
                               out.data_ptr(), _stream_ptr(qweight.device))
    _lib.check(rc, "w4_dequantize")
    return out
