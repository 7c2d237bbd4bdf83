"""Pure-torch reference functions kept for API compatibility with int4_triton.

The reference package exports ``quantize_int4_ref``, ``unpack_int4_ref`` and
``dequantize_int4_ref`` (int4_triton/quantize.py:102-135) so that callers can
check the GPU kernels against torch ops.  They are provided here with the same
names and semantics, written with torch ops.  Nothing in this package's
compute path calls them: ``quantize_int4``, ``w4a16_matmul`` and
``Int4Linear`` always run the HIP kernels.
"""
from __future__ import annotations

import torch


def quantize_int4_ref(w: torch.Tensor, group_size: int = 128):
    """Torch-op group-wise asymmetric int4 quantization (int4_triton/quantize.py:102-117)."""
    N, K = w.shape
    if group_size == -1:
        group_size = K
    grouped = w.float().reshape(N, K // group_size, group_size)
    hi = grouped.amax(-1).clamp(min=0)
    lo = grouped.amin(-1).clamp(max=0)
    scale = (hi - lo) / 15
    scale = torch.where(scale == 0, torch.ones_like(scale), scale).half().float()
    zero = torch.floor(-lo / scale + 0.5).clamp(0, 15)
    q = (torch.floor(grouped / scale[..., None] + 0.5) + zero[..., None]).clamp(0, 15).to(torch.int32)
    q = q.reshape(N, K // 8, 8)
    shifts = torch.arange(0, 32, 4, device=w.device, dtype=torch.int32)
    packed = (q << shifts).sum(-1, dtype=torch.int32)
    return packed.t().contiguous(), scale.half().t().contiguous(), zero.half().t().contiguous()


def unpack_int4_ref(qweight: torch.Tensor) -> torch.Tensor:
    """int32 [K/8, N] -> int32 [N, K] with values in [0, 15] (int4_triton/quantize.py:120-125)."""
    K8, N = qweight.shape
    shifts = torch.arange(0, 32, 4, device=qweight.device, dtype=torch.int32)
    return ((qweight.t()[:, :, None] >> shifts) & 0xF).reshape(N, K8 * 8)


def dequantize_int4_ref(qweight, scales, zeros, dtype=torch.float16) -> torch.Tensor:
    """W_hat[N, K] in fp32 rounded once to ``dtype`` (int4_triton/quantize.py:128-135)."""
    q = unpack_int4_ref(qweight).float()
    N, K = q.shape
    G = K // scales.shape[0]
    s = scales.t().repeat_interleave(G, dim=1).float()
    z = zeros.t().repeat_interleave(G, dim=1).float()
    return ((q - z) * s).to(dtype)
