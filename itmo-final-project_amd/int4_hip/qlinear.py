"""W4A16 linear layer and in-place conversion of a model's ``nn.Linear`` layers.

Interface kept from int4_triton/qlinear.py:8-68 (the names, defaults and
observable behaviour a caller or a checkpoint depends on):

* ``Int4Linear(in_features, out_features, group_size=128, bias=False,
  device=None)`` asserts ``in_features % group_size == 0`` and registers, in
  this order, the buffers ``qweight`` int32 [K/8, N], ``scales`` fp16 [K/G, N],
  ``zeros`` fp16 [K/G, N] and ``bias`` (or None), so ``state_dict`` keys,
  shapes and dtypes are the reference's and checkpoints load either way;
* ``from_linear``, ``forward`` (output in the activation dtype, bias added
  after the product), ``dequantize(dtype=bf16)``, ``extra_repr``;
* ``quantize_model_linears(model, group_size=128, skip=("lm_head",),
  fake=False)`` converts every ``nn.Linear`` whose dotted name contains none of
  the ``skip`` substrings; ``fake=True`` leaves the ``nn.Linear`` in place with
  its weight replaced by the dequantized int4 weight.
"""
from __future__ import annotations

from typing import Iterator

import torch
import torch.nn as nn

from .gemm import w4a16_matmul
from .quantize import dequantize_int4, dequantize_int4_ref, quantize_int4


class Int4Linear(nn.Module):
    """``y = x @ W_hat^T (+ bias)`` with W stored as packed int4 codes plus
    per-group fp16 scales and zero points; the product runs in the gfx950
    W4A16 kernels, on x's dtype (bf16/fp16) with fp32 accumulation."""

    def __init__(self, in_features: int, out_features: int, group_size: int = 128, bias: bool = False, device=None):
        super().__init__()
        assert in_features % group_size == 0
        self.in_features, self.out_features, self.group_size = in_features, out_features, group_size
        words, groups = in_features // 8, in_features // group_size
        # the registration order fixes the state_dict key order
        for name, shape, dtype in (("qweight", (words, out_features), torch.int32),
                                   ("scales", (groups, out_features), torch.float16),
                                   ("zeros", (groups, out_features), torch.float16)):
            self.register_buffer(name, torch.empty(shape, dtype=dtype, device=device))
        self.register_buffer("bias", torch.empty(out_features, device=device) if bias else None)

    @classmethod
    @torch.no_grad()
    def from_linear(cls, linear: nn.Linear, group_size: int = 128) -> "Int4Linear":
        """Quantize ``linear.weight`` on its GPU (group_size -1: one group per row)."""
        weight = linear.weight.detach()
        G = linear.in_features if group_size == -1 else group_size
        layer = cls(linear.in_features, linear.out_features, G, bias=False, device=weight.device)
        layer.qweight, layer.scales, layer.zeros = quantize_int4(weight.contiguous(), G)
        if linear.bias is not None:
            layer.bias = linear.bias.detach().clone()
        return layer

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = w4a16_matmul(x, self.qweight, self.scales, self.zeros)
        return out if self.bias is None else out + self.bias.to(out.dtype)

    def dequantize(self, dtype=torch.bfloat16) -> torch.Tensor:
        """W_hat [out_features, in_features] in ``dtype``, rounded once from the exact
        fp32 value.  Buffers on a GPU go through the HIP kernel; buffers on the
        CPU (e.g. a state dict loaded there) through the torch-op version, which
        gives the same bits -- the reference's method works on any device too."""
        bufs = (self.qweight, self.scales, self.zeros)
        if self.qweight.is_cuda:
            return dequantize_int4(*bufs, dtype)
        return dequantize_int4_ref(*bufs, dtype)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, group_size={self.group_size}"


def _iter_linears(model: nn.Module, skip) -> Iterator[tuple[nn.Module, str, nn.Linear]]:
    """``(owner, attribute, linear)`` for every ``nn.Linear`` attached to a module
    of ``model`` whose dotted path contains none of the ``skip`` substrings.

    Owners are visited depth-first in registration order, each module once even
    when it is reachable by several paths (its first path names it), which is
    the order and naming of ``model.named_modules()``."""
    seen: set[int] = set()

    def visit(owner: nn.Module, path: str):
        seen.add(id(owner))
        kids = list(owner.named_children())
        for attr, sub in kids:
            dotted = path + attr
            if isinstance(sub, nn.Linear) and not any(tag in dotted for tag in skip):
                yield owner, attr, sub
        for attr, sub in kids:
            if id(sub) not in seen:
                yield from visit(sub, path + attr + ".")

    yield from visit(model, "")


@torch.no_grad()
def quantize_model_linears(model: nn.Module, group_size: int = 128, skip=("lm_head",), fake: bool = False) -> nn.Module:
    """Convert ``model`` in place and return it.

    Every selected ``nn.Linear`` (see ``_iter_linears``) becomes an
    ``Int4Linear`` holding its quantized weight and bias.  With ``fake=True``
    the ``nn.Linear`` stays and its weight is overwritten by the dequantized
    int4 weight in its own dtype: the same numbers, multiplied by torch
    instead of the W4A16 kernels (the quality check the reference runs).
    All targets are collected before the first one is replaced.
    """
    for owner, attr, linear in list(_iter_linears(model, skip)):
        layer = Int4Linear.from_linear(linear, group_size)
        if fake:
            linear.weight.copy_(layer.dequantize(linear.weight.dtype))
        else:
            setattr(owner, attr, layer)
        del layer
    return model
