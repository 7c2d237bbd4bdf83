"""Group-wise asymmetric int4 quantization of a 2-D weight W[N, K].

Public names, defaults, storage layout and assertions are those of the
reference module int4_triton/quantize.py (:67-135), so that module's callers
(``from int4_triton.quantize import unpack_int4_ref`` included) can import
this one instead.

Storage (int4_triton/quantize.py:8-12): ``qweight`` int32 [K/8, N] with
nibble i (bits 4i..4i+3) of word (k8, n) holding row 8*k8 + i of W^T;
``scales`` and ``zeros`` fp16 [K/G, N], the zeros integer-valued in [0, 15].
Per group of G consecutive k of one output column n:

    scale = fp16((max(w, 0) - min(w, 0)) / 15), an exact-zero range -> 1
    zero  = clamp(floor(-min(w, 0) / scale + 0.5), 0, 15)
    q     = clamp(floor(w / scale + 0.5) + zero, 0, 15)
    w_hat = (q - zero) * scale          (exact in fp32, then one rounding)

Two implementations live here:

* ``quantize_int4`` / ``dequantize_int4``: the product path, hand-written
  gfx950 kernels behind the C-ABI (``w4_quantize`` / ``w4_dequantize``).
  They raise if the library is missing; there is no fallback.
* ``quantize_int4_ref`` / ``unpack_int4_ref`` / ``dequantize_int4_ref``:
  torch-op versions on whatever device the tensors live (CPU included), the
  counterparts of int4_triton/quantize.py:102-135, which the reference's users
  call to check the kernels.  They are bit-exact with the kernels on CPU and
  GPU tensors alike: every step is an IEEE operation whose result torch
  fixes on both (division by a 15.0 tensor, never a multiply by its
  reciprocal; floor of x + 0.5; NaN-propagating extremes; NaN codes mapped to
  INT32_MIN before the integer cast).
"""
from __future__ import annotations

import sys
import types

import torch

from . import _lib

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16, torch.float32: _lib.DTYPE_FP32}
_NIBBLE_SHIFTS = tuple(range(0, 32, 4))


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _resolve_group(K: int, group_size: int) -> int:
    return K if group_size == -1 else group_size


# ----------------------------------------------------------------- HIP path
def quantize_int4(w: torch.Tensor, group_size: int = 128):
    """Quantize W[N, K] (fp16/bf16 on the GPU, any strides) with the gfx950 kernel.

    Returns fresh contiguous ``(qweight int32 [K/8, N], scales fp16 [K/G, N],
    zeros fp16 [K/G, N])``; ``group_size=-1`` means one group per row (G = K).
    Misuse raises ``AssertionError`` as int4_triton/quantize.py:69-75 does.
    """
    assert w.dim() == 2 and w.is_cuda
    assert w.dtype in (torch.float16, torch.bfloat16)
    N, K = w.shape
    G = _resolve_group(K, group_size)
    assert K % G == 0 and G % 8 == 0
    assert G > 0 and (G & (G - 1)) == 0, "group_size must be a power of 2"

    qweight = torch.empty((K // 8, N), dtype=torch.int32, device=w.device)
    scales = torch.empty((K // G, N), dtype=torch.float16, device=w.device)
    zeros = torch.empty_like(scales)
    lib = _lib.load()
    with torch.cuda.device(w.device):
        rc = lib.w4_quantize(w.data_ptr(), _DT[w.dtype], N, K, w.stride(0), w.stride(1), G,
                             qweight.data_ptr(), scales.data_ptr(), zeros.data_ptr(), _stream_ptr(w.device))
    _lib.check(rc, "w4_quantize")
    return qweight, scales, zeros


def quantize_int4_grouped(ws, group_size: int = 128):
    """Quantize several weights W_i[N_i, K_i] (one dtype, on one GPU) as
    ``quantize_int4`` does, bit for bit, in one kernel launch when every
    weight has dense 16-byte-aligned rows (and the group size is <= 512);
    else one launch per weight.  Returns a list of ``(qweight, scales,
    zeros)`` triples.  No single counterpart in the reference: it fuses the
    per-linear ``quantize_int4`` calls of one block
    (int4_triton/qlinear.py:55-68)."""
    ws = list(ws)
    assert 1 <= len(ws) <= _lib.MAX_GROUPED
    dt, dev = ws[0].dtype, ws[0].device
    assert dt in (torch.float16, torch.bfloat16)
    probs = (_lib.QuantProblem * len(ws))()
    outs = []
    for i, w in enumerate(ws):
        assert w.dim() == 2 and w.is_cuda and w.dtype == dt and w.device == dev
        N, K = w.shape
        G = _resolve_group(K, group_size)
        assert K % G == 0 and G % 8 == 0
        assert G > 0 and (G & (G - 1)) == 0, "group_size must be a power of 2"
        qweight = torch.empty((K // 8, N), dtype=torch.int32, device=dev)
        scales = torch.empty((K // G, N), dtype=torch.float16, device=dev)
        zeros = torch.empty_like(scales)
        probs[i] = _lib.QuantProblem(w.data_ptr(), qweight.data_ptr(), scales.data_ptr(), zeros.data_ptr(), N, K,
                                     w.stride(0), w.stride(1), group_size, 0)
        outs.append((qweight, scales, zeros))
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.w4_quantize_grouped(probs, len(ws), _DT[dt], _stream_ptr(dev))
    _lib.check(rc, "w4_quantize_grouped")
    return outs


def dequantize_int4(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                    dtype=torch.float16) -> torch.Tensor:
    """W_hat[N, K] = one rounding to ``dtype`` of the exact fp32 (q - z) * s, on the GPU.

    Bit-identical to ``dequantize_int4_ref`` on the same buffers.
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


# ------------------------------------------------------- torch-op versions
def quantize_int4_ref(w: torch.Tensor, group_size: int = 128):
    """Torch-op quantization on ``w``'s device; same outputs as ``quantize_int4``.

    Counterpart of int4_triton/quantize.py:102-117.  The extremes are taken
    with ``amax``/``amin`` (a NaN anywhere in a group makes its scale, zero
    and codes follow IEEE NaN arithmetic), the code of every weight is found
    in fp32 and the eight codes of a word are OR-ed into place, so a code
    >= 8 in nibble 7 sets the int32 sign bit.
    """
    N, K = w.shape
    G = _resolve_group(K, group_size)
    groups = w.float().unflatten(1, (K // G, G))                 # [N, K/G, G]
    top = torch.clamp(groups.amax(dim=2), min=0.0)
    bottom = torch.clamp(groups.amin(dim=2), max=0.0)
    # divide by a tensor on w's device: torch turns GPU division by a host
    # scalar into a multiply by its fp32 reciprocal, which differs from the
    # correctly rounded quotient in the last bit for some ranges
    fifteen = torch.full((), 15.0, dtype=torch.float32, device=w.device)
    step = (top - bottom) / fifteen
    step = step.masked_fill(step == 0.0, 1.0).to(torch.float16)  # the stored scale
    step32 = step.float()
    zp = torch.clamp(torch.floor(bottom.neg() / step32 + 0.5), 0.0, 15.0)
    codes = torch.floor(groups / step32.unsqueeze(2) + 0.5).add_(zp.unsqueeze(2))
    codes = codes.clamp_(0.0, 15.0)
    # a NaN code (a group holding NaN or both infinities) becomes INT32_MIN, the
    # value of the x86 truncating conversion the reference's CPU path applies;
    # the GPU conversion would give 0
    codes = codes.masked_fill_(codes.isnan(), -2.0**31)
    codes = codes.to(torch.int32).reshape(N, K // 8, 8)
    words = codes[..., 0].clone()
    for i in range(1, 8):
        words.bitwise_or_(codes[..., i] << _NIBBLE_SHIFTS[i])
    return (words.transpose(0, 1).contiguous(), step.transpose(0, 1).contiguous(),
            zp.to(torch.float16).transpose(0, 1).contiguous())


def unpack_int4_ref(qweight: torch.Tensor) -> torch.Tensor:
    """Codes of a packed ``qweight`` int32 [K/8, N] as int32 [N, K], values 0..15.

    Counterpart of int4_triton/quantize.py:120-125 (layout of :9).
    """
    K8, N = qweight.shape
    cols = qweight.transpose(0, 1)                               # [N, K/8]
    planes = [(cols >> s) & 0xF for s in _NIBBLE_SHIFTS]         # code of row 8*k8 + i
    return torch.stack(planes, dim=2).reshape(N, K8 * 8)


def dequantize_int4_ref(qweight, scales, zeros, dtype=torch.float16) -> torch.Tensor:
    """W_hat[N, K] as the exact fp32 (q - z) * s rounded once to ``dtype``.

    Counterpart of int4_triton/quantize.py:128-135 (default dtype fp16, as there).
    """
    codes = unpack_int4_ref(qweight).float()                     # [N, K]
    N, K = codes.shape
    n_groups = scales.shape[0]
    codes = codes.view(N, n_groups, K // n_groups)
    s = scales.float().transpose(0, 1).unsqueeze(2)              # [N, K/G, 1]
    z = zeros.float().transpose(0, 1).unsqueeze(2)
    return ((codes - z) * s).reshape(N, K).to(dtype)


class _CallableModule(types.ModuleType):
    """This module can be called: ``int4_hip.quantize(w, group_size=128)`` is
    ``quantize_int4``.  The package attribute ``quantize`` is thus both the
    quantizer and the submodule the reference's callers import names from."""

    def __call__(self, w: torch.Tensor, group_size: int = 128):
        return quantize_int4(w, group_size)


sys.modules[__name__].__class__ = _CallableModule
