"""CPU oracle for the W4A16 quantize + GEMM path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker (or as the timed CPU port of
the reference's torch CPU path).  The product package ``int4_hip`` never
imports it; its entry points raise if the HIP library is missing.

This is a numpy restatement of the reference's pure-torch functions in
``int4_triton/quantize.py`` (homomorfism/itmo-final-project), op for op and
dtype for dtype, so that its outputs are bit-identical to them:

* ``quantize_int4``   <- ``quantize_int4_ref``   (int4_triton/quantize.py:102-117)
* ``unpack_int4``     <- ``unpack_int4_ref``     (int4_triton/quantize.py:120-125)
* ``dequantize_int4`` <- ``dequantize_int4_ref`` (int4_triton/quantize.py:128-135)
* ``w4a16_matmul``    <- the reference's torch "dequantize, then matmul" path
  (tests/test_kernels.py:56-57, 93, 109): ``x.float() @ w_hat.float().t()``.

Tensors cross this module as numpy arrays.  Half-precision values travel as
their raw 16-bit patterns (``uint16``) because numpy has no bfloat16 type:
``dtype`` arguments are the strings ``"bf16"``, ``"fp16"`` or ``"fp32"``.

How each function is pinned (checked by tests/test_oracle.py):

* quantize_int4: golden vectors written by the reference's own
  ``quantize_int4_ref`` (tests/golden/make_golden.py), including the
  degenerate groups no closed form fixes (fp16-underflowing scales, NaN/Inf,
  exact .5 ties, signed zeros, G=-1, fp16 input, int32 wrap of nibble 7);
  closed forms (constant-0.5 group, all-zero group); the invariants
  q, zero in [0, 15] and |w_hat - w| <= scale/2; and planted mistakes that
  the golden vectors must catch.
* unpack_int4 / dequantize_int4: golden vectors from the reference, a
  bit-by-bit brute force with Python ints, and the exact-product argument
  ((q - z) * s is exact in fp32, so one rounding to the target dtype).
* w4a16_matmul: torch's CPU ``F.linear`` on the same dequantized weights
  (a library routine) and the closed-form case y = 2**23
  (tests/test_kernels.py:100-110).
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_bits_to_f32",
    "f32_to_bf16_bits",
    "f16_bits_to_f32",
    "f32_to_f16_bits",
    "half_bits_to_f32",
    "f32_to_half_bits",
    "quantize_int4",
    "unpack_int4",
    "dequantize_int4",
    "w4a16_matmul",
    "round_to_dtype",
]

_SHIFTS = np.arange(0, 32, 4, dtype=np.uint32)


# ----------------------------------------------------------------- bit helpers
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even.

    Same rule as torch's CPU float->bfloat16 cast (c10::BFloat16
    round_to_nearest_even): NaN becomes the quiet NaN 0x7FC0.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    bias = np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))
    out = ((b + bias) >> np.uint32(16)).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), out).astype(np.uint16)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> float16 bit patterns (IEEE round to nearest even, subnormals kept)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def half_bits_to_f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(bits)
    if dtype == "fp16":
        return f16_bits_to_f32(bits)
    raise ValueError(f"unsupported half dtype {dtype!r}")


def f32_to_half_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return f32_to_bf16_bits(x)
    if dtype == "fp16":
        return f32_to_f16_bits(x)
    raise ValueError(f"unsupported half dtype {dtype!r}")


def round_to_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values once to ``dtype`` and return them as float32."""
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    return half_bits_to_f32(f32_to_half_bits(x, dtype), dtype)


def _f32_to_i32_like_torch_cpu(q: np.ndarray) -> np.ndarray:
    """float32 -> int32 the way x86 truncating conversion does it.

    q is already clamped to [0, 15] or NaN; NaN converts to INT32_MIN
    (0x80000000), which is what torch's CPU ``.to(torch.int32)`` yields
    (pinned by the NaN-group golden vectors).
    """
    out = np.zeros(q.shape, dtype=np.int32)
    finite = ~np.isnan(q)
    out[finite] = q[finite].astype(np.int32)
    out[~finite] = np.int32(-(2**31))
    return out


# ----------------------------------------------------------------- quantize
def quantize_int4(w_bits: np.ndarray, dtype: str = "bf16", group_size: int = 128):
    """Group-wise asymmetric RTN int4 quantization of W[N, K].

    Restates int4_triton/quantize.py:102-117 op for op:
      wg    = w.float().reshape(N, K/G, G)                       (:107)
      wmax  = amax(-1).clamp(min=0); wmin = amin(-1).clamp(max=0) (:108-109)
      scale = (wmax - wmin) / 15   -- true IEEE fp32 division      (:110)
      scale = where(scale == 0, 1, scale) -> fp16 -> fp32          (:111)
      zero  = clamp(floor(-wmin / scale + 0.5), 0, 15)             (:112)
      q     = clamp(floor(w / scale + 0.5) + zero, 0, 15) -> int32 (:113)
      packed word = sum_i q[8*k8 + i] << 4*i, int32 wrap-around    (:114-116)

    Args:
      w_bits: uint16 [N, K] bit patterns of a bf16 or fp16 weight (``dtype``).
      group_size: power of two, multiple of 8 dividing K; -1 means K (:105-106).
    Returns:
      (qweight int32 [K/8, N], scales uint16 fp16 bits [K/G, N],
       zeros uint16 fp16 bits [K/G, N]), all C-contiguous.
    """
    w_bits = np.asarray(w_bits, dtype=np.uint16)
    N, K = w_bits.shape
    G = K if group_size == -1 else group_size
    assert K % G == 0 and G % 8 == 0, (K, G)
    wg = half_bits_to_f32(w_bits, dtype).reshape(N, K // G, G)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        wmax = np.maximum(wg.max(axis=-1), np.float32(0))
        wmin = np.minimum(wg.min(axis=-1), np.float32(0))
        scale = (wmax - wmin) / np.float32(15)
        scale = np.where(scale == 0, np.float32(1), scale).astype(np.float32)
        scale = scale.astype(np.float16).astype(np.float32)
        zero = np.clip(np.floor(-wmin / scale + np.float32(0.5)), np.float32(0), np.float32(15))
        qf = np.floor(wg / scale[..., None] + np.float32(0.5)) + zero[..., None]
        qf = np.clip(qf, np.float32(0), np.float32(15)).astype(np.float32)
    q = _f32_to_i32_like_torch_cpu(qf).reshape(N, K // 8, 8)
    packed = (q.view(np.uint32) << _SHIFTS).sum(axis=-1, dtype=np.uint32).view(np.int32)
    qweight = np.ascontiguousarray(packed.T)
    scales = np.ascontiguousarray(f32_to_f16_bits(scale).T)
    zeros = np.ascontiguousarray(f32_to_f16_bits(zero).T)
    return qweight, scales, zeros


# ----------------------------------------------------------------- unpack / dequant
def unpack_int4(qweight: np.ndarray) -> np.ndarray:
    """int32 [K/8, N] -> int32 [N, K] with values in [0, 15] (quantize.py:120-125)."""
    qweight = np.asarray(qweight, dtype=np.int32)
    K8, N = qweight.shape
    q = (qweight.T[:, :, None].view(np.uint32) >> _SHIFTS) & np.uint32(0xF)
    return q.reshape(N, K8 * 8).astype(np.int32)


def dequantize_int4(qweight, scales_bits, zeros_bits, dtype: str = "fp16") -> np.ndarray:
    """W_hat[N, K] = round_once_to_dtype((q - z) * s), computed in fp32.

    Restates quantize.py:128-135.  (q - z) * s is exact in fp32 (a <=5-bit
    integer times an 11-bit significand), so the only rounding is the final
    cast.  Returns float32 values that are exactly representable in ``dtype``.
    """
    q = unpack_int4(qweight).astype(np.float32)
    N, K = q.shape
    G = K // scales_bits.shape[0]
    s = np.repeat(f16_bits_to_f32(scales_bits).T, G, axis=1)
    z = np.repeat(f16_bits_to_f32(zeros_bits).T, G, axis=1)
    with np.errstate(invalid="ignore", over="ignore"):
        w = (q - z) * s
    return round_to_dtype(w, dtype)


# ----------------------------------------------------------------- GEMM
def w4a16_matmul(x_bits: np.ndarray, x_dtype: str, qweight, scales_bits, zeros_bits,
                 w_hat_dtype: str | None = None, accumulate: str = "f64") -> np.ndarray:
    """y[M, N] = x[M, K] @ W_hat[N, K]^T, returned unrounded (float64 or float32).

    ``w_hat_dtype`` defaults to the activation dtype: the reference's kernels
    round the dequantized weight once to the activation dtype before the
    product (int4_triton/gemm.py:139, 147 and :211-212).  Pass "fp32" for the
    unrounded weight used by tests/test_kernels.py:56-57.  ``accumulate="f64"``
    gives a near-exact reference; "f32" mirrors torch's fp32 matmul.
    """
    x = half_bits_to_f32(np.asarray(x_bits, dtype=np.uint16), x_dtype)
    w_hat = dequantize_int4(qweight, scales_bits, zeros_bits, w_hat_dtype or x_dtype)
    if accumulate == "f64":
        return x.astype(np.float64) @ w_hat.astype(np.float64).T
    return x @ w_hat.T
