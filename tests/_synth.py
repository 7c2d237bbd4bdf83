"""Seeded synthetic inputs shared by the tests (CPU generation, so the oracle
and the GPU kernels see identical bits)."""
from __future__ import annotations

import numpy as np
import torch


def bits_of(t: torch.Tensor) -> np.ndarray:
    """Raw 16-bit patterns of a bf16/fp16 tensor as a numpy uint16 array."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def dtype_name(dt: torch.dtype) -> str:
    return {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dt]


def randn(shape, seed: int, sigma: float = 1.0, dtype=torch.bfloat16) -> torch.Tensor:
    """N(0, sigma) drawn in fp32 from a CPU generator, rounded once to ``dtype``."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * sigma).to(dtype)


def assert_bits_equal_nan_aware(a: np.ndarray, b: np.ndarray, dtype: str, msg: str = ""):
    """Bit equality, except that any two NaNs compare equal (sign/payload free)."""
    from oracle.w4a16_oracle import half_bits_to_f32

    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if dtype == "fp32":
        fa, fb = a.view(np.float32), b.view(np.float32)
        ia, ib = a.view(np.uint32), b.view(np.uint32)
    else:
        fa, fb = half_bits_to_f32(a, dtype), half_bits_to_f32(b, dtype)
        ia, ib = a.view(np.uint16), b.view(np.uint16)
    nan_a, nan_b = np.isnan(fa), np.isnan(fb)
    assert np.array_equal(nan_a, nan_b), f"{msg}: NaN positions differ"
    diff = (ia != ib) & ~nan_a
    assert not diff.any(), f"{msg}: {int(diff.sum())} bit mismatches, first at {np.argwhere(diff)[0]}"
