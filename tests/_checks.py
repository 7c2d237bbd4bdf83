"""Tolerance checks of W4A16 products against the CPU oracle, shared by the
GPU tests.

Tolerances (stated per the task's floating-point bar):
* ``max |y - ref| <= 1e-2 * max |ref|`` with ref = x @ W_hat^T in float64 and
  W_hat rounded once to the activation dtype (the reference's own kernels
  round W_hat that way, int4_triton/gemm.py:139,211) -- the north-star bound;
* elementwise ``|y - ref| <= u_out * |ref| + 2**-20 * (|x| @ |W_hat|^T)``:
  one rounding of the output (u_out = 2**-8 bf16, 2**-11 fp16) plus fp32
  accumulation error;
* the reference's own check against the unrounded fp32 W_hat
  (tests/test_kernels.py:60): rtol 2e-2, atol 2e-2 * max |ref|.

The decode regime (M <= 64, or M <= 128 with N <= 4096 for a lone product
or for every product of a grouped call, except grouped calls of 49..64 rows
that the several-row kernel takes, see ``_rows``, and lone products of more
than 64 rows with K > 4096 that the prefill kernel splits, see
``_pf5_split``; group size >= 32, dense activation rows) applies
scales and zero points after the matrix-core sums, so it multiplies by the
exact fp32 W_hat instead of W_hat rounded to the activation dtype.  Its
elementwise check is against ref = x @ W_hat_fp32^T with
``|y - ref| <= u_out * |ref| + c * sum_k |x_k| s_{g(k)}``: the fp32 rounding of
the per-group sums of x_k * (OFF + QS q_k), whose terms are at most 143 |x_k|
(bf16: 128 + q) or 31 |x_k| (fp16: (1024 + 64 q) / 64), c = 2**-10 (bf16),
2**-12 (fp16).  A wrong zero point, scale, nibble or group is off by about
s * |sum_g x|, orders of magnitude above that slack.
"""
import numpy as np
import torch

import int4_hip
from oracle import w4a16_oracle as O
from _synth import bits_of, dtype_name, randn

DEV = "cuda"
U_OUT = {torch.bfloat16: 2.0**-8, torch.float16: 2.0**-11}


def _rows(M: int, G: int, N: int, K: int) -> bool:
    """True when a product of a grouped call of 49..64 rows on dense aligned
    rows fits the several-row kernel (w4_rows.hip, rows_plan), which rounds
    W_hat to the activation dtype: group >= 32, N a multiple of 4, K a
    multiple of 128 cut into at most 8 parts of at most 2048 (each a multiple
    of 128)."""
    if not (49 <= M <= 64 and G >= 32 and N >= 4 and N % 4 == 0 and K % 128 == 0):
        return False
    ks = 1
    while K // ks > 2048:
        ks *= 2
    return ks <= 8 and K % (128 * ks) == 0


def _pf5_split(M: int, G: int, N: int, K: int) -> bool:
    """True when a lone product of 65..128 dense aligned rows with K > 4096
    takes the prefill kernel's K-split launch (w4_prefill.hip, pf5_plan;
    W_hat rounded to the activation dtype): group >= 64, N a multiple of 64,
    K cut into ks <= 4 ranges of at most 2048 (each a multiple of 512), one
    workgroup per 64 x 64 tile and range within the MI355X's 256 CUs."""
    if not (64 < M <= 128 and G >= 64 and N % 64 == 0 and K > 4096):
        return False
    ks = 2
    while K // ks > 2048:
        ks *= 2
    return ks <= 4 and K % ks == 0 and (K // ks) % 512 == 0 and -(-M // 64) * (N // 64) * ks <= 256


def _decode(M: int, G: int, N: int = 1 << 30, K: int = 1 << 30) -> bool:
    """True when a lone w4a16_matmul takes the factored decode kernel (dense,
    aligned rows, group >= 32; exact fp32 W_hat): M <= 16 directly,
    17 <= M <= 64 as slices of at most 16 rows in one decode launch, and
    65 <= M <= 128 the same way when N <= 4096, unless the product takes the
    prefill kernel's K-split launch (``_pf5_split``)."""
    return G >= 32 and (M <= 64 or (M <= 128 and N <= 4096 and not _pf5_split(M, G, N, K)))


def _rows_workgroups(probs) -> int:
    """Workgroups of the several-row kernel's launch (rows_plan): 128-column
    tiles x K parts of at most 2048."""
    total = 0
    for N, K, G in probs:
        ks = 1
        while K // ks > 2048:
            ks *= 2
        total += -(-N // 128) * ks
    return total


def _grouped_exact(M: int, probs) -> bool:
    """The same for w4a16_matmul_grouped over problems (N, K, G), all with
    group >= 32 and dense rows: 49..64 rows take the several-row kernel when
    every problem fits it and the launch has at least three quarters of the
    MI355X's 256 CUs in workgroups, else the decode launch's row slices."""
    if M <= 48:
        return True
    if M <= 64:
        return not (all(_rows(M, G, N, K) for N, K, G in probs) and _rows_workgroups(probs) >= 192)
    return M <= 128 and all(N <= 4096 for N, K, G in probs)


def _check(out: torch.Tensor, x: torch.Tensor, qw, s, z, ref_unrounded: bool = True, exact_w=False):
    """exact_w: True for the decode kernels (exact fp32 W_hat), False for the
    kernels that round W_hat to the activation dtype, "either" where a grouped
    call may take either kind of launch (the result must pass one of the two
    bounds)."""
    if exact_w == "either":
        try:
            return _check(out, x, qw, s, z, ref_unrounded=False, exact_w=True)
        except AssertionError:
            return _check(out, x, qw, s, z, ref_unrounded=ref_unrounded, exact_w=False)
    xd = dtype_name(x.dtype)
    x2 = x.reshape(-1, x.shape[-1])
    qn, sn, zn = qw.cpu().numpy(), bits_of(s), bits_of(z)
    xa = np.abs(O.half_bits_to_f32(bits_of(x2), xd).astype(np.float64))
    if exact_w:
        ref = O.w4a16_matmul(bits_of(x2), xd, qn, sn, zn, w_hat_dtype="fp32")  # float64
        G = x2.shape[1] // sn.shape[0]
        s_abs = np.abs(O.half_bits_to_f32(sn, "fp16").astype(np.float64))
        slack = (2.0**-10 if x.dtype == torch.bfloat16 else 2.0**-12) * (xa @ np.repeat(s_abs, G, axis=0))
    else:
        ref = O.w4a16_matmul(bits_of(x2), xd, qn, sn, zn)               # float64
        w_hat = O.dequantize_int4(qn, sn, zn, xd).astype(np.float64)
        slack = 2.0**-20 * (xa @ np.abs(w_hat).T)
    y = out.reshape(-1, out.shape[-1]).float().cpu().numpy().astype(np.float64)
    assert y.shape == ref.shape
    err = np.abs(y - ref)
    scale = max(np.abs(ref).max(), 1e-30)
    assert err.max() <= 1e-2 * scale, f"max rel err {err.max() / scale:.3e}"
    bound = U_OUT[x.dtype] * np.abs(ref) + slack + 1e-30
    bad = err > bound
    assert not bad.any(), f"{int(bad.sum())} elements outside the elementwise bound, first {np.argwhere(bad)[0]}"
    if ref_unrounded:
        ref32 = O.w4a16_matmul(bits_of(x2), xd, qn, sn, zn, w_hat_dtype="fp32")
        torch.testing.assert_close(torch.from_numpy(y), torch.from_numpy(ref32), rtol=2e-2,
                                   atol=2e-2 * np.abs(ref32).max())


def _weights(N, K, G, seed, wdtype=torch.bfloat16):
    w = randn((N, K), seed=seed, sigma=0.02, dtype=wdtype).to(DEV)
    return int4_hip.quantize_int4(w, G)


