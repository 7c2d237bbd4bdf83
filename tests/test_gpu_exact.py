"""Bit-exact parity of every W4A16 route on exact-arithmetic inputs.

Inputs are built so that no fp32 operation any route performs can round:

* ``qweight``: random nibbles;
* ``scales``: powers of two 2**e, e in [-4, -1] (fp16, exact);
* ``zeros``: integers in [0, 15] (fp16);
* activations: integers in [-A, A] (A = 8), exact in bf16 and fp16.

Then W_hat = (q - z) * s is a 4-bit integer times a power of two, exact in
bf16, fp16 and fp32, so rounding W_hat to the activation dtype (the
reference's kernels, int4_triton/gemm.py:139,211) and keeping it in fp32 (the
decode kernels' factored form) give the same values.  Every product x * W_hat
and every partial sum, in any order and any split of K, is a multiple of
2**-4 of magnitude at most K * A * 15 * 2**-1, i.e. it needs at most
log2(K * A * 15 * 2**3) < 24 significant bits (checked by ``_bound_ok``), so
fp32 accumulation is exact.  The factored decode kernels also form sums of
x * (OFF + QS q) over a correction interval of at most 512 k before applying
the scale; those are integers below 512 * A * (OFF + 15 QS) <= 2**23 for both
dtypes.  The only rounding left is the final cast of the exact value to the
output dtype (round to nearest even), so every correct route must return
exactly ``round(x @ W_hat^T)`` -- whatever its tiling, K split, summation
order or W_hat rounding.  The oracle computes that value in float64 and
rounds it once (oracle/w4a16_oracle.py).

Two kinds of activation rows.  Dense rows (uniform integers) make every
k count: a dropped k slice, a swapped nibble pair, a wrong group, scale or
zero, or a lost K part moves most outputs by several output ulps.  Sparse rows
(two +-1 entries per row) make every output exactly representable even in
bf16, so one wrong weight at those k changes the bits of every column it
feeds; at bf16's 8-bit significand a dense row could round such a
single-weight error away.  The tolerance tests in test_gpu_gemm.py cannot see
single-weight mistakes at all.

Covered: the four distinct Llama-3.2-1B linear shapes (bench_gemm.py:18-26 of
the reference) at M in {1, 3, 8, 16, 24, 64, 65, 128, 512, 2048}, bf16 and
fp16, lone products and grouped calls (the 7-linear block with one input per
linear, and q/k/v + gate/up sharing their input); the per-channel case
G = K (int4_triton/quantize.py:72-73, qlinear.py:25-27) at K = 2048 and 8192;
the untied 128256 x 2048 lm_head (eval_llama.py:208-211) at M = 1 and 512 on
a column subset; and the side routes (group sizes below 32, strided or
misaligned activation rows, K not a multiple of 64, odd N).
"""
from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

import int4_hip
from oracle import w4a16_oracle as O
from _checks import DEV
from _synth import bits_of

pytestmark = pytest.mark.gpu

A = 8                 # |x| <= A
E_MIN, E_MAX = -4, -1  # scales 2**e
LLAMA = [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192)]  # (N, K)
BLOCK = [(2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (8192, 2048), (8192, 2048), (2048, 8192)]
MS = [1, 3, 8, 16, 24, 64, 65, 128, 512, 2048]
_TDT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _bound_ok(K: int, amp: int = A) -> None:
    # every partial sum is a multiple of 2**E_MIN below K * amp * 15 * 2**E_MAX
    span = K * amp * 15 * 2.0 ** (E_MAX - E_MIN)
    assert span < 2.0**24, f"K={K}: partial sums would need {np.log2(span):.1f} bits"
    # factored decode sums over at most 512 k of x * (OFF + QS q), fp16 worst case
    assert 512 * amp * (1024 + 15 * 64) < 2.0**24


@functools.lru_cache(maxsize=64)
def _exact_weights_np(N: int, K: int, G: int, seed: int):
    """(qweight int32 [K/8, N], scale bits fp16 [K/G, N], zero bits fp16 [K/G, N])."""
    rng = np.random.default_rng(seed)
    nib = rng.integers(0, 16, size=(K // 8, N, 8), dtype=np.uint32)
    words = np.zeros((K // 8, N), np.uint32)
    for i in range(8):
        words |= nib[..., i] << np.uint32(4 * i)
    e = rng.integers(E_MIN, E_MAX + 1, size=(K // G, N))
    s_bits = ((e + 15) << 10).astype(np.uint16)  # 2**e in fp16
    z_bits = rng.integers(0, 16, size=(K // G, N)).astype(np.float16).view(np.uint16)
    return words.view(np.int32), s_bits, z_bits


@functools.lru_cache(maxsize=64)
def _exact_x_np(M: int, K: int, seed: int, amp: int = A, kind: str = "dense") -> np.ndarray:
    """Integer activations as float32 (exact in bf16 and fp16).

    dense: uniform in [-amp, amp].  sparse: two entries of +-1 per row at
    random k (distinct per row), zeros elsewhere, so every output is the sum
    or difference of two W_hat values -- a multiple of 2**-4 below 16, exact
    in bf16 -- and a wrong weight at those k changes every column's bits."""
    rng = np.random.default_rng(seed)
    if kind == "dense":
        return rng.integers(-amp, amp + 1, size=(M, K)).astype(np.float32)
    x = np.zeros((M, K), np.float32)
    for m in range(M):
        k = rng.choice(K, 2, replace=False)
        x[m, k] = rng.choice([-1.0, 1.0], 2)
    return x


def _to_dev_weights(N, K, G, seed):
    qw, s, z = _exact_weights_np(N, K, G, seed)
    return (torch.from_numpy(qw).to(DEV),
            torch.from_numpy(s.view(np.int16)).view(torch.float16).to(DEV),
            torch.from_numpy(z.view(np.int16)).view(torch.float16).to(DEV))


def _to_dev_x(x: np.ndarray, dt: str) -> torch.Tensor:
    return torch.from_numpy(x).to(_TDT[dt]).to(DEV)


def _w_hat_T(N, K, G, seed, cols=None) -> np.ndarray:
    """Exact W_hat^T [K, n] in float64 (optionally a subset of columns)."""
    qw, s, z = _exact_weights_np(N, K, G, seed)
    if cols is not None:
        qw, s, z = qw[:, cols], s[:, cols], z[:, cols]
    w = O.dequantize_int4(qw, s, z, "fp32").astype(np.float64)  # exact (q - z) * s
    return np.ascontiguousarray(w.T)


@functools.lru_cache(maxsize=32)
def _exact_y(M, N, K, G, wseed, xseed, amp=A, kind="dense") -> np.ndarray:
    """Exact x @ W_hat^T in float64 (every value exactly representable in fp32)."""
    y = _exact_x_np(M, K, xseed, amp, kind).astype(np.float64) @ _w_hat_T(N, K, G, wseed)
    assert np.array_equal(y.astype(np.float32).astype(np.float64), y), "inputs are not exact-arithmetic"
    return y


def _expect_bits(y: np.ndarray, dt: str) -> np.ndarray:
    return O.f32_to_half_bits(y.astype(np.float32), dt)


def _assert_bits(out: torch.Tensor, y: np.ndarray, dt: str, what: str) -> None:
    got = bits_of(out.reshape(-1, out.shape[-1]))
    want = _expect_bits(y, dt)
    assert got.shape == want.shape, (got.shape, want.shape)
    bad = got != want
    if bad.any():
        i, j = np.argwhere(bad)[0]
        g = O.half_bits_to_f32(got[i:i + 1, j:j + 1], dt)[0, 0]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outputs differ from the exact value, "
                             f"first at ({i}, {j}): got {g!r}, exact {y[i, j]!r}")


# ------------------------------------------------------------ lone products
@pytest.mark.parametrize("kind", ["dense", "sparse"])
@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("NK", LLAMA)
@pytest.mark.parametrize("M", MS)
def test_exact_lone(M, NK, dt, kind):
    N, K = NK
    G = 128
    _bound_ok(K)
    print(f"[exact lone] M={M} N={N} K={K} {dt} {kind}", flush=True)
    qw, s, z = _to_dev_weights(N, K, G, seed=N + K)
    x = _to_dev_x(_exact_x_np(M, K, M + K, A, kind), dt)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    _assert_bits(out, _exact_y(M, N, K, G, N + K, M + K, A, kind), dt, f"M={M} N={N} K={K} {dt} {kind}")


# ------------------------------------------------------------ grouped calls
@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("M", MS)
def test_exact_grouped_block(M, dt):
    """The 7 linears of a decoder block in one grouped call, one input each."""
    print(f"[exact grouped block] M={M} {dt}", flush=True)
    G = 128
    ws, xs, ys = [], [], []
    for i, (N, K) in enumerate(BLOCK):
        _bound_ok(K)
        ws.append(_to_dev_weights(N, K, G, seed=N + K))  # q/o, k/v, gate/up share weights per shape
        xs.append(_to_dev_x(_exact_x_np(M, K, seed=1000 + 7 * M + i), dt))
        ys.append(_exact_y(M, N, K, G, N + K, 1000 + 7 * M + i))
    outs = int4_hip.w4a16_matmul_grouped(xs, ws)
    for i, (out, y) in enumerate(zip(outs, ys)):
        _assert_bits(out, y, dt, f"block linear {i} M={M} {dt}")


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("M", MS)
def test_exact_grouped_shared_input(M, dt):
    """q/k/v and gate/up, each set sharing one input (the shared-activation
    prefill launch above 64 rows, the decode launch below)."""
    print(f"[exact grouped shared] M={M} {dt}", flush=True)
    G, K = 128, 2048
    xn = _exact_x_np(M, K, seed=2000 + M)
    x = _to_dev_x(xn, dt)
    for Ns in ((2048, 512, 512), (8192, 8192)):
        ws = [_to_dev_weights(N, K, G, seed=3000 + N + i) for i, N in enumerate(Ns)]
        outs = int4_hip.w4a16_matmul_grouped([x] * len(Ns), ws)
        for i, (N, out) in enumerate(zip(Ns, outs)):
            _assert_bits(out, _exact_y(M, N, K, G, 3000 + N + i, 2000 + M), dt, f"shared {Ns}[{i}] M={M} {dt}")


# ------------------------------------------------------------ per-channel (G = K)
@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("K", [2048, 8192])
@pytest.mark.parametrize("M", [1, 16, 64, 128, 2048])
def test_exact_per_channel(M, K, dt):
    """group_size=-1 (one group per column, G = K), as Int4Linear.from_linear
    passes it through (qlinear.py:25-27) and w4a16_matmul derives it
    (gemm.py:308): lone and in a grouped call."""
    N = 2048
    _bound_ok(K)
    print(f"[exact G=K] M={M} K={K} {dt}", flush=True)
    qw, s, z = _to_dev_weights(N, K, K, seed=5000 + K)
    assert s.shape == (1, N)
    x = _to_dev_x(_exact_x_np(M, K, seed=5100 + M), dt)
    y = _exact_y(M, N, K, K, 5000 + K, 5100 + M)
    _assert_bits(int4_hip.w4a16_matmul(x, qw, s, z), y, dt, f"G=K lone M={M} K={K}")
    other = _to_dev_weights(512, 2048, 128, seed=5200)
    xo = _to_dev_x(_exact_x_np(M, 2048, seed=5300 + M), dt)
    outs = int4_hip.w4a16_matmul_grouped([x, xo], [(qw, s, z), other])
    _assert_bits(outs[0], y, dt, f"G=K grouped M={M} K={K}")
    _assert_bits(outs[1], _exact_y(M, 512, 2048, 128, 5200, 5300 + M), dt, f"G=K grouped partner M={M}")


# ------------------------------------------------------------ lm_head
@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("M", [1, 512])
def test_exact_lm_head(M, dt):
    """The untied, quantized 128256 x 2048 lm_head (eval_llama.py:198,208-211),
    the widest product of the model: all columns computed, a subset of 1536
    (the first and last 512 and 512 random ones) checked bit for bit."""
    N, K, G = 128256, 2048, 128
    print(f"[exact lm_head] M={M} {dt}", flush=True)
    qw, s, z = _to_dev_weights(N, K, G, seed=6000)
    xn = _exact_x_np(M, K, seed=6100 + M)
    out = int4_hip.w4a16_matmul(_to_dev_x(xn, dt), qw, s, z)
    assert out.shape == (M, N)
    rng = np.random.default_rng(6200)
    cols = np.unique(np.concatenate([np.arange(512), N - 512 + np.arange(512),
                                     rng.choice(np.arange(512, N - 512), 512, replace=False)]))
    y = xn.astype(np.float64) @ _w_hat_T(N, K, G, 6000, cols)
    _assert_bits(out[:, torch.from_numpy(cols).to(DEV)], y, dt, f"lm_head M={M} {dt}")


# ------------------------------------------------------------ side routes
# group sizes below 32 (full-dequantization kernels and split-K + reduce),
# strided rows (split-K skinny / general prefill kernels), a misaligned row
# start (generic decode kernel), K not a multiple of 64 (register-staged
# prefill), odd N (partial tiles), long K with small groups
SIDE = [  # M, N, K, G, layout
    (1, 73, 256, 8, "dense"), (1, 2048, 8192, 16, "dense"), (1, 2048, 2048, 128, "offset"),
    (3, 2048, 2048, 128, "offset"), (5, 2048, 8192, 128, "strided"), (16, 300, 2048, 16, "dense"),
    (16, 3072, 14336, 128, "strided"), (24, 520, 8192, 32, "dense"), (40, 2048, 8192, 32, "strided"),
    (64, 300, 4096, 8, "dense"), (65, 96, 520, 8, "dense"), (130, 73, 512, 64, "dense"),
    (200, 300, 512, 64, "strided"), (512, 2048, 2048, 16, "dense"), (777, 1000, 1024, 32, "strided"),
    (2048, 96, 520, 8, "dense"), (300, 8192, 2048, 128, "offset"),
    (33, 73, 2048, 64, "dense"), (100, 300 + 2, 1024, 128, "dense"),  # generic decode kernel in 16-row slices
    (700, 1000, 1024, 64, "dense"), (2048, 520, 2048, 128, "dense"),  # pf3 with a partial last column tile
    (700, 2048, 8192, 64, "dense"),   # pf5 128 x 128 tiles, K in two ranges, partial last row tile
    (1900, 2048, 8192, 128, "dense"),  # pf3 two K splits finished in the kernel, partial last row tile
]


# the sixteen-row slice kernel: a partial last slice, K split into 2 / 4 / 8
# parts (finished by the last part to arrive), every group class, column
# tiles not a multiple of 8 (the tail of the XCD-ordered workgroup blocks),
# lone and grouped, repeated calls
SLICES = [  # M, N, K, G
    (17, 520, 4096, 32), (33, 96, 8192, 64), (40, 2048, 6144, 128), (63, 72, 16384, 256),
    (100, 4096, 2048, 128), (128, 200, 8192, 512), (9, 8, 12288, 64), (120, 1000, 4096, 32),
]


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("M,N,K,G", SLICES)
def test_exact_row_slices(M, N, K, G, dt):
    _bound_ok(K)
    print(f"[exact slices] M={M} N={N} K={K} G={G} {dt}", flush=True)
    qw, s, z = _to_dev_weights(N, K, G, seed=8000 + N + K + G)
    xn = _exact_x_np(M, K, seed=8100 + M)
    x = _to_dev_x(xn, dt)
    y = _exact_y(M, N, K, G, 8000 + N + K + G, 8100 + M)
    for _ in range(2):
        _assert_bits(int4_hip.w4a16_matmul(x, qw, s, z), y, dt, f"slices lone M={M} N={N} K={K} G={G}")
    other = _to_dev_weights(512, 2048, G, seed=8200)
    xo = _to_dev_x(_exact_x_np(M, 2048, seed=8300 + M), dt)
    outs = int4_hip.w4a16_matmul_grouped([x, xo], [(qw, s, z), other])
    _assert_bits(outs[0], y, dt, f"slices grouped M={M} N={N} K={K} G={G}")
    _assert_bits(outs[1], _exact_y(M, 512, 2048, G, 8200, 8300 + M), dt, f"slices grouped partner M={M}")


# grouped calls of 49..64 rows: the several-row kernel (every weight
# dequantized once for all rows) when every problem fits it and the launch
# fills most of the chip (each case has a wide filler problem for that) -- a
# partial last 128-column tile, K parts of 2048 finished by the last part to
# arrive (2, 4, 8 parts), short K, every group class; with one problem it
# does not take (N not a multiple of 4) the whole call goes to the decode
# kernel's slices
ROWS = [  # M, [(N, K, G), ...]
    (49, [(1000, 4096, 32), (136, 2048, 64), (22528, 2048, 128)]),
    (57, [(520, 8192, 256), (4, 16384, 1024), (21504, 2048, 32)]),
    (64, [(2048, 8192, 128), (1032, 1024, 64), (8, 128, 32), (16384, 2048, 128)]),
    (60, [(2048, 2048, 128), (73, 256, 32), (22528, 2048, 128)]),
]


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("M,probs", ROWS)
def test_exact_rows_grouped(M, probs, dt):
    print(f"[exact rows] M={M} {probs} {dt}", flush=True)
    ws, xs, ys = [], [], []
    for i, (N, K, G) in enumerate(probs):
        _bound_ok(K)
        ws.append(_to_dev_weights(N, K, G, seed=9000 + N + K + G))
        xs.append(_to_dev_x(_exact_x_np(M, K, seed=9100 + M + i), dt))
        ys.append(_exact_y(M, N, K, G, 9000 + N + K + G, 9100 + M + i))
    for _ in range(2):  # repeat: arrival counters left at zero, partial tiles rewritten
        for i, (out, y) in enumerate(zip(int4_hip.w4a16_matmul_grouped(xs, ws), ys)):
            _assert_bits(out, y, dt, f"rows grouped M={M} problem {i} {probs[i]} {dt}")


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("M,N,K,G,layout", SIDE)
def test_exact_side_routes(M, N, K, G, layout, dt):
    _bound_ok(K)
    print(f"[exact side] M={M} N={N} K={K} G={G} {layout} {dt}", flush=True)
    qw, s, z = _to_dev_weights(N, K, G, seed=7000 + N + K + G)
    xn = _exact_x_np(M, K, seed=7100 + M)
    if layout == "dense":
        x = _to_dev_x(xn, dt)
    elif layout == "strided":  # every other element of a wider tensor
        wide = np.zeros((M, 2 * K), np.float32)
        wide[:, ::2] = xn
        x = _to_dev_x(wide, dt)[:, ::2]
    else:  # rows start 2 bytes past a 16-byte boundary (dense, misaligned)
        flat = np.zeros(M * K + 1, np.float32)
        flat[1:] = xn.reshape(-1)
        x = _to_dev_x(flat, dt)[1:].view(M, K)
        assert x.data_ptr() % 16 != 0
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    y = _exact_y(M, N, K, G, 7000 + N + K + G, 7100 + M)
    _assert_bits(out, y, dt, f"side M={M} N={N} K={K} G={G} {layout} {dt}")
    again = int4_hip.w4a16_matmul(x, qw, s, z)
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))
