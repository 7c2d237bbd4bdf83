"""Y = X @ W_hat^T with X in bf16/fp16 and W given as packed int4 (W4A16), on gfx950.

Same public entry point, regime boundaries and error behaviour as the
reference (int4_triton/gemm.py:223-317):

  * M <= 16:       decode kernel, one launch, no workspace (group sizes >= 32
                   and dense rows; else split-K with a fixed-order reduce);
  * 17 <= M <= 64: the same decode kernel in one launch, the rows cut into
                   slices of 16 (dense, 16-byte aligned rows, group >= 32);
                   otherwise split-K with fp32 partials and a fixed-order
                   reduce kernel;
  * M > 64:        tiled MFMA GEMM writing the output dtype directly, split
                   over K (same partials and reduce) for shapes with too few
                   output tiles to fill the chip; a lone product with
                   M <= 128 and N <= 4096 on dense rows takes the decode
                   kernel's row slices instead (up to eight).

The kernels are hand-written HIP (itmo-final-project_amd/csrc); the split
counts come from a static table inside the library, so results are
bit-identical from run to run and process to process (the reference picks its
tiles by timing, gemm.py:161-168).  Every call launches on the caller's
current stream and never synchronizes.  The split-K workspace is one
persistent zero-initialised buffer per (device, stream), allocated on the first
call and never freed (the kernels leave its counters zero); a call captured on a
stream that has none uses one buffer per capture stream, shared by every graph
captured there (see ``_with_workspace``), so graphs can be captured with or
without a warm-up call on the capture stream.
"""
from __future__ import annotations

import threading
from typing import Sequence

import torch
import torch.nn.functional as F

from . import _lib

_XDT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}
SMALL_M = 64  # reference regime boundary (int4_triton/gemm.py:17)


def _check_weight(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, K: int):
    assert qweight.dtype == torch.int32 and qweight.dim() == 2
    assert scales.dtype == torch.float16 and zeros.dtype == torch.float16
    assert scales.shape == zeros.shape and scales.shape[1] == qweight.shape[1]
    G = K // scales.shape[0]
    assert G * scales.shape[0] == K and G >= 8 and (G & (G - 1)) == 0, (K, scales.shape)
    return G


_WS: dict = {}       # (device, stream) -> persistent zero-initialised workspace
_CAP_WS: dict = {}   # (device, capture stream) -> workspace of calls captured there
_WS_RETIRED: list = []  # outgrown buffers, still referenced by captured graphs
_WS_LOCK = threading.Lock()
_COUNTER_BYTES = 65536  # W4_WORKSPACE_COUNTER_BYTES


def _stream_workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    """The persistent zero-initialised workspace of (device, stream), grown to
    ``nbytes`` outside graph capture; None if it is missing or too small while
    the stream is capturing.

    The kernels leave its counter area zero, so it is reused as is; buffers are
    never freed, so graphs that captured one keep a valid pointer.  Calls on
    one stream are ordered, so sharing it between them is safe."""
    key = (device.index, stream)
    with _WS_LOCK:
        ws = _WS.get(key)
        if ws is not None and ws.numel() >= nbytes:
            return ws
        if torch.cuda.is_current_stream_capturing():
            return None
        if ws is not None:
            _WS_RETIRED.append(ws)
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WS[key] = ws
        return ws


def _capture_workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Workspace for a call captured on a stream that has no (large enough)
    persistent one: one buffer per (device, capture stream), taken from the
    graph's private pool the first time and replaced only by a larger one, so
    capturing many graphs on one stream (torch's default capture stream among
    them) keeps at most one live buffer per size it had to grow to."""
    key = (device.index, stream)
    with _WS_LOCK:
        ws = _CAP_WS.get(key)
        if ws is None or ws.numel() < nbytes:
            if ws is not None:
                _WS_RETIRED.append(ws)  # graphs captured before still use it
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _CAP_WS[key] = ws
        return ws


def _with_workspace(device: torch.device, stream: int, nbytes: int, launch) -> int:
    """``launch(ptr, nbytes)`` with a workspace of at least ``nbytes`` (``nbytes``
    is the library's size query, an upper bound over every route the call may
    take).

    A graph may be captured on a stream that never ran an eager call (torch's
    own capture stream, as ``torch.cuda.graph(g)`` without a stream and
    ``triton.testing.do_bench_cudagraph`` use).  There the call takes the
    capture stream's buffer (``_capture_workspace``) and records, ahead of the
    product, a fill kernel (no memset node) that zeroes its counter area: the
    buffer is shared by every graph captured on that stream and its memory is
    never written at capture time, so each replay starts from zero counters
    whichever graph ran last.  Graphs that share a capture stream share its
    buffer, so their replays must be ordered (as calls on one stream are)."""
    if nbytes == 0:
        return launch(None, 0)
    ws = _stream_workspace(device, stream, nbytes)
    if ws is None:
        ws = _capture_workspace(device, stream, nbytes)
        ws[:_COUNTER_BYTES].zero_()
    return launch(ws.data_ptr(), ws.numel())


_WS_BYTES: dict = {}


def _ws_bytes(lib, M: int, N: int, K: int, G: int) -> int:
    """Workspace size of one product; a pure function of the shape, memoised."""
    key = (M, N, K, G)
    b = _WS_BYTES.get(key)
    if b is None:
        b = _WS_BYTES[key] = lib.w4a16_workspace_bytes(M, N, K, G)
    return b


def _gemm_call(lib, x2, dt, M, N, K, qweight, scales, zeros, G, y, device):
    # torch's raw current-stream query is a fraction of the cost of
    # torch.cuda.current_stream(); the library reads the current device (for
    # its CU count), which the caller has made the tensors' device
    stream = torch._C._cuda_getCurrentRawStream(device.index)
    return _with_workspace(device, stream, _ws_bytes(lib, M, N, K, G), lambda ws, nb: lib.w4a16_gemm(
        x2.data_ptr(), dt, M, N, K, x2.stride(0), x2.stride(1),
        qweight.data_ptr(), scales.data_ptr(), zeros.data_ptr(), G,
        y.data_ptr(), N, ws, nb, stream))


def w4a16_matmul(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor) -> torch.Tensor:
    """x[..., K] (bf16/fp16) @ W^T, W given as packed int4 (see quantize.py). Returns x.dtype [..., N].

    Mirrors int4_triton/gemm.py:303-309 (assertions included).
    """
    assert x.dtype in (torch.bfloat16, torch.float16)
    K = x.shape[-1]
    assert qweight.shape[0] * 8 == K, (qweight.shape, K)
    G = _check_weight(qweight, scales, zeros, K)
    dev = x.device
    assert x.is_cuda and qweight.device == dev and scales.device == dev and zeros.device == dev
    N = qweight.shape[1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    qweight, scales, zeros = qweight.contiguous(), scales.contiguous(), zeros.contiguous()
    y = torch.empty((M, N), dtype=x.dtype, device=dev)
    if M == 0 or N == 0:
        return y.reshape(*x.shape[:-1], N)
    lib = _lib.load()
    if torch._C._cuda_getDevice() == dev.index:
        rc = _gemm_call(lib, x2, _XDT[x.dtype], M, N, K, qweight, scales, zeros, G, y, dev)
    else:
        with torch.cuda.device(dev):
            rc = _gemm_call(lib, x2, _XDT[x.dtype], M, N, K, qweight, scales, zeros, G, y, dev)
    if rc:
        _lib.check(rc, "w4a16_gemm")
    return y.reshape(*x.shape[:-1], N)


def w4a16_matmul_grouped(xs: Sequence[torch.Tensor], weights: Sequence[tuple],
                         out: Sequence[torch.Tensor] | None = None) -> list[torch.Tensor]:
    """Several independent products ``xs[i] @ W_i^T``, fused into one launch.

    ``weights[i]`` is a ``(qweight, scales, zeros)`` triple.  All ``xs[i]`` share
    dtype and the leading size M.  For M <= 64, and up to M = 128 when every
    problem has N <= 4096, every problem runs in one decode launch (rows in
    slices of 16 above M = 16; group sizes >= 32); otherwise
    products of one shared activation tensor (q/k/v, gate/up: pass the same
    tensor) run as one prefill launch when the library's plan allows it, else
    one launch each.  This fuses the per-linear launches
    of a transformer block; it has no single counterpart in the reference.
    """
    assert 1 <= len(xs) == len(weights) <= _lib.MAX_GROUPED
    dt = xs[0].dtype
    assert dt in _XDT
    dev = xs[0].device
    M = xs[0].reshape(-1, xs[0].shape[-1]).shape[0]
    assert M >= 1
    probs = (_lib.Problem * len(xs))()
    outs, keep, dense = [], [], {}
    for i, (x, (qw, s, z)) in enumerate(zip(xs, weights)):
        assert x.dtype == dt and x.device == dev
        K = x.shape[-1]
        # one dense, 16-byte aligned copy per distinct input (shared inputs stay shared)
        x2 = dense.get(id(x))
        if x2 is None:
            x2 = x.reshape(-1, K).contiguous()
            if x2.data_ptr() % 16:
                x2 = x2.clone()
            dense[id(x)] = x2
        assert x2.shape[0] == M and qw.shape[0] * 8 == K
        G = _check_weight(qw, s, z, K)
        qw, s, z = qw.contiguous(), s.contiguous(), z.contiguous()
        N = qw.shape[1]
        y = out[i] if out is not None else torch.empty((M, N), dtype=dt, device=dev)
        assert y.shape == (M, N) and y.is_contiguous() and y.dtype == dt
        probs[i] = _lib.Problem(x2.data_ptr(), qw.data_ptr(), s.data_ptr(), z.data_ptr(), y.data_ptr(), N, K, G, 0)
        keep += [x2, qw, s, z]
        outs.append(y)
    lib = _lib.load()

    def call():
        stream = torch._C._cuda_getCurrentRawStream(dev.index)
        nbytes = lib.w4a16_grouped_workspace_bytes(probs, len(xs), M)
        return _with_workspace(dev, stream, nbytes, lambda ws, nb: lib.w4a16_gemm_grouped(
            probs, len(xs), _XDT[dt], M, ws, nb, stream))

    if torch._C._cuda_getDevice() == dev.index:
        rc = call()
    else:
        with torch.cuda.device(dev):
            rc = call()
    if rc:
        _lib.check(rc, "w4a16_gemm_grouped")
    return [y.reshape(*x.shape[:-1], y.shape[-1]) for x, y in zip(xs, outs)]


def grouped_workspace_bytes(xs: Sequence[torch.Tensor], weights: Sequence[tuple]) -> int:
    """Workspace bytes ``w4a16_matmul_grouped(xs, weights)`` uses (0 if none)."""
    M = xs[0].reshape(-1, xs[0].shape[-1]).shape[0]
    probs = (_lib.Problem * len(xs))()
    for i, (x, (qw, s, z)) in enumerate(zip(xs, weights)):
        K = x.shape[-1]
        probs[i] = _lib.Problem(x.data_ptr(), qw.data_ptr(), s.data_ptr(), z.data_ptr(), x.data_ptr(), qw.shape[1],
                                K, K // s.shape[0], 0)
    return _lib.load().w4a16_grouped_workspace_bytes(probs, len(xs), M)


def w16a16_matmul(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x[..., K] @ w[N, K]^T with full-precision weights (the reference's W16 baseline,
    int4_triton/gemm.py:312-317).

    On MI355X this baseline is the vendor library (hipBLASLt through
    ``F.linear``); no hand-written kernel is provided for it.
    """
    assert x.dtype == w.dtype and x.dtype in (torch.bfloat16, torch.float16)
    return F.linear(x, w)
