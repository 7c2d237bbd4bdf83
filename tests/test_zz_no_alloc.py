"""GPU: ``w4a16_gemm_noalloc`` (the allocation-free variant of ``w4a16_gemm``,
split-K scratch in a fixed array inside the library) called through the C-ABI,
against ``w4a16_gemm`` (through ``int4_hip.w4a16_matmul``, whose workspace the
Python wrapper allocates).  Both take the same launch route for the same
shapes and alignment, so the outputs must be bit-identical.  Each case makes
two calls in a row, the second with a smaller problem, so that the second one
runs on the scratch contents the first one left: a route that reads stale
partials or counters shows up as a changed bit."""
import pytest
import torch

import int4_hip
from int4_hip import _lib
from _checks import DEV, _check, _decode, _weights
from _synth import randn

pytestmark = pytest.mark.gpu
_XDT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}


def _noalloc(x, qw, s, z):
    lib = _lib.load()
    M, K = x.shape
    N = qw.shape[1]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    rc = lib.w4a16_gemm_noalloc(x.data_ptr(), _XDT[x.dtype], M, N, K, x.stride(0), x.stride(1), qw.data_ptr(),
                                s.data_ptr(), z.data_ptr(), K // s.shape[0], y.data_ptr(), N,
                                torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "w4a16_gemm_noalloc")
    return y


# (M, N, K, G) pairs, the second call smaller than the first:
#   fp32 split-K partials (prefill kernel with 32/64-row tiles, M <= 64);
#   the M = 1 decode kernel's K split (long K: partials and arrival counters);
#   in-kernel split fixup with arrival counters (M = 1, group 16);
#   prefill split-K at M > 64; the prefill kernel's K split across
#   workgroups on 128 x 128 tiles (2 ranges, then 4); the decode kernel,
#   which uses no scratch; the skinny split-K kernel (strided activation rows)
PAIRS = [((64, 8192, 2048, 128), (40, 2048, 2048, 128)),
         ((1, 2048, 8192, 128), (1, 1024, 6144, 64)),
         ((1, 2048, 8192, 16), (1, 300, 2048, 16)),
         ((128, 2048, 8192, 128), (65, 512, 2048, 128)),
         ((1024, 2048, 8192, 128), (512, 2048, 8192, 128)),
         ((1, 8192, 2048, 128), (1, 512, 2048, 128)),
         ((48, 2048, 4104, 8), (20, 1024, 1032, 8))]


@pytest.mark.parametrize("first,second", PAIRS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_workspace_entry_point(first, second, dtype):
    for M, N, K, G in (first, second):
        print(f"[noalloc] M={M} N={N} K={K} G={G} {dtype}", flush=True)
        qw, s, z = _weights(N, K, G, seed=M + N + K + G)
        x = randn((M, K), seed=7 * M + 1, dtype=dtype).to(DEV)
        want = int4_hip.w4a16_matmul(x, qw, s, z)
        got = _noalloc(x, qw, s, z)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (M, N, K, G)
        _check(got, x, qw, s, z, ref_unrounded=False, exact_w=_decode(M, G, N, K))


def test_noalloc_strided_rows():
    # row stride not a multiple of 8: the skinny split-K kernel at M <= 16 too
    for M, N, K in ((16, 2048, 8192), (5, 512, 2048)):
        print(f"[noalloc strided] M={M} N={N} K={K}", flush=True)
        qw, s, z = _weights(N, K, 128, seed=N + K)
        x = randn((M, K + 4), seed=K).to(DEV)[:, :K]
        want = int4_hip.w4a16_matmul(x, qw, s, z)
        got = _noalloc(x, qw, s, z)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (M, N, K)


def test_noalloc_rejects_oversized_problem():
    lib = _lib.load()
    M, N, K, G = 2048, 2048, 28672, 128
    assert lib.w4a16_workspace_bytes(M, N, K, G) > _lib.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(16, dtype=torch.bfloat16, device=DEV)  # never read: rejected before launch
    rc = lib.w4a16_gemm_noalloc(x.data_ptr(), 0, M, N, K, K, 1, x.data_ptr(), x.data_ptr(), x.data_ptr(), G,
                                x.data_ptr(), N, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.ERR_WORKSPACE
    assert b"scratch" in lib.w4_last_error()
