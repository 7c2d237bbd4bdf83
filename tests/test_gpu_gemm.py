"""GPU parity of the W4A16 GEMM regimes against the CPU oracle, with the
tolerances stated in tests/_checks.py (max relative error <= 1e-2, an
elementwise bound from the output rounding and fp32 accumulation, and the
reference's own rtol/atol check), plus bit-identical repeat runs, graph
capture and workspace handling."""
import numpy as np
import pytest
import torch

import int4_hip
from _checks import DEV, _check, _decode, _grouped_exact, _weights
from _synth import randn

pytestmark = pytest.mark.gpu
# int4_triton tests/test_kernels.py:47-60 (M x shape x dtype grid)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1, 7, 24, 128, 512, 2048])
@pytest.mark.parametrize("NK", [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192), (300, 256)])
def test_w4a16_matmul(M, NK, dtype):
    N, K = NK
    print(f"[gemm] M={M} N={N} K={K} {dtype}", flush=True)
    qw, s, z = _weights(N, K, 128, seed=N + K, wdtype=torch.float16)
    x = randn((M, K), seed=M, dtype=dtype).to(DEV)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    assert out.dtype == dtype and out.shape == (M, N)
    _check(out, x, qw, s, z, exact_w=_decode(M, 128, N, K))


def _poison_workspace():
    """NaN into the scratch part of the current stream's persistent workspace
    (past the counter area, which must stay zero), so that a kernel reading a
    partial it did not write this call shows up as NaN or a changed bit."""
    from int4_hip import gemm as _gemm
    ws = _gemm._WS.get((torch.cuda.current_device(), torch.cuda.current_stream().cuda_stream))
    if ws is not None:
        scratch = ws[65536:]
        scratch[: scratch.numel() // 4 * 4].view(torch.float32).fill_(float("nan"))


# split-K regime over the block's shapes (all four distinct N x K of
# bench_gemm.py:18-26) and the three group sizes
@pytest.mark.parametrize("G", [128, 64, 32])
@pytest.mark.parametrize("M", [2, 4, 8, 16, 24, 32, 64])
@pytest.mark.parametrize("NK", [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192)])
def test_split_k_regime(M, NK, G):
    N, K = NK
    print(f"[split-k] M={M} N={N} K={K} G={G}", flush=True)
    qw, s, z = _weights(N, K, G, seed=7 * N + K + G)
    x = randn((M, K), seed=100 + M).to(DEV)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    _check(out, x, qw, s, z, ref_unrounded=False, exact_w=_decode(M, G, N, K))
    # bit-identical repeat runs, with the workspace's scratch poisoned in between
    for _ in range(2):
        _poison_workspace()
        again = int4_hip.w4a16_matmul(x, qw, s, z)
        assert torch.equal(again.view(torch.int16), out.view(torch.int16))


# int4_triton tests/test_kernels.py:86-97
@pytest.mark.parametrize("M", [1, 16, 64, 65])
@pytest.mark.parametrize("group_size", [32, 64])
def test_small_groups_strided_input_and_repeatability(M, group_size):
    x = randn((M, 512), seed=1).to(DEV)[:, ::2]
    qw, s, z = _weights(73, 256, group_size, seed=2)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    _check(out, x, qw, s, z)
    torch.testing.assert_close(int4_hip.w4a16_matmul(x, qw, s, z), out, rtol=0, atol=0)


# int4_triton tests/test_kernels.py:100-110: closed form y = 2**23, exact
@pytest.mark.parametrize("M", [1, 16, 65])
def test_native_bf16_preserves_large_activation_range(M):
    x = torch.full((M, 128), 131072.0, device=DEV, dtype=torch.bfloat16)
    w = torch.full((73, 128), 0.5, device=DEV, dtype=torch.bfloat16)
    qw, s, z = int4_hip.quantize_int4(w)
    ref4 = torch.nn.functional.linear(x.float(), int4_hip.dequantize_int4(qw, s, z, torch.bfloat16).float())
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    assert torch.equal(out.float(), ref4)
    assert torch.all(out.float() == 2.0**23)


# int4_triton tests/test_kernels.py:75-83
def test_int4_linear_3d_input():
    lin = torch.nn.Linear(2048, 512, bias=True, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(randn((512, 2048), seed=11, sigma=0.02))
    lin = lin.to(DEV)
    q = int4_hip.Int4Linear.from_linear(lin, 128)
    x = randn((2, 33, 2048), seed=12).to(DEV)
    ref = torch.nn.functional.linear(x.float(), q.dequantize(torch.float32), lin.bias.float())
    out = q(x)
    assert out.shape == (2, 33, 512)
    torch.testing.assert_close(out.float(), ref, rtol=2e-2, atol=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("M", [1, 4, 16, 40, 64])
def test_grouped_matches_single(M):
    shapes = [(2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (8192, 2048), (8192, 2048), (2048, 8192)]
    ws = [_weights(N, K, 128, seed=i) for i, (N, K) in enumerate(shapes)]
    xs = [randn((M, K), seed=50 + i).to(DEV) for i, (N, K) in enumerate(shapes)]
    outs = int4_hip.w4a16_matmul_grouped(xs, ws)
    ew = _grouped_exact(M, [(N, K, 128) for N, K in shapes])
    for x, (qw, s, z), y in zip(xs, ws, outs):
        _check(y, x, qw, s, z, ref_unrounded=False, exact_w=ew)
    singles = [int4_hip.w4a16_matmul(x, *w) for x, w in zip(xs, ws)]
    for x, (qw, s, z), b, (N, K) in zip(xs, ws, singles, shapes):
        # a lone product may take other tiles (another summation order)
        _check(b, x, qw, s, z, ref_unrounded=False, exact_w=_decode(M, 128, N, K))
    again = int4_hip.w4a16_matmul_grouped(xs, ws)
    for a, b in zip(outs, again):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


# grouped products of 65..128 rows whose every N <= 4096 (q/k/v/o shapes): one
# decode launch of 16-row slices (exact W_hat; the shared-activation prefill
# launch would round W_hat and miss this bound), repeat calls bit-identical,
# shared and separate inputs; a wider problem in the group (gate_proj) sends
# the call back to the prefill kernels
@pytest.mark.parametrize("M", [65, 96, 128])
def test_grouped_row_slices_up_to_128(M):
    print(f"[grouped-slices] M={M}", flush=True)
    shapes = [(2048, 2048), (512, 2048), (512, 2048), (2048, 2048)]
    ws = [_weights(N, K, 128, seed=60 + i) for i, (N, K) in enumerate(shapes)]
    x = randn((M, 2048), seed=70 + M).to(DEV)
    outs = int4_hip.w4a16_matmul_grouped([x] * len(ws), ws)
    for (qw, s, z), y in zip(ws, outs):
        _check(y, x, qw, s, z, ref_unrounded=False, exact_w=True)
    again = int4_hip.w4a16_matmul_grouped([x] * len(ws), ws)
    for a, b in zip(outs, again):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    xs = [randn((M, 2048), seed=80 + i).to(DEV) for i in range(len(ws))]
    for xi, (qw, s, z), y in zip(xs, ws, int4_hip.w4a16_matmul_grouped(xs, ws)):
        _check(y, xi, qw, s, z, ref_unrounded=False, exact_w=True)
    wide = ws[:1] + [_weights(8192, 2048, 128, seed=69)]
    for (qw, s, z), y in zip(wide, int4_hip.w4a16_matmul_grouped([x] * 2, wide)):
        _check(y, x, qw, s, z, exact_w="either")


def test_graph_capture_replays_match_eager():
    qw, s, z = _weights(2048, 2048, 128, seed=5)
    x = randn((16, 2048), seed=6).to(DEV)
    eager = int4_hip.w4a16_matmul(x, qw, s, z)
    g = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        int4_hip.w4a16_matmul(x, qw, s, z)  # warm-up on the capture stream
        with torch.cuda.graph(g, stream=stream):
            out = int4_hip.w4a16_matmul(x, qw, s, z)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        x.mul_(1.0)


@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_ragged_shapes(M, dtype):
    # odd N (16-column tiles), N smaller than a tile, K long enough to split
    shapes = [(73, 256, 32), (300, 2048, 64), (4, 8192, 128), (8, 4096, 16)]
    ws = [_weights(N, K, G, seed=30 + i) for i, (N, K, G) in enumerate(shapes)]
    xs = [randn((M, K), seed=40 + i, dtype=dtype).to(DEV) for i, (N, K, G) in enumerate(shapes)]
    for _ in range(3):  # repeated calls reuse the split-K workspace (counters back at zero)
        outs = int4_hip.w4a16_matmul_grouped(xs, ws)
        for x, (qw, s, z), y in zip(xs, ws, outs):
            _check(y, x, qw, s, z, ref_unrounded=False)


def test_regimes_share_one_workspace():
    # M=1 (in-kernel split fixup, counters) and M=16 / M=40 (split-K partials +
    # reduce kernel) interleaved on one stream reuse the same persistent
    # workspace; the partials must never disturb the counters.
    qw, s, z = _weights(2048, 8192, 128, seed=21)
    xs = {M: randn((M, 8192), seed=60 + M).to(DEV) for M in (1, 16, 40)}
    first = {M: int4_hip.w4a16_matmul(x, qw, s, z) for M, x in xs.items()}
    for M in (1, 16, 40):
        _check(first[M], xs[M], qw, s, z, ref_unrounded=False, exact_w=_decode(M, 128, 2048, 8192))
    for _ in range(3):
        for M in (16, 1, 40, 1):
            assert torch.equal(int4_hip.w4a16_matmul(xs[M], qw, s, z).view(torch.int16), first[M].view(torch.int16))


# factored decode kernel: odd N (one column per lane), N below one tile, long K
# (32-column tiles), K with a tail chunk, group sizes of every correction class
@pytest.mark.parametrize("G", [32, 128, 256])
@pytest.mark.parametrize("M", [1, 3, 16, 33])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_ragged_shapes(M, dtype, G):
    shapes = [(N, K) for N, K in [(73, 256), (300, 2048), (4, 8192), (8, 4352), (24, 1024 + G)] if K % G == 0]
    print(f"[decode] M={M} G={G} {dtype} shapes={shapes}", flush=True)
    ws = [_weights(N, K, G, seed=70 + i) for i, (N, K) in enumerate(shapes)]
    xs = [randn((M, K), seed=80 + i, dtype=dtype).to(DEV) for i, (N, K) in enumerate(shapes)]
    outs = int4_hip.w4a16_matmul_grouped(xs, ws)
    ew = _grouped_exact(M, [(N, K, G) for N, K in shapes])
    for x, (qw, s, z), y, (N, K) in zip(xs, ws, outs, shapes):
        _check(y, x, qw, s, z, ref_unrounded=False, exact_w=ew)
        # alone a product may take another tiling (another summation order)
        _check(int4_hip.w4a16_matmul(x, qw, s, z), x, qw, s, z, ref_unrounded=False,
               exact_w=_decode(M, G, N, K))


# one-workgroup-per-CU tilings (M <= 4): 128 columns (K <= 2048, short runs at
# K = 512), 64 columns (K = 4096, and rounds of 4 loads for group 32 at long
# K), 32 columns (K = 6144 / 8192, rounds for K = 16384, which M > 1 leaves to
# the generic kernel); partial last tiles; group sizes from 32 to 1024 (the
# largest beyond the kernel's size classes); M = 3 / 6 / 11 leave activation
# rows of the four-, eight- and sixteen-row kernels empty (M > 4: K <= 4096
# tilings only, M > 8: 64 columns); M = 24 / 64: two and four 16-row slices
# of each problem (the last one half empty at 24)
@pytest.mark.parametrize("M", [1, 3, 4, 6, 8, 11, 16, 24, 64])
@pytest.mark.parametrize("G", [32, 64, 128, 1024])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_cu_tiles(dtype, G, M):
    shapes = [(N, K) for N, K in [(200, 2048), (8, 512), (96, 4096), (40, 8192), (48, 6144), (16, 16384)]
              if K % G == 0]
    print(f"[decode-cu] M={M} G={G} {dtype} shapes={shapes}", flush=True)
    ws = [_weights(N, K, G, seed=90 + i) for i, (N, K) in enumerate(shapes)]
    xs = [randn((M, K), seed=100 + i, dtype=dtype).to(DEV) for i, (N, K) in enumerate(shapes)]
    outs = int4_hip.w4a16_matmul_grouped(xs, ws)
    ew = _grouped_exact(M, [(N, K, G) for N, K in shapes])
    for x, (qw, s, z), y, (N, K) in zip(xs, ws, outs, shapes):
        _check(y, x, qw, s, z, ref_unrounded=False, exact_w=ew)
        # alone, a small product takes narrower tiles (another summation order)
        _check(int4_hip.w4a16_matmul(x, qw, s, z), x, qw, s, z, ref_unrounded=False,
               exact_w=_decode(M, G, N, K))


# prefill (M > 64) on dense rows: split-K with fp32 partials for small M x N,
# partial row tiles, every group-size path (per-lane groups below 64); K a
# multiple of 64 (deep pipeline), K = 512 + 8 (register-staged pipeline), odd N
# (general tile kernel)
@pytest.mark.parametrize("G", [8, 32, 64, 256])
@pytest.mark.parametrize("M", [65, 130])
@pytest.mark.parametrize("NK", [(96, 512), (96, 520), (73, 512)])
def test_prefill_group_sizes_and_partial_tiles(M, G, NK):
    N, K = NK
    if K % G:
        pytest.skip("group size must divide K")
    print(f"[prefill] M={M} N={N} K={K} G={G}", flush=True)
    qw, s, z = _weights(N, K, G, seed=200 + G)
    x = randn((M, K), seed=201 + M).to(DEV)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    # M = 65 with group >= 32 takes the decode kernel's row slices (N <= 4096)
    _check(out, x, qw, s, z, exact_w=_decode(M, G, N, K))


# tiles whose weight tile is dequantized once per workgroup into LDS: 64 x 64
# (K in 1 / 2 / 4 parts per workgroup) for products with at most one such
# tile per CU, and 128 x 128 (two K parts, a 64 x 64 quarter per wave) for
# products with 0.75 to 1 such tile per CU (256 CUs: 192..256 tiles); K <=
# 4096, group >= 64; ragged M; bit-identical repeats; an output row stride of
# N + 4 (no 16-byte stores) through the C-ABI, which must leave the padding
# columns untouched
@pytest.mark.parametrize("M,N,K,G,dtype", [(2048, 512, 2048, 128, torch.bfloat16),   # two K parts (M > N)
                                           (512, 2048, 2048, 128, torch.float16),    # four parts
                                           (128, 8192, 2048, 64, torch.bfloat16),    # four parts, group 64
                                           (200, 1024, 1024, 256, torch.bfloat16),   # ragged M, group 256
                                           (130, 2048, 384, 128, torch.float16),     # one part, ragged M
                                           (320, 640, 768, 64, torch.bfloat16),      # two parts
                                           (2048, 2048, 2048, 128, torch.bfloat16),  # 128 x 128, 256 tiles
                                           (512, 8192, 2048, 256, torch.float16),    # 128 x 128, group 256
                                           (1536, 2048, 1024, 64, torch.float16),    # 128 x 128, 192 tiles, group 64
                                           (1900, 2048, 768, 128, torch.bfloat16),   # 128 x 128, ragged M
                                           (512, 2048, 8192, 128, torch.bfloat16),   # 128 x 128, K in 4 ranges
                                           (700, 2048, 8192, 64, torch.float16),     # 2 ranges, ragged M
                                           (1024, 1024, 12288, 128, torch.bfloat16)])  # 4 ranges of 3072
def test_prefill_lds_dequant_tiles(M, N, K, G, dtype):
    from int4_hip import _lib
    print(f"[prefill-lds] M={M} N={N} K={K} G={G} {dtype}", flush=True)
    qw, s, z = _weights(N, K, G, seed=M + N + K)
    x = randn((M, K), seed=M + 5, dtype=dtype).to(DEV)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    _check(out, x, qw, s, z, exact_w=_decode(M, G, N, K))
    for _ in range(2):
        assert torch.equal(int4_hip.w4a16_matmul(x, qw, s, z).view(torch.int16), out.view(torch.int16))
    lib = _lib.load()
    xdt = _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_FP16
    ypad = torch.full((M, N + 4), float("nan"), dtype=dtype, device=DEV)
    nb = lib.w4a16_workspace_bytes(M, N, K, G)  # K split across workgroups: counters and partial tiles
    ws = torch.zeros(max(nb, 1), dtype=torch.uint8, device=DEV)
    rc = lib.w4a16_gemm(x.data_ptr(), xdt, M, N, K, K, 1, qw.data_ptr(), s.data_ptr(), z.data_ptr(), G,
                        ypad.data_ptr(), N + 4, ws.data_ptr() if nb else None, nb,
                        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "w4a16_gemm")
    torch.cuda.synchronize()
    assert torch.equal(ypad[:, :N].view(torch.int16), out.view(torch.int16))
    assert torch.isnan(ypad[:, N:].float()).all()


# the same tiles on activation rows with a stride above K (a column slice of a
# wider tensor: rows still dense and 16-byte aligned)
@pytest.mark.parametrize("M,N,K", [(512, 2048, 2048), (2048, 512, 1024), (2048, 2048, 2048)])
def test_prefill_lds_dequant_tiles_row_stride(M, N, K):
    print(f"[prefill-lds strided] M={M} N={N} K={K}", flush=True)
    qw, s, z = _weights(N, K, 128, seed=M + 3 * N + K)
    x = randn((M, K + 64), seed=M + 9).to(DEV)[:, :K]
    assert x.stride(0) == K + 64
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    _check(out, x, qw, s, z, exact_w=_decode(M, 128, N, K))
    assert torch.equal(int4_hip.w4a16_matmul(x.contiguous(), qw, s, z).view(torch.int16), out.view(torch.int16))


# shapes whose static plan runs 32-row tiles as workgroups of two K halves
# (eight waves, the halves summed through LDS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(256, 8192, 2048), (1024, 2048, 2048)])
def test_prefill_two_k_halves(M, N, K, dtype):
    print(f"[prefill-kh] M={M} N={N} K={K} {dtype}", flush=True)
    qw, s, z = _weights(N, K, 128, seed=M + 7)
    x = randn((M, K), seed=M + 8, dtype=dtype).to(DEV)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    _check(out, x, qw, s, z)
    assert torch.equal(int4_hip.w4a16_matmul(x, qw, s, z).view(torch.int16), out.view(torch.int16))


# (M = 128 takes the decode kernel's row slices, with a K split for K = 8192)
@pytest.mark.parametrize("M", [128, 130, 512])
@pytest.mark.parametrize("NK", [(512, 2048), (2048, 8192)])
def test_prefill_split_k_bit_identical(M, NK):
    N, K = NK
    print(f"[prefill-split] M={M} N={N} K={K}", flush=True)
    qw, s, z = _weights(N, K, 128, seed=N + M)
    x = randn((M, K), seed=300 + M, dtype=torch.float16).to(DEV)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    _check(out, x, qw, s, z, ref_unrounded=False, exact_w=_decode(M, 128, N, K))
    for _ in range(2):
        assert torch.equal(int4_hip.w4a16_matmul(x, qw, s, z).view(torch.int16), out.view(torch.int16))


# grouped products for M > 16: a shared activation runs as one prefill launch
# when the plan for the concatenated width needs no split-K (these shapes), a
# mix of inputs falls back to one launch per problem; every output against the
# oracle, repeat calls bit-identical
@pytest.mark.parametrize("G", [32, 128])
@pytest.mark.parametrize("M,K,Ns", [(130, 512, (256, 64, 64)), (300, 256, (1024, 256, 256)),
                                     (512, 512, (192, 72, 120)), (40, 512, (128, 64)),
                                     (128, 2048, (2048, 512, 512)), (24, 2048, (2048, 512, 512))])
def test_grouped_shared_activation(M, K, Ns, G):
    print(f"[grouped-prefill] M={M} K={K} Ns={Ns} G={G}", flush=True)
    ws = [_weights(N, K, G, seed=400 + i) for i, N in enumerate(Ns)]
    x = randn((M, K), seed=410 + M).to(DEV)
    # M <= 64: decode launches (exact W_hat) or, where the library's plan
    # prefers it, one shared-activation prefill launch (W_hat rounded); up to
    # M = 128 the per-problem fallback of mixed inputs may take the decode
    # kernel's row slices (N <= 4096)
    ew = "either" if M <= 128 else False
    outs = int4_hip.w4a16_matmul_grouped([x] * len(Ns), ws)
    for (qw, s, z), y in zip(ws, outs):
        _check(y, x, qw, s, z, ref_unrounded=True, exact_w=ew)
    again = int4_hip.w4a16_matmul_grouped([x] * len(Ns), ws)
    for a, b in zip(outs, again):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    xs = [randn((M, K), seed=420 + i).to(DEV) for i in range(len(Ns))]
    mixed = int4_hip.w4a16_matmul_grouped(xs, ws)
    for xi, (qw, s, z), y in zip(xs, ws, mixed):
        _check(y, xi, qw, s, z, ref_unrounded=True, exact_w=ew)


def _replays_match(g, out, eager, reps=3):
    """Replay a captured graph several times, with eager work and host
    synchronisation between replays; every replay must equal the eager bits."""
    for _ in range(reps):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        torch.randn(1 << 16, device=DEV).sum().item()


# capture on torch's own capture stream after a warm-up on another stream, as
# eval_llama.py:145-161 (decode step) and triton's do_bench_cudagraph
# (bench_gemm.py:33-36) do: M = 1 decode shapes whose size query is nonzero,
# and split-K shapes that need the workspace (M = 128 / 512 / 2048 down_proj
# and M = 512 k_proj: the prefill kernels' K splits finished in the kernel,
# arrival counters and partial tiles in the workspace)
@pytest.mark.parametrize("M,N,K,G", [(1, 2048, 8192, 128), (1, 2048, 2048, 128), (1, 300, 2048, 16),
                                     (40, 2048, 8192, 128), (64, 8192, 2048, 128), (128, 512, 2048, 128),
                                     (128, 2048, 8192, 128), (512, 512, 2048, 128), (512, 2048, 8192, 128),
                                     (2048, 2048, 8192, 128)])
def test_capture_without_warmup_on_capture_stream(M, N, K, G):
    print(f"[capture] M={M} N={N} K={K} G={G}", flush=True)
    qw, s, z = _weights(N, K, G, seed=M + N + G)
    x = randn((M, K), seed=M + 3).to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = int4_hip.w4a16_matmul(x, qw, s, z)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _check(eager, x, qw, s, z, ref_unrounded=False, exact_w=_decode(M, G, N, K))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):  # no stream: torch's default capture stream
        out = int4_hip.w4a16_matmul(x, qw, s, z)
    _replays_match(g, out, eager)


# many graphs captured on torch's default capture stream, each with no warm-up
# and a route that needs the workspace (M = 40 with K = 8192: the decode
# kernel's K split, partial tiles and arrival counters): the captures share
# one buffer per (device, capture stream) instead of one each, and every
# graph, replayed in any order, starts from zero counters
def test_capture_many_graphs_shares_one_workspace():
    from int4_hip import gemm as _gemm
    qw, s, z = _weights(2048, 8192, 128, seed=77)
    x = randn((40, 8192), seed=78).to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = int4_hip.w4a16_matmul(x, qw, s, z)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    def buffers():
        return {t.data_ptr() for t in list(_gemm._WS.values()) + list(_gemm._CAP_WS.values()) + _gemm._WS_RETIRED}

    before = buffers()
    graphs = []
    for i in range(20):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = int4_hip.w4a16_matmul(x, qw, s, z)
        graphs.append((g, out))
    assert len(buffers() - before) <= 1, "captured calls must share the capture stream's workspace"
    order = list(range(19, -1, -1)) + [0, 7, 3, 19, 7]
    for i in order:
        _replays_match(graphs[i][0], graphs[i][1], eager, reps=1)


def test_capture_grouped_without_warmup():
    shapes = [(2048, 2048), (512, 2048), (512, 2048), (2048, 8192)]
    ws = [_weights(N, K, 32 if i == 3 else 128, seed=500 + i) for i, (N, K) in enumerate(shapes)]
    for M in (1, 40):
        print(f"[capture grouped] M={M}", flush=True)
        xs = [randn((M, K), seed=510 + i).to(DEV) for i, (N, K) in enumerate(shapes)]
        eager = int4_hip.w4a16_matmul_grouped(xs, ws)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs = int4_hip.w4a16_matmul_grouped(xs, ws)
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            for a, b in zip(outs, eager):
                assert torch.equal(a.view(torch.int16), b.view(torch.int16))
            torch.randn(1 << 16, device=DEV).sum().item()


def test_capture_grouped_block_m64_rows():
    """The 7-linear block at M = 64 in one grouped call takes the several-row
    kernel, whose down_proj K split needs the workspace: checked against the
    oracle (W_hat rounded to bf16), then captured without a warm-up and
    replayed with eager work between replays, every replay equal to the eager
    bits."""
    shapes = [(2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (8192, 2048), (8192, 2048), (2048, 8192)]
    assert not _grouped_exact(64, [(N, K, 128) for N, K in shapes])  # the several-row kernel's route
    ws = [_weights(N, K, 128, seed=600 + i) for i, (N, K) in enumerate(shapes)]
    xs = [randn((64, K), seed=610 + i).to(DEV) for i, (N, K) in enumerate(shapes)]
    eager = int4_hip.w4a16_matmul_grouped(xs, ws)
    for x, (qw, s, z), y in zip(xs, ws, eager):
        _check(y, x, qw, s, z, ref_unrounded=False, exact_w=False)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = int4_hip.w4a16_matmul_grouped(xs, ws)
    for _ in range(3):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))
        torch.randn(1 << 16, device=DEV).sum().item()


# strided activation rows (row stride not a multiple of 8) take the skinny
# split-K kernel even at M <= 16; a fresh stream sizes its workspace from the
# size query, which must cover that route too
@pytest.mark.parametrize("M,N,K", [(16, 3072, 14336), (5, 2048, 8192)])
def test_strided_rows_workspace_on_new_stream(M, N, K):
    print(f"[strided ws] M={M} N={N} K={K}", flush=True)
    qw, s, z = _weights(N, K, 128, seed=N + 1)
    big = randn((M, K + 4), seed=K).to(DEV)
    x = big[:, :K]
    assert x.stride(0) % 8 != 0
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        out = int4_hip.w4a16_matmul(x, qw, s, z)
        again = int4_hip.w4a16_matmul(x, qw, s, z)
    torch.cuda.synchronize()
    _check(out, x, qw, s, z, ref_unrounded=False)
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))


# M = 1 with K > 4096: the decode kernel splits K into two or four parts on
# 64-column tiles whose partial sums meet pairwise through 64-bit
# compare-and-swap words (one or two tree levels); every repeat, with the
# outputs poisoned in between, must give the same bits, lone and grouped
@pytest.mark.parametrize("N,K,G", [(2048, 8192, 128), (1024, 16384, 64), (200, 6144, 32), (72, 12288, 128)])
def test_decode_ksplit_pairs_repeat(N, K, G):
    print(f"[ksplit] N={N} K={K} G={G}", flush=True)
    qw, s, z = _weights(N, K, G, seed=N + K + G)
    x = randn((1, K), seed=K + 1).to(DEV)
    first = int4_hip.w4a16_matmul(x, qw, s, z)
    _check(first, x, qw, s, z, ref_unrounded=False, exact_w=True)
    other = [_weights(2048, 2048, G, seed=9), randn((1, 2048), seed=10).to(DEV)]
    grouped_first = None
    for _ in range(4):
        y = torch.full((1, N), float("nan"), dtype=torch.bfloat16, device=DEV)
        again = int4_hip.w4a16_matmul(x, qw, s, z)
        assert torch.equal(again.view(torch.int16), first.view(torch.int16))
        yo = torch.full((1, 2048), float("nan"), dtype=torch.bfloat16, device=DEV)
        int4_hip.w4a16_matmul_grouped([x, other[1]], [(qw, s, z), other[0]], out=[y, yo])
        if grouped_first is None:
            _check(y, x, qw, s, z, ref_unrounded=False, exact_w=True)
            grouped_first = y.clone()
        assert torch.equal(y.view(torch.int16), grouped_first.view(torch.int16))


# several-row decode kernels with K split (K > 4096 at 2 <= M <= 64): parts of
# 64 columns x K / ks combined by the last part to arrive; partial column
# tiles, several slices, ks = 2 and 4, every group size; repeated calls with
# the workspace's scratch poisoned in between must give the same bits (the
# arrival counters are left at zero, the partial tiles are always rewritten)
@pytest.mark.parametrize("M,N,K,G", [(2, 2048, 8192, 128), (3, 300, 6144, 32), (4, 1024, 16384, 64),
                                     (6, 2048, 8192, 256), (8, 200, 12288, 128),
                                     (9, 200, 6144, 64), (16, 2048, 8192, 128), (16, 2048, 16384, 32),
                                     (13, 4096, 14336, 128), (40, 520, 8192, 32), (64, 72, 12288, 128),
                                     (64, 2048, 8192, 64)])
def test_decode_rows_ksplit(M, N, K, G):
    print(f"[ksplit-rows] M={M} N={N} K={K} G={G}", flush=True)
    qw, s, z = _weights(N, K, G, seed=3 * N + K + G)
    x = randn((M, K), seed=M + K).to(DEV)
    first = int4_hip.w4a16_matmul(x, qw, s, z)
    _check(first, x, qw, s, z, ref_unrounded=False, exact_w=_decode(M, G, N, K))
    for _ in range(3):
        _poison_workspace()
        again = int4_hip.w4a16_matmul(x, qw, s, z)
        assert torch.equal(again.view(torch.int16), first.view(torch.int16))


def _random_cases(n=30, seed=2024, cap=1.5e9):
    """Seeded shapes over every routing regime: M = 1, 2..16, 17..64,
    65..128 and above; N odd or even, multiples of 128 half the time (the
    tiled fast paths); group sizes 32..256; K up to 8192; bf16 / fp16; a
    quarter of them on strided activations (x[:, ::2], the split-K paths)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        lo, hi = [(1, 1), (2, 16), (17, 64), (65, 128), (129, 2600)][i % 5]
        M = int(rng.integers(lo, hi + 1))
        G = int(rng.choice([32, 64, 128, 256]))
        K = G * int(rng.integers(1, max(2, 8192 // G) + 1))
        N = 128 * int(rng.integers(1, 65)) if rng.random() < 0.5 else int(rng.integers(1, 4097))
        while M * N * K > cap and (K > G or N > 1):  # K first: keep the tiled widths
            if K > G:
                K = max(G, K // 2 // G * G)
            else:
                N = max(1, N // 2)
        out.append((M, N, K, G, bool(rng.random() < 0.25), bool(rng.random() < 0.5)))
    return out


# every routing regime on seeded random shapes against the oracle (exact W_hat
# where the factored decode kernel takes the product, rounded W_hat elsewhere),
# repeat calls bit-identical
@pytest.mark.parametrize("M,N,K,G,strided,fp16", _random_cases())
def test_random_shapes_against_oracle(M, N, K, G, strided, fp16):
    dtype = torch.float16 if fp16 else torch.bfloat16
    print(f"[random] M={M} N={N} K={K} G={G} strided={strided} {dtype}", flush=True)
    qw, s, z = _weights(N, K, G, seed=M + 3 * N + 7 * K + G)
    if strided:
        x = randn((M, 2 * K), seed=M + K, dtype=dtype).to(DEV)[:, ::2]
    else:
        x = randn((M, K), seed=M + K, dtype=dtype).to(DEV)
    out = int4_hip.w4a16_matmul(x, qw, s, z)
    assert out.shape == (M, N) and out.dtype == dtype
    _check(out, x, qw, s, z, exact_w=(not strided) and _decode(M, G, N, K))
    assert torch.equal(int4_hip.w4a16_matmul(x, qw, s, z).view(torch.int16), out.view(torch.int16))


def _random_grouped_cases(n=12, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        lo, hi = [(1, 1), (2, 16), (17, 64), (65, 128), (129, 700)][i % 5]
        M = int(rng.integers(lo, hi + 1))
        G = int(rng.choice([32, 64, 128]))
        K = G * int(rng.integers(1, 4096 // G + 1))
        count = int(rng.integers(1, 5))
        Ns = tuple(128 * int(rng.integers(1, 49)) if rng.random() < 0.6 else int(rng.integers(1, 3000))
                   for _ in range(count))
        out.append((M, K, G, Ns, bool(rng.random() < 0.5)))
    return out


# grouped products on seeded random shapes: one shared activation or one per
# problem, every output against the oracle (exact W_hat where the grouped call
# must take the decode launch, rounded where it must take the prefill kernels,
# either bound where a per-problem fallback may take either), repeats
# bit-identical
@pytest.mark.parametrize("M,K,G,Ns,shared", _random_grouped_cases())
def test_random_grouped_against_oracle(M, K, G, Ns, shared):
    print(f"[random grouped] M={M} K={K} G={G} Ns={Ns} shared={shared}", flush=True)
    ws = [_weights(N, K, G, seed=500 + 11 * i + N) for i, N in enumerate(Ns)]
    if shared:
        xs = [randn((M, K), seed=600 + M).to(DEV)] * len(Ns)
    else:
        xs = [randn((M, K), seed=610 + M + i).to(DEV) for i in range(len(Ns))]
    if M <= 64 or (M <= 128 and all(N <= 4096 for N in Ns)):
        # one several-row or decode launch (group sizes >= 32)
        ew = _grouped_exact(M, [(N, K, G) for N in Ns])
    elif M > 128:
        ew = False       # prefill kernels (shared or one call per problem)
    else:
        ew = "either"    # 65..128 rows with a wide problem: per-problem routes
    outs = int4_hip.w4a16_matmul_grouped(xs, ws)
    for x, (qw, s, z), y in zip(xs, ws, outs):
        _check(y, x, qw, s, z, ref_unrounded=False, exact_w=ew)
    for a, b in zip(outs, int4_hip.w4a16_matmul_grouped(xs, ws)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
