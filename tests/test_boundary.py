"""CPU tests of the drop-in boundary: the C-ABI library, argument validation
(C side and Python side, mirroring the reference's assertions), module
structure.  No GPU compute is issued here."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn as nn

import int4_hip
from int4_hip import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "int4_hip.h"


def _header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\**\s+\**(w4[a-z0-9_]*)\s*\(", text, flags=re.M)))


def test_header_declares_expected_entry_points():
    assert _header_functions() == sorted(_lib.SIGNATURES)


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (run __graft_entry__.build())")
    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    for name in _header_functions():
        assert hasattr(lib, name), name
    assert lib.w4_abi_version() == _lib.ABI_VERSION


def test_c_abi_rejects_bad_quantize_arguments(lib):
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # bad dtype
    assert lib.w4_quantize(fake, 7, 4, 64, 64, 1, 32, fake, fake, fake, None) == _lib.ERR_INVALID
    assert b"dtype" in lib.w4_last_error()
    # group size not a power of two / not dividing K / not a multiple of 8
    for g in (24, 48, 12, 3):
        assert lib.w4_quantize(fake, 0, 4, 96, 96, 1, g, fake, fake, fake, None) == _lib.ERR_INVALID
    # per-channel with non power-of-two K (the reference asserts the same)
    assert lib.w4_quantize(fake, 0, 4, 96, 96, 1, -1, fake, fake, fake, None) == _lib.ERR_INVALID
    # null pointers
    assert lib.w4_quantize(None, 0, 4, 64, 64, 1, 32, fake, fake, fake, None) == _lib.ERR_INVALID
    # empty N is a no-op success
    assert lib.w4_quantize(None, 0, 0, 64, 64, 1, 32, None, None, None, None) == _lib.OK


def test_c_abi_rejects_bad_gemm_arguments(lib):
    fake = ctypes.c_void_p(16)
    args = dict(x=fake, dt=0, M=1, N=8, K=64, sxm=64, sxk=1, qw=fake, s=fake, z=fake, G=32, y=fake, ldy=8)

    def call(**kw):
        a = {**args, **kw}
        return lib.w4a16_gemm(a["x"], a["dt"], a["M"], a["N"], a["K"], a["sxm"], a["sxk"], a["qw"], a["s"],
                              a["z"], a["G"], a["y"], a["ldy"], None, 0, None)

    assert call(dt=2) == _lib.ERR_INVALID          # fp32 activations are not supported
    assert call(K=60) == _lib.ERR_INVALID          # K % 8
    assert call(G=48) == _lib.ERR_INVALID          # not a power of two
    assert call(G=128) == _lib.ERR_INVALID         # does not divide K
    assert call(ldy=4) == _lib.ERR_INVALID         # ldy < N
    assert call(x=None) == _lib.ERR_INVALID
    assert call(M=0) == _lib.OK                    # empty product
    for M in (1, 8, 40, 65, 512):  # any workspace starts with the counter area
        n = lib.w4a16_workspace_bytes(M, 2048, 8192, 128)
        assert n == 0 or n > 65536


def test_workspace_queries_over_regime_boundaries(lib):
    """The size queries run the launch planners on the host only: a sweep over
    the regime boundaries (M around 1 / 4 / 8 / 16 / 64 / 128, K around 4096 and
    8192, K without a whole-round split such as 4352, every group size)
    answers without error, and every non-zero size covers the counter area."""
    import ctypes

    count = 0
    for M in (1, 2, 3, 4, 5, 8, 9, 13, 16, 17, 24, 33, 40, 64, 65, 96, 128, 129):
        for N in (8, 72, 200, 2048, 8192):
            for K in (256, 2048, 4096, 4352, 6144, 8192, 12288, 14336, 16384):
                for G in (32, 64, 128, 256, 1024):
                    if K % G:
                        continue
                    n = lib.w4a16_workspace_bytes(M, N, K, G)
                    assert n == 0 or n > 65536
                    count += 1
    assert count > 2000
    # grouped queries on 256-byte aligned stand-ins (only the alignment is read)
    buf = ctypes.create_string_buffer(512)
    base = (ctypes.addressof(buf) + 255) // 256 * 256
    shapes = [(2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (8192, 2048), (8192, 2048), (2048, 8192)]
    for M in (1, 3, 8, 12, 16, 24, 40, 64, 65):
        for G in (32, 128):
            for shp in (shapes, [(300, 4352), (200, 6144)], [(72, 12288)]):
                probs = (_lib.Problem * len(shp))()
                for i, (N, K) in enumerate(shp):
                    probs[i] = _lib.Problem(base, base, base, base, base, N, K, G, 0)
                n = lib.w4a16_grouped_workspace_bytes(probs, len(shp), M)
                assert n == 0 or n >= 65536


def test_c_abi_rejects_bad_grouped_arguments(lib):
    probs = (_lib.Problem * 1)()
    assert lib.w4a16_gemm_grouped(probs, 0, 0, 1, None, 0, None) == _lib.ERR_INVALID
    assert lib.w4a16_gemm_grouped(probs, 1, 0, 17, None, 0, None) == _lib.ERR_INVALID
    assert lib.w4a16_gemm_grouped(probs, 1, 0, 1, None, 0, None) == _lib.ERR_INVALID  # null pointers
    assert lib.w4a16_gemm_grouped(probs, _lib.MAX_GROUPED + 1, 0, 1, None, 0, None) == _lib.ERR_INVALID
    assert lib.w4a16_gemm_grouped(probs, 1, 2, 1, None, 0, None) == _lib.ERR_INVALID  # fp32 activations
    assert lib.w4a16_grouped_workspace_bytes(probs, 0, 1) == 0


# ---------------------------------------------------------- Python-side asserts
# Same exception type as the reference (AssertionError) for the same misuse
# (int4_triton/quantize.py:69-75, int4_triton/gemm.py:305-307, qlinear.py:13).
def test_quantize_asserts_like_reference():
    w = torch.zeros(16, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        int4_hip.quantize_int4(w)  # not on the GPU
    with pytest.raises(AssertionError):
        int4_hip.quantize_int4(torch.zeros(16, 64, 2, dtype=torch.bfloat16))


def test_matmul_asserts_like_reference():
    qw = torch.zeros(8, 16, dtype=torch.int32)
    s = torch.ones(2, 16, dtype=torch.float16)
    with pytest.raises(AssertionError):
        int4_hip.w4a16_matmul(torch.zeros(1, 64, dtype=torch.float32), qw, s, s)
    with pytest.raises(AssertionError):
        int4_hip.w4a16_matmul(torch.zeros(1, 72, dtype=torch.bfloat16), qw, s, s)  # K != 8*qweight rows


def test_int4linear_buffers_match_reference_layout():
    m = int4_hip.Int4Linear(256, 48, group_size=64, bias=True, device="cpu")
    sd = m.state_dict()
    assert list(sd) == ["qweight", "scales", "zeros", "bias"]
    assert sd["qweight"].shape == (32, 48) and sd["qweight"].dtype == torch.int32
    assert sd["scales"].shape == (4, 48) and sd["scales"].dtype == torch.float16
    assert sd["zeros"].shape == (4, 48) and sd["zeros"].dtype == torch.float16
    assert "group_size=64" in repr(m)
    with pytest.raises(AssertionError):
        int4_hip.Int4Linear(100, 8, group_size=64)


def test_iter_linears_skip_rule():
    from int4_hip.qlinear import _iter_linears

    model = nn.Sequential()
    model.add_module("block", nn.Sequential(nn.Linear(8, 8), nn.ReLU(), nn.Linear(8, 8)))
    model.add_module("lm_head", nn.Linear(8, 4))
    names = [n for _, n, _ in _iter_linears(model, ("lm_head",))]
    assert names == ["0", "2"]
    assert len(list(_iter_linears(model, ()))) == 3


def test_product_package_does_not_import_the_oracle():
    pkg = ROOT / "itmo-final-project_amd"
    for p in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.cpp")):
        assert "oracle" not in p.read_text(), f"{p} references the test oracle"


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load(tmp_path / "nope.so")


def _pf3_max_reach(N, K, G, NW, szk, mask_cols):
    """Model of pf3_tile's weight / scale loads (w4_prefill.hip: w_lane, sz_col
    and `issue`): for every lane of every column tile and every step (plus the
    clamped prefetches), the raw-buffer range check rejects a load whose
    per-lane offset is >= the tensor's bytes, and otherwise the bytes
    [voffset + soffset, + size) are read.  Returns the largest end reached in
    qweight and in scales (zeros share the scales' offsets)."""
    OOB = 0x80000000
    qw_bytes, sz_bytes = K // 8 * N * 4, K // G * N * 2
    tiles_n = -(-N // (64 * NW))
    KT = K // 64
    reach_q = reach_s = 0
    for tn in range(tiles_n):
        for wn in range(NW):
            n0w = (tn * NW + wn) * 64
            for lane in range(64):
                l32, lh = lane & 31, lane >> 5
                col_in = (n0w + 2 * l32 < N) or not mask_cols
                w_lane = (lh * N + n0w + 2 * l32) * 4 if col_in else OOB
                sz_col = (n0w + 2 * l32) * 2 if col_in else OOB
                for kt in range(KT):  # prefetches past the end reload step KT - 1
                    for ks in range(4):
                        if w_lane < qw_bytes:
                            reach_q = max(reach_q, w_lane + kt * 8 * N * 4 + ks * 2 * N * 4 + 8)
                    for j in range(4 if szk else 1):
                        g = (kt * 64 + (j * 16 + lh * 8 if szk else 0)) // G
                        vo, so = (g * N * 2 + sz_col, 0) if szk else (sz_col, g * N * 2)
                        if vo < sz_bytes:
                            reach_s = max(reach_s, vo + so + 4)
    return (reach_q, qw_bytes), (reach_s, sz_bytes)


@pytest.mark.parametrize("N,K,G,NW", [(96, 256, 64, 4), (130, 192, 32, 2), (2050, 128, 128, 4), (64 * 4 + 2, 64, 8, 4)])
def test_pf3_loads_stay_inside_their_tensors(N, K, G, NW):
    """N not a multiple of the tile width: the lanes of a partial last tile
    whose columns lie past N must not read past the end of qweight or scales
    (the range check sees only the per-lane offset, the step travels in the
    scalar offset), so a C-ABI caller with exact-size buffers is safe."""
    for szk in (G < 64, False):
        (rq, nq), (rs, ns) = _pf3_max_reach(N, K, G, NW, szk, mask_cols=True)
        assert rq <= nq and rs <= ns, (N, K, G, NW, szk, rq, nq, rs, ns)
    # the same model without the column mask reaches past the end: the check
    # above would catch a regression of the mask
    (rq, nq), _ = _pf3_max_reach(N, K, G, NW, False, mask_cols=False)
    assert rq > nq


def _rows_model(M, N, K, G, ks, MR, sxm=None):
    """Model of rows_tile's addressing (w4_rows.hip: x_lane, w_lane, sz_lane,
    a_off, `issue_ring`, the packed-word loads and the partial-tile stores),
    for every workgroup (column
    tile, K part), wave, lane and step, including the ring's prefetches past
    the end of a run (offset | 0x80000000, rejected by the range check).
    Returns a dict of the largest end reached per tensor / LDS area against its
    size, the k8 rows each column of a tile reads (each must be read exactly
    once), and whether every A-fragment read finds the (row, k chunk) the
    MFMA expects at that LDS position."""
    OOB, RING, KWAVES, HALVES = 0x80000000, 4, 4, 2
    WAVES, TILE = KWAVES * HALVES, 64 * HALVES
    sxm = K if sxm is None else sxm
    RB, SLOT = MR // 16, MR * 64
    S = K // (ks * KWAVES * 32)
    qw_bytes, sz_bytes, x_bytes = K // 8 * N * 4, K // G * N * 2, ((M - 1) * sxm + K) * 2
    lds_bytes = WAVES * RING * SLOT
    reach = {"qw": 0, "sz": 0, "x": 0, "lds": 0, "red": 0}
    k8_reads = np.zeros((K // 8, N), np.int64)
    lane = np.arange(64)
    lq, lr = lane & 15, lane >> 4
    layout_ok = True
    for ct in range(-(-N // TILE)):
        for kp in range(ks):
            for wv in range(WAVES):
                n0 = ct * TILE + 64 * (wv % HALVES)
                col_in = n0 + 4 * lq < N
                col_oob = np.where(col_in, 0, OOB)
                w_lane = (lr * N + n0 + 4 * lq) * 4
                sz_lane = (n0 + 4 * lq) * 2
                st0 = (kp * KWAVES + wv // HALVES) * S
                ring = wv * RING * SLOT
                x_lane = []
                for j in range(RB):
                    row = 16 * j + (lane >> 2)
                    c = (lane & 3) ^ ((lane >> 3) & 3)
                    x_lane.append(np.where(row < M, (row * sxm + c * 8) * 2, OOB))
                for i in range(S + RING):
                    oob = 0 if i < S else OOB
                    st = st0 + min(i, S - 1)
                    slot = ring + (i & (RING - 1)) * SLOT
                    for j in range(RB):
                        vo = (x_lane[j] + st * 64) | oob
                        ok = vo < x_bytes
                        if ok.any():
                            reach["x"] = max(reach["x"], int((vo[ok] + 16).max()))
                        reach["lds"] = max(reach["lds"], slot + 1024 * j + 16 * 63 + 16)
                    so = ((st * 32 // G) * N * 2 + sz_lane) | col_oob | oob
                    ok = so < sz_bytes
                    if ok.any():
                        reach["sz"] = max(reach["sz"], int((so[ok] + 8).max()))
                for i in range(16):  # packed words: every step of the run at once (kRowsMaxWaveSteps)
                    oob = 0 if i < S else OOB
                    st = st0 + min(i, S - 1)
                    wo = (w_lane + st * 16 * N) | col_oob | oob
                    ok = wo < qw_bytes
                    if ok.any():
                        reach["qw"] = max(reach["qw"], int((wo[ok] + 16).max()))
                        # the words each lane multiplies: k8 row 4 st + lr, columns n0 + 4 lq .. + 3
                        for l in np.nonzero(ok)[0]:
                            k8_reads[4 * st + lr[l], n0 + 4 * lq[l]: n0 + 4 * lq[l] + 4] += 1
                # A fragments: where the stores above put (row, chunk), the reads find it
                pos = {}
                for j in range(RB):
                    for l in range(64):
                        row = 16 * j + (l >> 2)
                        pos[1024 * j + 16 * l] = (row, (l & 3) ^ ((l >> 3) & 3))
                for rb in range(RB):
                    for l in range(64):
                        a_off = (l & 15) * 64 + (((l >> 4) ^ (((l & 15) >> 1) & 3)) * 16)
                        layout_ok = layout_ok and pos[rb * 1024 + a_off] == (16 * rb + (l & 15), l >> 4)
                # partial tile: row 16 rb + 4 lr + r, columns 4 lq .. + 3 (floats)
                for rb in range(RB):
                    for r in range(4):
                        end = wv * MR * 64 + (16 * rb + 4 * lr + r) * 64 + 4 * lq + 4
                        reach["red"] = max(reach["red"], int(end.max()) * 4)
    sizes = {"qw": qw_bytes, "sz": sz_bytes, "x": x_bytes, "lds": lds_bytes, "red": lds_bytes}
    return reach, sizes, k8_reads, layout_ok


@pytest.mark.parametrize("M,N,K,G,ks,MR", [
    (49, 68, 128, 32, 1, 64), (55, 200, 512, 128, 1, 64), (64, 128, 1024, 64, 2, 64),
    (50, 2052, 256, 256, 2, 64), (63, 4, 4096, 4096, 8, 64), (64, 1000, 2048, 128, 4, 64),
    (64, 2048, 8192, 128, 4, 64),
])
def test_rows_kernel_accesses_stay_inside_and_cover_k(M, N, K, G, ks, MR):
    """The several-row kernel: every load's bytes lie inside its tensor (also in
    a partial last column tile and for the ring's prefetches past a run), LDS
    stores and reads stay inside the workgroup's array, every (k8 row, column)
    of the product is read exactly once over the K parts and waves, and the
    swizzled activation slots give each lane the row and k chunk its MFMA
    operand needs."""
    reach, sizes, k8_reads, layout_ok = _rows_model(M, N, K, G, ks, MR)
    for name in reach:
        assert reach[name] <= sizes[name], (name, reach[name], sizes[name])
    assert (k8_reads == 1).all()
    assert layout_ok


def _pf5_swizzle(TS: int, n: int) -> int:
    """The chunk swizzle of pf5's dequantized weight tile (w4_prefill.hip,
    pf5_kernel): chunk (column n, k8 row j) of a buffer at slot n * 8 + (j ^ f(n))."""
    return (n >> 1) & 7 if TS == 64 else ((n >> 2) ^ (n << 1)) & 7


@pytest.mark.parametrize("TS", [64, 128])
def test_pf5_weight_tile_swizzle_is_conflict_free(TS):
    """pf5's LDS weight tile under the bank model its layout is chosen for (64
    banks of 4 bytes; a 128-bit store serves 8 lanes at a time, a 128-bit read
    16): the slots of a column are a permutation of its 8 chunks; the 8 lanes of
    a store (thread t writes columns WPT (t % 32) + i of k8 row t / 32) and the
    16 lanes of a fragment read (consecutive columns, one chunk) cover distinct
    bank quads; the swizzle depends on n % 32 only (blocks 32 columns apart
    share the offsets).  The 64-wide form on 128-wide stores is the case that
    conflicts."""
    WPT = TS // 32

    def quad(n, j):  # bank quad (4 banks) of chunk (n, j)
        slot = n * 8 + (j ^ _pf5_swizzle(TS, n))
        return (slot * 16 // 4 % 64) // 4

    for n in range(TS):
        assert sorted(j ^ _pf5_swizzle(TS, n) for j in range(8)) == list(range(8))
        assert _pf5_swizzle(TS, n) == _pf5_swizzle(TS, n % 32)
    for j in range(8):  # stores: lanes l .. l + 7 of one k8 row
        for i in range(WPT):
            for l0 in range(0, 32, 8):
                quads = [quad(WPT * l + i, j) for l in range(l0, l0 + 8)]
                assert len(set(quads)) == 8, (TS, j, i, l0, quads)
    for c in range(8):  # fragment reads: 16 consecutive columns, chunk c
        for n0 in range(0, TS, 16):
            banks = set()
            for n in range(n0, n0 + 16):
                slot = n * 8 + (c ^ _pf5_swizzle(TS, n))
                b = slot * 16 // 4 % 64
                banks.update(range(b, b + 4))
            assert len(banks) == 64, (TS, c, n0)
    if TS == 128:  # the 64-wide swizzle on this tile's stores: two-way conflicts
        old = lambda n, j: ((n * 8 + (j ^ ((n >> 1) & 7))) * 16 // 4 % 64) // 4
        assert len({old(4 * l, 0) for l in range(8)}) == 4
