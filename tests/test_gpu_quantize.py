"""GPU parity: the HIP quantize/pack and dequantize kernels against the CPU
oracle (bit-exact) and the reference's golden vectors."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import int4_hip
from oracle import w4a16_oracle as O
from golden.make_golden import sha, synth_weight_bits
from _synth import assert_bits_equal_nan_aware, bits_of, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"
_G = np.load(GOLDEN / "quantize_golden.npz")
CASES = sorted({k.split("__")[0] for k in _G.files})
LLAMA = [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192)]
TDT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _to_dev(bits: np.ndarray, dt: str) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(TDT[dt]).to(DEV)


def _quantize_np(w: torch.Tensor, g: int):
    qw, s, z = int4_hip.quantize_int4(w, g)
    torch.cuda.synchronize()
    return qw.cpu().numpy(), bits_of(s), bits_of(z)


@pytest.mark.parametrize("name", CASES)
def test_quantize_golden_bit_exact(name):
    g, dt = _G[name + "__meta"]
    dt = "bf16" if dt == 0 else "fp16"
    print(f"[quantize golden] {name}", flush=True)
    qw, s, z = _quantize_np(_to_dev(_G[name + "__w"], dt), int(g))
    np.testing.assert_array_equal(qw, _G[name + "__qweight"])
    np.testing.assert_array_equal(s, _G[name + "__scales"])
    np.testing.assert_array_equal(z, _G[name + "__zeros"])


def test_quantize_golden_hashes_large():
    meta = json.loads((GOLDEN / "quantize_golden_hashes.json").read_text())
    for c in meta["cases"]:
        print(f"[quantize hash] {c['n']}x{c['k']} G={c['group_size']} {c['dtype']}", flush=True)
        bits = synth_weight_bits(c["n"], c["k"], c["seed"], c["dtype"], c["sigma"])
        qw, s, z = _quantize_np(_to_dev(bits, c["dtype"]), c["group_size"])
        assert sha(qw) == c["qweight_sha256"], c
        assert sha(s) == c["scales_sha256"], c
        assert sha(z) == c["zeros_sha256"], c


QCASES = ([(shape, g) for shape in LLAMA[:3] for g in (32, 128, -1)]
          + [((2048, 2048), g) for g in (8, 16, 64, 256, 512, 1024)]
          + [((100, 256), g) for g in (8, 32, 64, 128, 256, -1)]
          + [((73, 1024), g) for g in (16, 128, 1024)])


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("shape,g", QCASES)
def test_quantize_matches_oracle(shape, g, dt):
    N, K = shape
    print(f"[quantize] {shape} G={g} {dt}", flush=True)
    w = randn(shape, seed=N + K + max(g, 0), sigma=0.02, dtype=TDT[dt])
    qw, s, z = _quantize_np(w.to(DEV), g)
    rq, rs, rz = O.quantize_int4(bits_of(w), dt, g)
    np.testing.assert_array_equal(qw, rq)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(z, rz)


@pytest.mark.parametrize("layout", ["transposed", "sliced", "unaligned"])
def test_quantize_strided_input(layout):
    base = randn((512, 640), seed=3, sigma=0.02)
    views = {
        "transposed": lambda b: b.t(),              # [640, 512], stride_wk = 640
        "sliced": lambda b: b[:, 64:576],           # row stride 640, 16-byte aligned
        "unaligned": lambda b: b[:, 3:515],         # row stride 640, 6-byte offset
    }
    w = views[layout](base)
    assert not w.is_contiguous()
    qw, s, z = _quantize_np(views[layout](base.to(DEV)), 128)
    rq, rs, rz = O.quantize_int4(bits_of(w.contiguous()), "bf16", 128)
    np.testing.assert_array_equal(qw, rq)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(z, rz)


def test_memory_reduction_and_error():
    # int4_triton tests/test_kernels.py:34-44
    N, K = 2048, 8192
    w = (randn((N, K), seed=0, sigma=0.02, dtype=torch.float32)).half().to(DEV)
    qw, s, z = int4_hip.quantize_int4(w, 128)
    assert qw.dtype == torch.int32 and qw.shape == (K // 8, N)
    assert w.numel() * w.element_size() == 4 * qw.numel() * qw.element_size()
    w_hat = int4_hip.dequantize_int4(qw, s, z)
    step = s.t().repeat_interleave(128, dim=1).float()
    assert ((w_hat.float() - w.float()).abs() <= step * 0.5 + 1e-3).all()


@pytest.mark.parametrize("odt", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("name", CASES)
def test_dequantize_golden(name, odt):
    g, dt = _G[name + "__meta"]
    qw = torch.from_numpy(_G[name + "__qweight"]).to(DEV)
    s = _to_dev(_G[name + "__scales"], "fp16")
    z = _to_dev(_G[name + "__zeros"], "fp16")
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[odt]
    out = int4_hip.dequantize_int4(qw, s, z, tdt).cpu()
    if odt == "fp32":
        assert_bits_equal_nan_aware(out.numpy().view(np.uint32), _G[name + "__deq_fp32"].view(np.uint32), "fp32", name)
    else:
        assert_bits_equal_nan_aware(bits_of(out), _G[name + "__deq_" + odt], odt, name)


@pytest.mark.parametrize("g", [32, 128])
def test_dequantize_matches_oracle_large(g):
    w = randn((2048, 2048), seed=5, sigma=0.02)
    qw, s, z = int4_hip.quantize_int4(w.to(DEV), g)
    out = int4_hip.dequantize_int4(qw, s, z, torch.bfloat16).cpu()
    ref = O.f32_to_bf16_bits(O.dequantize_int4(qw.cpu().numpy(), bits_of(s), bits_of(z), "bf16"))
    np.testing.assert_array_equal(bits_of(out), ref)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("g", [32, 128])
def test_quantize_rounding_boundaries(dt, g):
    """Weights at and a few ulps around (k + 1/2) * scale, where
    floor(w / scale + 0.5) changes value: the kernel's reciprocal path must
    defer to the exact division on every one of them."""
    N, K = 256, 1024
    rng = np.random.default_rng(11 + g)
    tdt = TDT[dt]
    ngroups = K // g
    # scales m * 2^e (m odd, <= 7) keep 15 * scale and every (k + 1/2) * scale
    # exactly representable in bf16 and fp16, so exact ties occur
    m = rng.choice([1.0, 3.0, 5.0, 7.0], (N, ngroups))
    e = rng.integers(-12, -7, (N, ngroups)).astype(np.float64)
    scale = torch.from_numpy((m * 2.0 ** e).astype(np.float32))
    k = torch.from_numpy(rng.integers(-5, 9, (N, K)).astype(np.float32))
    w = ((k + 0.5) * scale.repeat_interleave(g, dim=1)).to(tdt)
    # nudge by -2..2 ulps of the weight dtype
    bits = w.view(torch.int16).to(torch.int32)
    bits = bits + torch.from_numpy(rng.integers(-2, 3, (N, K)).astype(np.int32))
    w = bits.to(torch.int16).view(tdt)
    # pin each group's range to [-5, 10] * scale: the scale is the chosen one
    # and the zero point 5
    w[:, 0::g] = (-5.0 * scale).to(tdt)
    w[:, 1::g] = (10.0 * scale).to(tdt)
    print(f"[quantize boundaries] G={g} {dt}", flush=True)
    qw, s, z = _quantize_np(w.to(DEV), g)
    rq, rs, rz = O.quantize_int4(bits_of(w), dt, g)
    np.testing.assert_array_equal(qw, rq)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(z, rz)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("g", [8, 16, 32, 64, 128, 256, 512, 1024, -1])
def test_quantize_degenerate_groups_every_width(dt, g):
    """NaN, +-inf, zero / underflowing / overflowing scales, ties and signed
    zeros at every group width (every lane-reduction width of the kernels),
    interleaved with ordinary rows: bit-exact against the oracle."""
    from golden.make_golden import degenerate_rows_f32, f32_to_bf16_bits

    K = 2 * g if g > 0 else 512
    rng = np.random.default_rng(100 + max(g, 0))
    deg = degenerate_rows_f32(K, g if g > 0 else K // 2, rng)  # (the generator places patterns per half row)
    ordinary = (rng.standard_normal((deg.shape[0], K)) * 0.02).astype(np.float32)
    w = np.empty((2 * deg.shape[0] + 1, K), np.float32)
    w[0:-1:2], w[1:-1:2], w[-1] = deg, ordinary, deg[4]  # odd N: a partial column strip
    with np.errstate(over="ignore"):  # the 1e30 row overflows fp16 on purpose
        bits = f32_to_bf16_bits(w) if dt == "bf16" else w.astype(np.float16).view(np.uint16)
    print(f"[quantize degenerate] G={g} {dt} {w.shape}", flush=True)
    qw, s, z = _quantize_np(_to_dev(bits, dt), g)
    rq, rs, rz = O.quantize_int4(bits, dt, g)
    np.testing.assert_array_equal(qw, rq)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(z, rz)


# grouped quantize (one launch for the weights of a block): every output bit
# equal to the lone kernel's, on the block's shapes and on the routes that fall
# back to one launch per weight (mixed group sizes, strided rows, G = K)
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("G", [32, 128, 512])
def test_quantize_grouped_matches_lone(dt, G):
    shapes = [(2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (8192, 2048), (8192, 2048), (2048, 8192),
              (100, 1024)]
    print(f"[quantize grouped] G={G} {dt}", flush=True)
    ws = [randn((N, K), seed=900 + i, sigma=0.02, dtype=dt).to(DEV) for i, (N, K) in enumerate(shapes)]
    ws[-1][3, 5] = float("nan")  # a NaN group takes the exact path in both
    grouped = int4_hip.quantize_int4_grouped(ws, G)
    for w, (gq, gs, gz) in zip(ws, grouped):
        q, s, z = int4_hip.quantize_int4(w, G)
        assert torch.equal(gq, q)
        assert torch.equal(gs.view(torch.int16), s.view(torch.int16))
        assert torch.equal(gz.view(torch.int16), z.view(torch.int16))


@pytest.mark.parametrize("case", ["mixed_groups", "strided", "per_channel"])
def test_quantize_grouped_fallbacks(case):
    print(f"[quantize grouped fallback] {case}", flush=True)
    ws = [randn((300, 1024), seed=950 + i, sigma=0.02).to(DEV) for i in range(3)]
    if case == "strided":
        ws[1] = randn((300, 2048), seed=960, sigma=0.02).to(DEV)[:, ::2]
    gsz = -1 if case == "per_channel" else 128
    outs = int4_hip.quantize_int4_grouped(ws, gsz)
    if case == "mixed_groups":  # the Python API takes one group size; the C-ABI takes one per weight
        outs = None
    for w, o in zip(ws, outs or []):
        q, s, z = int4_hip.quantize_int4(w, gsz)
        assert torch.equal(o[0], q) and torch.equal(o[1].view(torch.int16), s.view(torch.int16))
        assert torch.equal(o[2].view(torch.int16), z.view(torch.int16))
    if case == "mixed_groups":
        from int4_hip import _lib
        lib = _lib.load()
        gs = [32, 128, 64]
        probs = (_lib.QuantProblem * 3)()
        outs = []
        for i, (w, g) in enumerate(zip(ws, gs)):
            N, K = w.shape
            o = (torch.empty((K // 8, N), dtype=torch.int32, device=DEV),
                 torch.empty((K // g, N), dtype=torch.float16, device=DEV),
                 torch.empty((K // g, N), dtype=torch.float16, device=DEV))
            probs[i] = _lib.QuantProblem(w.data_ptr(), o[0].data_ptr(), o[1].data_ptr(), o[2].data_ptr(), N, K,
                                         w.stride(0), w.stride(1), g, 0)
            outs.append(o)
        _lib.check(lib.w4_quantize_grouped(probs, 3, _lib.DTYPE_BF16, torch.cuda.current_stream().cuda_stream),
                   "w4_quantize_grouped")
        for w, g, o in zip(ws, gs, outs):
            q, s, z = int4_hip.quantize_int4(w, g)
            assert torch.equal(o[0], q) and torch.equal(o[1].view(torch.int16), s.view(torch.int16))
