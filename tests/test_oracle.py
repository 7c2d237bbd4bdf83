"""Pin the CPU oracle (oracle/w4a16_oracle.py) before trusting it.

Checks, in order of strength:
1. golden vectors written by the reference's own torch functions
   (tests/golden/make_golden.py, int4_triton/quantize.py:102-135);
2. closed forms fixed by the formula (README.md:34-38 of the reference);
3. invariants (tests/test_kernels.py:34-44 of the reference);
4. planted mistakes: variants of the oracle with a plausible bug must fail (1).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import w4a16_oracle as O
from golden.make_golden import sha, synth_weight_bits
from _synth import assert_bits_equal_nan_aware

GOLDEN = Path(__file__).resolve().parent / "golden"
_G = np.load(GOLDEN / "quantize_golden.npz")
CASES = sorted({k.split("__")[0] for k in _G.files})


def _case(name):
    g, dt = _G[name + "__meta"]
    return _G[name + "__w"], ("bf16" if dt == 0 else "fp16"), int(g)


@pytest.mark.parametrize("name", CASES)
def test_quantize_matches_reference_golden(name):
    w, dt, g = _case(name)
    qw, s, z = O.quantize_int4(w, dt, g)
    assert qw.dtype == np.int32 and qw.shape == (w.shape[1] // 8, w.shape[0])
    np.testing.assert_array_equal(qw, _G[name + "__qweight"])
    np.testing.assert_array_equal(s, _G[name + "__scales"])
    np.testing.assert_array_equal(z, _G[name + "__zeros"])


@pytest.mark.parametrize("name", CASES)
def test_unpack_dequant_match_reference_golden(name):
    qw, s, z = (_G[name + "__" + k] for k in ("qweight", "scales", "zeros"))
    np.testing.assert_array_equal(O.unpack_int4(qw), _G[name + "__unpacked"])
    for dt in ("bf16", "fp16"):
        mine = O.f32_to_half_bits(O.dequantize_int4(qw, s, z, dt), dt)
        assert_bits_equal_nan_aware(mine, _G[name + "__deq_" + dt], dt, f"{name} {dt}")
    f32 = O.dequantize_int4(qw, s, z, "fp32")
    assert_bits_equal_nan_aware(f32.view(np.uint32), _G[name + "__deq_fp32"].view(np.uint32), "fp32", name)


def test_quantize_matches_reference_hashes_large():
    meta = json.loads((GOLDEN / "quantize_golden_hashes.json").read_text())
    for c in meta["cases"]:
        bits = synth_weight_bits(c["n"], c["k"], c["seed"], c["dtype"], c["sigma"])
        qw, s, z = O.quantize_int4(bits, c["dtype"], c["group_size"])
        assert sha(qw) == c["qweight_sha256"], c
        assert sha(s) == c["scales_sha256"], c
        assert sha(z) == c["zeros_sha256"], c


# ------------------------------------------------------------------ closed forms
def test_closed_form_constant_half_group():
    # README formula: range 0.5 -> scale fp16(0.5/15) = 0.0333251953125, zero 0, q 15
    w = O.f32_to_bf16_bits(np.full((3, 128), 0.5, np.float32))
    qw, s, z = O.quantize_int4(w, "bf16", 128)
    assert np.all(O.f16_bits_to_f32(s) == np.float32(0.0333251953125))
    assert np.all(O.f16_bits_to_f32(z) == 0)
    assert np.all(O.unpack_int4(qw) == 15)
    assert np.all(qw == np.int32(-1))  # 0xFFFFFFFF: eight nibbles of 15, int32 wrap
    deq = O.dequantize_int4(qw, s, z, "bf16")
    assert np.all(deq == np.float32(0.5))  # 15 * 0.0333251953125 rounds to bf16 0.5


def test_closed_form_all_zero_group():
    w = np.zeros((2, 64), np.uint16)
    qw, s, z = O.quantize_int4(w, "bf16", 32)
    assert np.all(O.f16_bits_to_f32(s) == 1.0) and np.all(z == 0) and np.all(qw == 0)


def test_closed_form_known_pack_layout():
    # weight row [0..15 step] chosen so that q[k] = k % 16 with scale exactly 1:
    # range 15 (min 0, max 15) -> scale 1, zero 0, q = w.
    row = np.arange(32, dtype=np.float32) % 16
    w = O.f32_to_bf16_bits(row[None, :])
    qw, s, z = O.quantize_int4(w, "bf16", 32)
    assert O.f16_bits_to_f32(s)[0, 0] == 1.0 and z[0, 0] == 0
    # nibble i of word k8 holds row 8*k8 + i (int4_triton/quantize.py:9)
    expect = [sum(((8 * k8 + i) % 16) << (4 * i) for i in range(8)) for k8 in range(4)]
    expect = np.array(expect, dtype=np.uint64).astype(np.uint32).view(np.int32)
    np.testing.assert_array_equal(qw[:, 0], expect)


def test_unpack_brute_force_python_ints():
    rng = np.random.default_rng(5)
    qw = rng.integers(-(2**31), 2**31, size=(6, 5), dtype=np.int64).astype(np.int32)
    q = O.unpack_int4(qw)
    for k8 in range(6):
        for n in range(5):
            word = int(qw[k8, n]) & 0xFFFFFFFF
            for i in range(8):
                assert q[n, 8 * k8 + i] == (word >> (4 * i)) & 0xF


def test_dequant_single_rounding_against_exact_product():
    rng = np.random.default_rng(6)
    qw = rng.integers(-(2**31), 2**31, size=(4, 16), dtype=np.int64).astype(np.int32)
    s = O.f32_to_f16_bits(rng.random((1, 16), dtype=np.float32) * 0.01 + 1e-4)
    z = O.f32_to_f16_bits(rng.integers(0, 16, size=(1, 16)).astype(np.float32))
    q = O.unpack_int4(qw).astype(np.float64)
    exact = (q - O.f16_bits_to_f32(z).astype(np.float64).T) * O.f16_bits_to_f32(s).astype(np.float64).T
    assert np.array_equal(O.dequantize_int4(qw, s, z, "fp32").astype(np.float64), exact)
    # bf16: one RNE of the exact product (torch's own cast as the library routine)
    want = torch.from_numpy(exact).float().to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.dequantize_int4(qw, s, z, "bf16"), want)


# ------------------------------------------------------------------ invariants
@pytest.mark.parametrize("g", [32, 64, 128, -1])
@pytest.mark.parametrize("dt", ["bf16", "fp16"])
def test_invariants_random(g, dt):
    w = synth_weight_bits(96, 512, 17, dt)
    qw, s, z = O.quantize_int4(w, dt, g)
    G = 512 if g == -1 else g
    q = O.unpack_int4(qw)
    zf = O.f16_bits_to_f32(z)
    assert q.min() >= 0 and q.max() <= 15
    assert zf.min() >= 0 and zf.max() <= 15 and np.all(zf == np.floor(zf))
    w_hat = O.dequantize_int4(qw, s, z, "fp32")
    step = np.repeat(O.f16_bits_to_f32(s).T, G, axis=1)
    wf = O.half_bits_to_f32(w, dt)
    err = np.abs(w_hat - wf)
    # the reference's own bound (tests/test_kernels.py:41-44)
    assert np.all(err <= step * 0.5 + 1e-3)
    # tighter: inside the clamp range the error is half a step (to fp32 rounding) ...
    inside = (q > 0) & (q < 15)
    assert np.all(err[inside] <= step[inside] * 0.5 * (1 + 1e-6))
    # ... and the rounded zero point shifts the grid by at most half a step
    assert np.all(err <= step * (1 + 1e-6))


def test_bf16_conversion_matches_torch():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-30, 30, 100000))).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.f32_to_bf16_bits(x), want)


# ------------------------------------------------------------------ GEMM oracle
def test_gemm_oracle_matches_torch_linear():
    from _synth import bits_of, randn

    x = randn((5, 256), 1)
    w = randn((48, 256), 2, 0.02)
    qw, s, z = O.quantize_int4(bits_of(w), "bf16", 64)
    w_hat = torch.from_numpy(O.dequantize_int4(qw, s, z, "bf16"))
    ref = torch.nn.functional.linear(x.float(), w_hat)
    got = O.w4a16_matmul(bits_of(x), "bf16", qw, s, z)
    np.testing.assert_allclose(got, ref.double().numpy(), rtol=1e-5, atol=1e-5)


def test_gemm_oracle_closed_form_2pow23():
    # tests/test_kernels.py:100-110 of the reference: x = 131072, w = 0.5 -> y = 2**23
    x = O.f32_to_bf16_bits(np.full((2, 128), 131072.0, np.float32))
    w = O.f32_to_bf16_bits(np.full((7, 128), 0.5, np.float32))
    qw, s, z = O.quantize_int4(w, "bf16", 128)
    y = O.w4a16_matmul(x, "bf16", qw, s, z)
    assert np.all(y == 2.0 ** 23)


# ------------------------------------------------------------------ planted mistakes
def _mutant_quantize(w_bits, dt, g, bug):
    """The oracle with one plausible bug; the golden vectors must reject it."""
    N, K = w_bits.shape
    G = K if g == -1 else g
    wg = O.half_bits_to_f32(w_bits, dt).reshape(N, K // G, G)
    with np.errstate(all="ignore"):
        wmax = np.maximum(wg.max(-1), np.float32(0))
        wmin = np.minimum(wg.min(-1), np.float32(0))
        scale = (wmax - wmin) / np.float32(15)
        scale = np.where(scale == 0, np.float32(1), scale).astype(np.float32)
        if bug != "no_fp16_scale":
            scale = scale.astype(np.float16).astype(np.float32)
        half = np.float32(0.0 if bug == "no_half" else 0.5)
        zero = np.clip(np.floor(-wmin / scale + half), 0, 15).astype(np.float32)
        if bug == "rint":
            qf = np.rint(wg / scale[..., None]) + zero[..., None]
        elif bug == "recip":  # reciprocal multiply instead of a true division
            qf = np.floor(wg * (np.float32(1) / scale[..., None]) + half) + zero[..., None]
        else:
            qf = np.floor(wg / scale[..., None] + half) + zero[..., None]
        qf = np.clip(qf, 0, 15).astype(np.float32)
    q = O._f32_to_i32_like_torch_cpu(qf).reshape(N, K // 8, 8)
    shifts = O._SHIFTS[::-1] if bug == "nibble_order" else O._SHIFTS
    packed = (q.view(np.uint32) << shifts).sum(-1, dtype=np.uint32).view(np.int32)
    return np.ascontiguousarray(packed.T), O.f32_to_f16_bits(scale).T, O.f32_to_f16_bits(zero).T


@pytest.mark.parametrize("bug", ["recip", "no_fp16_scale", "no_half", "rint", "nibble_order"])
def test_planted_mistakes_are_caught(bug):
    caught = False
    for name in CASES:
        w, dt, g = _case(name)
        qw, s, z = _mutant_quantize(w, dt, g, bug)
        same = (np.array_equal(qw, _G[name + "__qweight"]) and np.array_equal(s, _G[name + "__scales"])
                and np.array_equal(z, _G[name + "__zeros"]))
        caught |= not same
    if not caught:  # rare-rounding bugs need the large seeded cases
        meta = json.loads((GOLDEN / "quantize_golden_hashes.json").read_text())
        for c in meta["cases"]:
            bits = synth_weight_bits(c["n"], c["k"], c["seed"], c["dtype"], c["sigma"])
            qw, s, z = _mutant_quantize(bits, c["dtype"], c["group_size"], bug)
            if (sha(qw), sha(np.ascontiguousarray(s)), sha(np.ascontiguousarray(z))) != (
                    c["qweight_sha256"], c["scales_sha256"], c["zeros_sha256"]):
                caught = True
                break
    assert caught, f"golden vectors do not detect the planted bug {bug!r}"
