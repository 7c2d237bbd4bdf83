"""CPU pinning of the product's torch-op functions (``int4_hip.quantize``):
``quantize_int4_ref``, ``unpack_int4_ref``, ``dequantize_int4_ref`` and the
CPU route of ``Int4Linear.dequantize``.

They are the API counterparts of int4_triton/quantize.py:102-135 and the
torch CPU path the bench times as its CPU baseline; each is checked bit for
bit against the golden vectors the reference's own functions wrote
(tests/golden/), including the degenerate groups (NaN/Inf weights,
underflowing scales, .5 ties, signed zeros, the int32 wrap of nibble 7) and
the sha256 hashes of large seeded cases.  A planted mistake (OR-ing the
nibbles one place off) must fail the same comparison.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import int4_hip
from int4_hip import quantize as Q
from golden.make_golden import sha, synth_weight_bits
from _synth import assert_bits_equal_nan_aware

GOLDEN = Path(__file__).resolve().parent / "golden"
_G = np.load(GOLDEN / "quantize_golden.npz")
CASES = sorted({k.split("__")[0] for k in _G.files})
_TDT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _weight(name):
    g, dt = _G[name + "__meta"]
    dt = "bf16" if dt == 0 else "fp16"
    bits = _G[name + "__w"].astype(np.int16)
    return torch.from_numpy(bits).view(_TDT[dt]), dt, int(g)


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("name", CASES)
def test_quantize_ref_matches_golden(name):
    w, _, g = _weight(name)
    qw, s, z = int4_hip.quantize_int4_ref(w, g)
    assert qw.dtype == torch.int32 and s.dtype == z.dtype == torch.float16
    assert qw.is_contiguous() and s.is_contiguous() and z.is_contiguous()
    np.testing.assert_array_equal(qw.numpy(), _G[name + "__qweight"])
    np.testing.assert_array_equal(_bits16(s), _G[name + "__scales"])
    np.testing.assert_array_equal(_bits16(z), _G[name + "__zeros"])


@pytest.mark.parametrize("name", CASES)
def test_unpack_and_dequantize_ref_match_golden(name):
    qw = torch.from_numpy(_G[name + "__qweight"])
    s = torch.from_numpy(_G[name + "__scales"].astype(np.int16)).view(torch.float16)
    z = torch.from_numpy(_G[name + "__zeros"].astype(np.int16)).view(torch.float16)
    np.testing.assert_array_equal(int4_hip.unpack_int4_ref(qw).numpy(), _G[name + "__unpacked"])
    for dt in ("bf16", "fp16"):
        got = _bits16(int4_hip.dequantize_int4_ref(qw, s, z, _TDT[dt]))
        assert_bits_equal_nan_aware(got, _G[name + "__deq_" + dt], dt, f"{name} {dt}")
    f32 = int4_hip.dequantize_int4_ref(qw, s, z, torch.float32).numpy()
    assert_bits_equal_nan_aware(f32.view(np.uint32), _G[name + "__deq_fp32"].view(np.uint32), "fp32", name)
    # default dtype is fp16, as in the reference
    assert int4_hip.dequantize_int4_ref(qw, s, z).dtype == torch.float16


def test_quantize_ref_matches_reference_hashes_large():
    meta = json.loads((GOLDEN / "quantize_golden_hashes.json").read_text())
    for c in meta["cases"]:
        bits = synth_weight_bits(c["n"], c["k"], c["seed"], c["dtype"], c["sigma"])
        w = torch.from_numpy(bits.astype(np.int16)).view(_TDT[c["dtype"]])
        qw, s, z = int4_hip.quantize_int4_ref(w, c["group_size"])
        assert sha(qw.numpy()) == c["qweight_sha256"], c
        assert sha(_bits16(s)) == c["scales_sha256"], c
        assert sha(_bits16(z)) == c["zeros_sha256"], c


def test_planted_nibble_order_mistake_is_caught():
    name = "normal_bf16_g128"
    w, _, g = _weight(name)
    qw, _, _ = int4_hip.quantize_int4_ref(w, g)
    codes = int4_hip.unpack_int4_ref(qw).reshape(qw.shape[1], -1, 8)
    wrong = codes[..., 1].clone()  # nibbles shifted one place
    for i in range(1, 8):
        wrong |= codes[..., (i + 1) % 8] << (4 * i)
    assert not np.array_equal(wrong.t().contiguous().numpy(), _G[name + "__qweight"])


def test_int4linear_dequantize_on_cpu_buffers():
    """A state dict loaded on the CPU dequantizes there (the reference's
    Int4Linear.dequantize is device-agnostic, qlinear.py:39-40)."""
    name = "normal_bf16_g128"
    qw = torch.from_numpy(_G[name + "__qweight"])
    s = torch.from_numpy(_G[name + "__scales"].astype(np.int16)).view(torch.float16)
    z = torch.from_numpy(_G[name + "__zeros"].astype(np.int16)).view(torch.float16)
    K, N = qw.shape[0] * 8, qw.shape[1]
    layer = int4_hip.Int4Linear(K, N, group_size=K // s.shape[0], device="cpu")
    layer.load_state_dict({"qweight": qw, "scales": s, "zeros": z})
    got = layer.dequantize()  # default bf16
    assert got.dtype == torch.bfloat16
    np.testing.assert_array_equal(_bits16(got), _G[name + "__deq_bf16"])


def test_quantize_name_is_callable_and_a_module():
    # north_star's quantize() and the reference's `from int4_triton.quantize import ...`
    assert Q is int4_hip.quantize and callable(int4_hip.quantize)
    assert int4_hip.quantize.unpack_int4_ref is int4_hip.unpack_int4_ref
    with pytest.raises(AssertionError):  # same checks as quantize_int4 (CPU tensor)
        int4_hip.quantize(torch.zeros(8, 64, dtype=torch.bfloat16), 32)
