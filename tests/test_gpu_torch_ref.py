"""The product's torch-op functions on GPU tensors, pinned to the golden
vectors the reference's own functions wrote (tests/golden/).

The reference's tests call ``quantize_int4_ref`` / ``dequantize_int4_ref`` on
CUDA tensors (tests/test_kernels.py:17-31,41,55,91); through the drop-in shim
those calls reach ``int4_hip.quantize_int4_ref`` and friends, so the GPU
route must give the same bits as the CPU one: division by 15 correctly
rounded (torch would otherwise multiply by the fp32 reciprocal on the GPU),
NaN codes mapped to INT32_MIN (the GPU integer cast would give 0), every
other step an IEEE operation.  Also checks them against the HIP kernels on
the large seeded cases.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import int4_hip
from golden.make_golden import sha, synth_weight_bits
from _synth import assert_bits_equal_nan_aware

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
_G = np.load(GOLDEN / "quantize_golden.npz")
CASES = sorted({k.split("__")[0] for k in _G.files})
_TDT = {"bf16": torch.bfloat16, "fp16": torch.float16}
DEV = "cuda"


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _half(name, key):
    return torch.from_numpy(_G[name + "__" + key].astype(np.int16)).view(torch.float16).to(DEV)


@pytest.mark.parametrize("name", CASES)
def test_quantize_ref_on_gpu_matches_golden(name):
    g, dt = _G[name + "__meta"]
    dt = "bf16" if dt == 0 else "fp16"
    w = torch.from_numpy(_G[name + "__w"].astype(np.int16)).view(_TDT[dt]).to(DEV)
    qw, s, z = int4_hip.quantize_int4_ref(w, int(g))
    assert qw.is_cuda and qw.dtype == torch.int32 and s.dtype == z.dtype == torch.float16
    np.testing.assert_array_equal(qw.cpu().numpy(), _G[name + "__qweight"])
    np.testing.assert_array_equal(_bits16(s), _G[name + "__scales"])
    np.testing.assert_array_equal(_bits16(z), _G[name + "__zeros"])


@pytest.mark.parametrize("name", CASES)
def test_unpack_and_dequantize_ref_on_gpu_match_golden(name):
    qw = torch.from_numpy(_G[name + "__qweight"]).to(DEV)
    s, z = _half(name, "scales"), _half(name, "zeros")
    np.testing.assert_array_equal(int4_hip.unpack_int4_ref(qw).cpu().numpy(), _G[name + "__unpacked"])
    for dt in ("bf16", "fp16"):
        got = _bits16(int4_hip.dequantize_int4_ref(qw, s, z, _TDT[dt]))
        assert_bits_equal_nan_aware(got, _G[name + "__deq_" + dt], dt, f"{name} {dt}")
    f32 = int4_hip.dequantize_int4_ref(qw, s, z, torch.float32).cpu().numpy()
    assert_bits_equal_nan_aware(f32.view(np.uint32), _G[name + "__deq_fp32"].view(np.uint32), "fp32", name)


def test_quantize_ref_on_gpu_matches_hashes_and_kernel():
    meta = json.loads((GOLDEN / "quantize_golden_hashes.json").read_text())
    for c in meta["cases"]:
        print(f"[torch ref gpu] {c['n']}x{c['k']} {c['dtype']} G={c['group_size']}", flush=True)
        bits = synth_weight_bits(c["n"], c["k"], c["seed"], c["dtype"], c["sigma"])
        w = torch.from_numpy(bits.astype(np.int16)).view(_TDT[c["dtype"]]).to(DEV)
        qw, s, z = int4_hip.quantize_int4_ref(w, c["group_size"])
        assert sha(qw.cpu().numpy()) == c["qweight_sha256"], c
        assert sha(_bits16(s)) == c["scales_sha256"], c
        assert sha(_bits16(z)) == c["zeros_sha256"], c
        kq, ks, kz = int4_hip.quantize_int4(w, c["group_size"])
        assert torch.equal(kq, qw) and torch.equal(ks.view(torch.int16), s.view(torch.int16))
        assert torch.equal(kz.view(torch.int16), z.view(torch.int16))
        deq = int4_hip.dequantize_int4_ref(qw, s, z, torch.bfloat16)
        assert torch.equal(int4_hip.dequantize_int4(qw, s, z, torch.bfloat16).view(torch.int16),
                           deq.view(torch.int16))
