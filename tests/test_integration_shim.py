"""The ``int4_triton`` drop-in shim (itmo-final-project_amd/dropin): in a fresh
interpreter, every name the reference's scripts and tests import resolves to
this backend's object (benchmarks/bench_gemm.py:15, benchmarks/eval_llama.py:31,
tests/test_kernels.py:4-12 of the reference).  CPU only: nothing is launched."""
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
DROPIN = ROOT / "itmo-final-project_amd" / "dropin"

PROBE = r"""
import int4_triton, int4_hip
from int4_triton import quantize_int4, w4a16_matmul, w16a16_matmul
from int4_triton import Int4Linear, quantize_model_linears
from int4_triton import dequantize_int4_ref, quantize_int4_ref
from int4_triton.quantize import unpack_int4_ref
from int4_triton.gemm import w4a16_matmul as mm
from int4_triton.qlinear import Int4Linear as L
assert quantize_int4 is int4_hip.quantize_int4 and w4a16_matmul is int4_hip.w4a16_matmul is mm
assert Int4Linear is int4_hip.Int4Linear is L and unpack_int4_ref is int4_hip.unpack_int4_ref
assert quantize_model_linears is int4_hip.quantize_model_linears
print("shim ok")
"""


def test_shim_resolves_reference_imports():
    env = {k: v for k, v in os.environ.items() if k != "PYTHONPATH"}
    env["PYTHONPATH"] = str(DROPIN)
    r = subprocess.run([sys.executable, "-c", PROBE], env=env, capture_output=True, text=True, timeout=300,
                       cwd="/")
    assert r.returncode == 0 and "shim ok" in r.stdout, r.stderr[-2000:]
