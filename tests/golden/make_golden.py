"""Write golden vectors for the quantize/unpack/dequantize oracle.

Run once, in the build container where the reference checkout exists:

    python tests/golden/make_golden.py /root/reference

It imports the reference's pure-torch functions ``quantize_int4_ref``,
``unpack_int4_ref`` and ``dequantize_int4_ref`` (int4_triton/quantize.py:102-135)
and runs them on the CPU.  Nothing from the reference is copied: only inputs
and outputs are written, as data:

* ``quantize_golden.npz``: small inputs (bit patterns) with the reference's
  outputs, covering the degenerate groups that no closed form pins
  (fp16-underflowing scales, NaN/Inf weights, exact .5 ties, signed zeros,
  per-channel G=-1, fp16 input, int32 wrap of nibble 7);
* ``quantize_golden_hashes.json``: sha256 of the reference's outputs for
  larger seeded inputs whose recipe (``synth_weight_bits`` below) the tests
  rebuild bit for bit.

The tests never import the reference; they only read these files.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    out = ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), out).astype(np.uint16)


def synth_weight_bits(n: int, k: int, seed: int, dtype: str, sigma: float = 0.02) -> np.ndarray:
    """Seeded N(0, sigma) weight as bf16/fp16 bit patterns (one rounding from fp32)."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(sigma)
    if dtype == "bf16":
        return f32_to_bf16_bits(w)
    return w.astype(np.float16).view(np.uint16)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def degenerate_rows_f32(k: int, g: int, rng: np.random.Generator) -> np.ndarray:
    """float32 rows, one degenerate pattern per row (each row is K = 2 groups)."""
    rows = []
    z = np.zeros(k, np.float32)
    rows.append(z.copy())                                      # all-zero groups -> scale 1
    rows.append(np.full(k, 0.5, np.float32))                   # closed form: q=15, s=0.0333251953125
    rows.append((rng.standard_normal(k) * 1e-8).astype(np.float32))   # fp16 scale underflows to 0
    rows.append((np.abs(rng.standard_normal(k)) * 1e-9).astype(np.float32))  # wmin = 0, scale 0 -> 0/0
    r = (rng.standard_normal(k) * 0.02).astype(np.float32); r[3] = np.nan
    rows.append(r)                                             # NaN in first group
    r = (rng.standard_normal(k) * 0.02).astype(np.float32); r[g + 5] = np.inf
    rows.append(r)                                             # +inf in second group
    r = (rng.standard_normal(k) * 0.02).astype(np.float32); r[1] = -np.inf
    rows.append(r)                                             # -inf
    rows.append(np.full(k, -0.0, np.float32))                  # signed zeros
    ties = np.array([-7.5, 7.5, -2.5, 2.5, 0.5, -0.5, 1.5, -1.5], np.float32)
    rows.append(np.resize(ties, k))                            # range 15 -> scale exactly 1, .5 ties
    rows.append((rng.standard_normal(k) * 1e30).astype(np.float32))  # fp16 scale overflows to inf
    rows.append((0.1 + 0.1 * rng.random(k)).astype(np.float32))       # all positive: wmin clamps to 0
    rows.append((-0.1 - 0.1 * rng.random(k)).astype(np.float32))      # all negative: wmax clamps to 0
    rows.append((rng.standard_normal(k) * 2e-7).astype(np.float32))   # subnormal fp16 scale
    r = np.resize(np.array([3.0e38, -3.0e38], np.float32), k)
    rows.append(r)                                             # wmax - wmin overflows fp32
    r = (rng.standard_normal(k) * 0.02).astype(np.float32); r[::8] = 0.3
    rows.append(r)                                             # nibble 0 large
    r = (rng.standard_normal(k) * 0.02).astype(np.float32); r[7::8] = 0.3
    rows.append(r)                                             # nibble 7 >= 8: int32 sign bit
    return np.stack(rows)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from int4_triton.quantize import dequantize_int4_ref, quantize_int4_ref, unpack_int4_ref

    def to_torch(bits: np.ndarray, dtype: str) -> torch.Tensor:
        t = torch.from_numpy(bits.view(np.int16).copy())
        return t.view(torch.bfloat16 if dtype == "bf16" else torch.float16)

    def run(bits: np.ndarray, dtype: str, g: int):
        w = to_torch(bits, dtype)
        qw, s, z = quantize_int4_ref(w, g)
        out = {
            "qweight": qw.numpy(),
            "scales": s.view(torch.int16).numpy().view(np.uint16),
            "zeros": z.view(torch.int16).numpy().view(np.uint16),
            "unpacked": unpack_int4_ref(qw).numpy(),
            "deq_bf16": dequantize_int4_ref(qw, s, z, torch.bfloat16).view(torch.int16).numpy().view(np.uint16),
            "deq_fp16": dequantize_int4_ref(qw, s, z, torch.float16).view(torch.int16).numpy().view(np.uint16),
            "deq_fp32": dequantize_int4_ref(qw, s, z, torch.float32).numpy(),
        }
        return out

    rng = np.random.default_rng(20240607)
    cases = {}
    # normal groups
    cases["normal_bf16_g32"] = (synth_weight_bits(16, 256, 1, "bf16"), "bf16", 32)
    cases["normal_bf16_g128"] = (synth_weight_bits(24, 256, 2, "bf16"), "bf16", 128)
    cases["normal_bf16_gm1"] = (synth_weight_bits(8, 256, 3, "bf16"), "bf16", -1)
    cases["normal_fp16_g64"] = (synth_weight_bits(16, 256, 4, "fp16"), "fp16", 64)
    cases["normal_fp16_g32_n100"] = (synth_weight_bits(100, 64, 5, "fp16"), "fp16", 32)
    # degenerate groups
    d = degenerate_rows_f32(64, 32, rng)
    cases["degenerate_bf16_g32"] = (f32_to_bf16_bits(d), "bf16", 32)
    d16 = np.where(np.abs(d) > 6e4, np.sign(d) * 6e4, d).astype(np.float32)
    cases["degenerate_fp16_g32"] = (d16.astype(np.float16).view(np.uint16), "fp16", 32)
    cases["degenerate_bf16_g64"] = (f32_to_bf16_bits(d), "bf16", 64)

    arrays = {}
    for name, (bits, dtype, g) in cases.items():
        out = run(bits, dtype, g)
        arrays[f"{name}__w"] = bits
        arrays[f"{name}__meta"] = np.array([g, 0 if dtype == "bf16" else 1], np.int32)
        for k, v in out.items():
            arrays[f"{name}__{k}"] = v
    np.savez_compressed(HERE / "quantize_golden.npz", **arrays)

    hashed = []
    for (n, k, seed, dtype, g) in [
        (2048, 2048, 1234, "bf16", 128),
        (512, 2048, 0, "fp16", 32),
        (2048, 8192, 7, "bf16", 128),
        (100, 256, 9, "bf16", -1),
        (8192, 2048, 11, "bf16", 64),
    ]:
        bits = synth_weight_bits(n, k, seed, dtype)
        out = run(bits, dtype, g)
        hashed.append({
            "n": n, "k": k, "seed": seed, "dtype": dtype, "group_size": g, "sigma": 0.02,
            "qweight_sha256": sha(out["qweight"]),
            "scales_sha256": sha(out["scales"]),
            "zeros_sha256": sha(out["zeros"]),
        })
    (HERE / "quantize_golden_hashes.json").write_text(json.dumps({
        "recipe": "numpy.random.default_rng(seed).standard_normal((n,k), float32) * float32(sigma), "
                  "one RNE cast to the weight dtype",
        "torch": torch.__version__,
        "cases": hashed,
    }, indent=1) + "\n")
    print("wrote", HERE / "quantize_golden.npz", "and", HERE / "quantize_golden_hashes.json")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
