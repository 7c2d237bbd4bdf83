"""Build libint4_hip.so (gfx950) in-tree with hipcc.

    python itmo-final-project_amd/build_lib.py [--jobs N]

Every call recompiles every source (object files go to ``_build/``, the
library to ``int4_hip/libint4_hip.so``).  hipcc cross-compiles for gfx950 on a
machine without a GPU.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "int4_hip" / "libint4_hip.so"
# measurement helpers for bench.py (not part of the library)
BENCH_SRC = CSRC / "bench"
BENCH_LIB = HERE / "int4_hip" / "libw4_bench.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU instructions stay off: ordinary float code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(ROOT / "include"),
    "-I", str(CSRC),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm not installed?)")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = BUILD / ((src.parent.name + "_" if src.parent == BENCH_SRC else "") + src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [hipcc(), "-O3", "-std=c++17", "-fPIC", "-I", str(ROOT / "include"), "-I", str(CSRC),
               "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{err}")
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    bench_srcs = sorted(list(BENCH_SRC.glob("*.hip")) + list(BENCH_SRC.glob("*.cpp")))
    if bench_srcs:
        bobjs = [_compile(s) for s in bench_srcs]
        btmp = BENCH_LIB.with_suffix(".so.tmp")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(btmp), *map(str, bobjs)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stderr}")
        os.replace(btmp, BENCH_LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources (+ {BENCH_LIB.name})", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    build(ap.parse_args().jobs)
