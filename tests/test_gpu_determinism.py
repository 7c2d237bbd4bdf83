"""Bit-identical results across processes: quantize outputs and one product
per launch regime (split-K ones included) hashed in this process and in a
fresh child process (the reference's split-K is only run-to-run
deterministic when its reduce order is fixed, gemm.py:171-182)."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

from _determinism_cases import hashes

pytestmark = pytest.mark.gpu
HERE = Path(__file__).resolve().parent


def test_bit_identical_across_processes():
    print("[determinism] in-process hashes", flush=True)
    mine = hashes()
    again = hashes()
    assert mine == again
    print("[determinism] child process", flush=True)
    env_path = [str(HERE), str(HERE.parent), str(HERE.parent / "itmo-final-project_amd")]
    code = ("import sys; sys.path[:0] = %r; from _determinism_cases import hashes; import json; "
            "print(json.dumps(hashes()))" % env_path)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-2000:]
    theirs = json.loads(r.stdout.strip().splitlines()[-1])
    assert theirs == mine
