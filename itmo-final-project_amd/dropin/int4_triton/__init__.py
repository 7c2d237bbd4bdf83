"""``int4_triton`` import name routed to the MI355X backend ``int4_hip``.

Put ``itmo-final-project_amd/dropin`` on ``sys.path`` ahead of the reference
checkout and the reference's scripts and tests run on the gfx950 kernels
unchanged: ``from int4_triton import quantize_int4, w4a16_matmul, ...`` and
``from int4_triton.quantize import unpack_int4_ref`` resolve to this backend's
objects of the same names.
"""
import sys
from pathlib import Path

_PKG_ROOT = str(Path(__file__).resolve().parents[2])  # holds the int4_hip package
if _PKG_ROOT not in sys.path:
    sys.path.insert(0, _PKG_ROOT)

import int4_hip  # noqa: E402
from int4_hip import *  # noqa: E402,F401,F403  the reference's public names

# the reference's submodules of the same names
for _sub in ("quantize", "gemm", "qlinear"):
    sys.modules[f"{__name__}.{_sub}"] = getattr(int4_hip, _sub)
