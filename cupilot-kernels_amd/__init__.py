"""MI355X (gfx950) GEMM-family operators: a drop-in for the GEMM path of
champloo2878/cuPilot-Kernels (kernels/1..18), its pointwise convolution
(kernels/87) and its scaled dot-product attention (kernels/97).

    import torch
    from __graft_entry__ import load_package
    ck = load_package()                 # this directory as ``cupilot_kernels_amd``
    C = ck.p01.matmul_cuda(A, B)        # the reference's own function names
    C = ck.ModelNew(16)(A, B)           # KernelBench-style module for PID 16

Layers (top to bottom): the per-PID Python submodules and ``ModelNew``
(models.py) -> the ATen operator layer (_C, csrc/aten_ops.cpp) -> the C ABI
(include/mi355_gemm.h, libmi355gemm.so; ctypes binding in abi.py) -> the tile
scheduler (csrc/scheduler.cpp) -> the gfx950 kernels (csrc/*.hip).

There is no CPU or PyTorch fallback: importing this package without the built
extension raises ImportError.
"""
import importlib

import torch  # noqa: F401  -- load torch's HIP runtime before the native libraries

try:
    _C = importlib.import_module(__name__ + "._C")
except ImportError as e:  # pragma: no cover - exercised when the build is missing
    raise ImportError(
        "cupilot-kernels_amd native extension is not built "
        "(run `python cupilot-kernels_amd/build.py`): " + str(e)) from e

from . import abi  # noqa: E402
from .models import ModelNew, PIDS, OPS  # noqa: E402,F401

p01, p02, p03, p04, p05 = _C.p01, _C.p02, _C.p03, _C.p04, _C.p05
p06, p07, p08, p09 = _C.p06, _C.p07, _C.p08, _C.p09
p10, p11, p12, p13 = _C.p10, _C.p11, _C.p12, _C.p13
p14, p15, p16, p17, p18 = _C.p14, _C.p15, _C.p16, _C.p17, _C.p18
p87, p97 = _C.p87, _C.p97

__version__ = _C.version()
