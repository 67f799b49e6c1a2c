"""Build the package's native code in-tree.

  libmi355gemm.so  HIP kernels for gfx950 + tile scheduler + C ABI  (Makefile, hipcc)
  _C.<abi>.so      ATen operator layer + Python module, linked to libmi355gemm.so

Run ``python cupilot-kernels_amd/build.py`` or call ``build()``.  Both outputs
land next to this file so they travel with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _ext_name() -> str:
    return "_C" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so")


def build_hip(jobs: int = 8) -> str:
    subprocess.run(["make", "-s", "-C", HERE, f"-j{jobs}"], check=True)
    return os.path.join(HERE, "libmi355gemm.so")


def build_aten() -> str:
    import torch
    from torch.utils import cpp_extension

    out = os.path.join(HERE, _ext_name())
    src = os.path.join(HERE, "csrc", "aten_ops.cpp")
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        "g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-I{sysconfig.get_paths()['include']}",
        f"-I{ROCM}/include",
    ]
    cmd += [f"-I{p}" for p in cpp_extension.include_paths()]
    cmd += [src, "-o", out + ".tmp",
            f"-L{HERE}", "-lmi355gemm", "-Wl,-rpath,$ORIGIN",
            f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    subprocess.run(cmd, check=True)
    os.replace(out + ".tmp", out)
    return out


def build() -> None:
    build_hip()
    build_aten()


if __name__ == "__main__":
    build()
    print("built", os.path.join(HERE, "libmi355gemm.so"), os.path.join(HERE, _ext_name()))
    sys.exit(0)
