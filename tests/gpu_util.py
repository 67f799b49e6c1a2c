"""Helpers for the GPU parity tests: device buffers, C-ABI calls, oracle checks."""
from __future__ import annotations

import ctypes

import numpy as np
import torch


def vp(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def cur_stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def dev_uniform(ck, shape, seed: int, offset: int = 0) -> torch.Tensor:
    """Device tensor filled by the library's generator (bit-identical to
    oracle.uniform(shape, seed, offset))."""
    t = torch.empty(shape, dtype=torch.float32, device="cuda")
    ck.abi.check(ck.abi.lib().mi_fill_uniform_f32(vp(t), t.numel(), seed, offset, cur_stream()),
                 "fill")
    return t


def to_dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def to_host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def gemm_args(ck, A, B, C, M, N, K, op_a=0, op_b=0, batch=1, lda=None, ldb=None, ldc=None,
              sa=0, sb=0, sc=0, structure=0, override=0, ws=None):
    a = ck.abi.GemmArgs()
    a.A = A.data_ptr() if A is not None else None
    a.B = B.data_ptr() if B is not None else None
    a.C = C.data_ptr() if C is not None else None
    a.M, a.N, a.K, a.batch = M, N, K, batch
    a.op_a, a.op_b = op_a, op_b
    a.lda = lda if lda is not None else (K if op_a == 0 else M)
    a.ldb = ldb if ldb is not None else (N if op_b == 0 else K)
    a.ldc = ldc if ldc is not None else N
    a.stride_a, a.stride_b, a.stride_c = sa, sb, sc
    a.structure = structure
    a.plan_override = override
    if ws is not None:
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel() * ws.element_size()
    # The struct holds raw pointers only; keep the tensors alive with it so a
    # caller may pass temporaries.
    a._keep = (A, B, C, ws)
    return a


def run_gemm(ck, args) -> int:
    return ck.abi.lib().mi_gemm_f32(ctypes.byref(args), cur_stream())


def workspace(ck, args):
    n = ck.abi.lib().mi_gemm_workspace_bytes(ctypes.byref(args))
    split = (args.plan_override >> 8) & 0xFFF
    if split > 1:
        # an explicit split needs split * batch * M * N floats
        n = max(n, split * max(args.batch, 1) * args.M * args.N * 4)
    return torch.empty(max(n, 1), dtype=torch.uint8, device="cuda") if n else None


def assert_close(orc, got, ref, K, amax=1.0, bmax=1.0, what=""):
    err = orc.norm_err(got, ref, K, amax, bmax)
    assert err <= orc.TOL, f"{what}: normalised error {err:.3e} > {orc.TOL}"
    return err
