"""mi_gemm_f32_noalloc (the allocation-free variant of mi_gemm_f32) against
mi_gemm_f32 with a workspace, through the C ABI: the same plan, so the same
bits, and within the north-star tolerance of the fp64 oracle.  Two calls in a
row, the second on a smaller problem (the fixed device array keeps the first
call's partials; nothing may depend on them)."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, cur_stream, gemm_args, run_gemm, to_dev, to_host, workspace

pytestmark = pytest.mark.gpu


def _pair(ck, orc, M, N, K, op_a, op_b, seed):
    L = ck.abi.lib()
    a = orc.uniform((M, K) if op_a == 0 else (K, M), seed)
    b = orc.uniform((K, N) if op_b == 0 else (N, K), seed + 1)
    A, B = to_dev(a), to_dev(b)
    C_ref = torch.empty((M, N), device="cuda")
    C_na = torch.full((M, N), float("nan"), device="cuda")
    args = gemm_args(ck, A, B, C_ref, M, N, K, op_a=op_a, op_b=op_b)
    plan_rc, plan = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b)
    assert plan_rc == 0
    ws = workspace(ck, args)
    args_ws = gemm_args(ck, A, B, C_ref, M, N, K, op_a=op_a, op_b=op_b, ws=ws)
    ck.abi.check(run_gemm(ck, args_ws), "mi_gemm_f32")
    args_na = gemm_args(ck, A, B, C_na, M, N, K, op_a=op_a, op_b=op_b)
    ck.abi.check(L.mi_gemm_f32_noalloc(ctypes.byref(args_na), cur_stream()), "mi_gemm_f32_noalloc")
    got, want = to_host(C_na), to_host(C_ref)
    np.testing.assert_array_equal(got, want)
    la = a if op_a == 0 else a.T
    lb = b if op_b == 0 else b.T
    assert_close(orc, got, orc.gemm(la, lb), K, what=f"noalloc {M}x{N}x{K}")
    return ws is not None


@pytest.mark.parametrize("first,second", [
    ((256, 256, 1 << 18, 0, 0), (128, 192, 1 << 16, 0, 0)),   # split-K both times
    ((512, 512, 8192, 0, 0), (520, 264, 1000, 1, 1)),        # k-split tile split 4, then odd T/T
    ((2048, 2048, 2048, 0, 1), (64, 64, 4096, 1, 0)),        # unsplit, then split-K
    ((1280, 1280, 8192, 0, 0), (1024, 2048, 8192, 1, 0)),    # stream-K, then split-K
])
def test_noalloc_matches_workspace_entry_point(ck, orc, dev, first, second):
    used = [_pair(ck, orc, *first, seed=1200), _pair(ck, orc, *second, seed=1300)]
    if first[2] >= 1 << 16:
        assert used[0], "the first case is meant to take split-K"
    if first[:3] == (1280, 1280, 8192):
        rc, p = ck.abi.plan(*first[:3], workspace_bytes=1 << 40)
        assert rc == 0 and p.stream_k == 1 and used[0]


def _limited(ck, orc, M, N, K, op_a, op_b, seed):
    """A problem whose preferred plan wants more scratch than the array: the
    no-alloc call runs the plan mi_gemm_f32 picks with a workspace of exactly
    the array's size (same bits), within tolerance of the oracle."""
    L = ck.abi.lib()
    lim = ck.abi.NOALLOC_SCRATCH_BYTES
    rc, pref = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40)
    assert rc == 0 and pref.workspace_bytes > lim
    rc, fit = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, workspace_bytes=lim)
    assert rc == 0 and fit.workspace_bytes <= lim
    a = orc.uniform((M, K) if op_a == 0 else (K, M), seed)
    b = orc.uniform((K, N) if op_b == 0 else (N, K), seed + 1)
    A, B = to_dev(a), to_dev(b)
    ws = torch.empty(lim, dtype=torch.uint8, device="cuda")
    C_ref = torch.empty((M, N), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C_ref, M, N, K, op_a=op_a, op_b=op_b, ws=ws)),
                 "mi_gemm_f32 with a scratch-sized workspace")
    C_na = torch.full((M, N), float("nan"), device="cuda")
    args_na = gemm_args(ck, A, B, C_na, M, N, K, op_a=op_a, op_b=op_b)
    ck.abi.check(L.mi_gemm_f32_noalloc(ctypes.byref(args_na), cur_stream()), "mi_gemm_f32_noalloc")
    got = to_host(C_na)
    np.testing.assert_array_equal(got, to_host(C_ref))
    la = a if op_a == 0 else a.T
    lb = b if op_b == 0 else b.T
    assert_close(orc, got, orc.gemm(la, lb), K, what=f"noalloc limited {M}x{N}x{K}")


def test_noalloc_plans_within_its_scratch(ck, orc, dev):
    """Preferred plans past the 64 MiB array (1280 x 1024 x 8192: split 16 of
    5 MiB partials, 80 MiB) take the best plan that fits it instead of being
    refused; then a smaller split-K problem in the same array."""
    _limited(ck, orc, 1280, 1024, 8192, 0, 0, 1400)
    _limited(ck, orc, 1280, 512, 65536, 1, 0, 1410)
    _pair(ck, orc, 128, 192, 1 << 16, 0, 0, seed=1420)


def test_noalloc_rejects_forced_plans_beyond_its_scratch(ck, dev):
    L = ck.abi.lib()
    M = N = 2048                       # split 8 of 16 MiB partials: 128 MiB
    K = 1 << 20
    args = ck.abi.make_args(M, N, K, plan_override=3 | (8 << 8))
    need = L.mi_gemm_workspace_bytes(ctypes.byref(args))
    assert need > ck.abi.NOALLOC_SCRATCH_BYTES
    # nothing is launched: the operands are never touched
    assert L.mi_gemm_f32_noalloc(ctypes.byref(args), cur_stream()) == ck.abi.MI_ERR_SCRATCH_LIMIT
    assert b"64 MiB" in L.mi_status_string(ck.abi.MI_ERR_SCRATCH_LIMIT)
