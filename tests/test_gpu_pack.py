"""Operand packing on the GPU, through the C ABI: operands the 16-byte loaders
cannot stage (rows or K not a multiple of 4 floats, K not of 32) are copied
into the workspace K-contiguous with K zero-padded to a multiple of 32, and
the product runs as the N/T product of the copies on the 16-byte kernels.

Parity with the fp64 oracle in all four layouts and on several tile configs
of the packed product (forced with MI_PLAN_PACK), every element of a large
packed product through fp64 checksums, bitwise repeatability, integer inputs
exact, and the allocation-free entry point falling back to the unpacked plan
when the packed copies exceed its scratch.

Bar: normalised max error <= 1e-4 against fp64; bitwise equality where stated.
"""
import ctypes

import numpy as np
import pytest
import torch

import freivalds as fv
from gpu_util import assert_close, cur_stream, gemm_args, run_gemm, to_dev, to_host, workspace

pytestmark = pytest.mark.gpu

PACK, NO_PACK = 0x80, 0x40
LAYOUTS = [(0, 0), (1, 0), (0, 1), (1, 1)]


def _operands(orc, M, N, K, op_a, op_b, seed):
    a_st = orc.uniform((K, M) if op_a else (M, K), seed)
    b_st = orc.uniform((N, K) if op_b else (K, N), seed + 1)
    return a_st, b_st, (a_st.T if op_a else a_st), (b_st.T if op_b else b_st)


def _run(ck, A, B, M, N, K, op_a, op_b, override, fill=float("nan")):
    C = torch.full((M, N), fill, device="cuda")
    args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=override)
    ws = workspace(ck, args)
    args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=override, ws=ws)
    ck.abi.check(run_gemm(ck, args), "mi_gemm_f32")
    return C


def _plan(ck, M, N, K, op_a, op_b, override):
    rc, p = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40, plan_override=override)
    assert rc == 0
    return p


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("M,N,K,cfg", [
    (1000, 1100, 1021, 0),    # K odd: every row of A (N) or B (T) misaligned
    (643, 517, 2047, 3),      # all extents odd, the 256 tile on the copies
    (1024, 1022, 1000, 10),   # N not a multiple of 4, K of 32: the k-split 64 tile
    (768, 640, 1040, 2),      # 16-byte rows, K % 32 == 16: K padded to 1056
    (96, 200, 37, 0),         # K below one slice
])
def test_packed_parity(ck, orc, dev, op_a, op_b, M, N, K, cfg):
    p = _plan(ck, M, N, K, op_a, op_b, PACK | cfg)
    assert p.packed == 1 and p.packed_k % 32 == 0 and K <= p.packed_k < K + 32
    if cfg:
        assert p.plan_id == cfg
    a_st, b_st, a, b = _operands(orc, M, N, K, op_a, op_b, seed=5100 + cfg)
    C = _run(ck, to_dev(a_st), to_dev(b_st), M, N, K, op_a, op_b, PACK | cfg)
    assert_close(orc, to_host(C), orc.gemm(a, b), K, what=f"packed {op_a}{op_b} {M}x{N}x{K} cfg{cfg}")


def test_packed_stream_k_on_the_256_tile(ck, orc, dev):
    """Packing, then stream-K on the copies (the bits below MI_PLAN_PACK apply
    to the packed product)."""
    M, N, K = 2001, 1799, 3001
    p = _plan(ck, M, N, K, 1, 0, PACK | 0x13)
    assert p.packed == 1 and p.plan_id == 3 and p.stream_k == 1
    a_st, b_st, a, b = _operands(orc, M, N, K, 1, 0, seed=5200)
    C = to_host(_run(ck, to_dev(a_st), to_dev(b_st), M, N, K, 1, 0, PACK | 0x13))
    rows = sorted({0, 1, 255, 256, M // 2, M - 1})
    assert_close(orc, C[rows], orc.gemm(a, b, rows=rows), K, what="packed stream-K rows")
    v, u = fv.signs(N, 5), fv.signs(M, 6)
    fv.check(orc, *orc.checksums(C, v, u), *fv.reference(orc, a, b, v, u), K, 1.0, 1.0,
             "packed stream-K every element")


@pytest.mark.parametrize("M,N,K,ops", [
    (8205, 5921, 2949, (0, 0)),   # the planner packs (PID 8-style irregular extents)
    (4095, 4095, 4095, (1, 0)),
    (8205, 2949, 5921, (0, 0)),   # packed where the unpacked plan is 4-byte stream-K
    (1471, 1329, 1188, (0, 0)),   # packed below K = 1536 (the k-split 64 tile on the copies)
    (4245, 918, 1081, (1, 0)),
])
def test_auto_packed_large_every_element(ck, orc, dev, M, N, K, ops):
    op_a, op_b = ops
    p = _plan(ck, M, N, K, op_a, op_b, 0)
    a_st, b_st, a, b = _operands(orc, M, N, K, op_a, op_b, seed=5300)
    C = to_host(_run(ck, to_dev(a_st), to_dev(b_st), M, N, K, op_a, op_b, 0))
    rows = sorted({0, 1, 127, 128, 255, 256, M // 2, M - 1})
    assert_close(orc, C[rows], orc.gemm(a, b, rows=rows), K, what=f"auto (packed={p.packed}) rows")
    v, u = fv.signs(N, 7), fv.signs(M, 8)
    fv.check(orc, *orc.checksums(C, v, u), *fv.reference(orc, a, b, v, u), K, 1.0, 1.0,
             f"auto {M}x{N}x{K} every element (packed={p.packed})")


def test_packed_bitwise_repeatable_and_integer_exact(ck, orc, dev):
    M, N, K = 1000, 1100, 1021
    a_st, b_st, _, _ = _operands(orc, M, N, K, 0, 1, seed=5400)
    A, B = to_dev(a_st), to_dev(b_st)
    first = to_host(_run(ck, A, B, M, N, K, 0, 1, PACK))
    for _ in range(9):
        np.testing.assert_array_equal(to_host(_run(ck, A, B, M, N, K, 0, 1, PACK)), first)
    # integer inputs: every partial sum exact, so packed == unpacked == int64 product
    a = orc.integers((M, K), 5401)
    b = orc.integers((K, N), 5402)
    A, B = to_dev(a), to_dev(b)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(to_host(_run(ck, A, B, M, N, K, 0, 0, PACK)), want)
    np.testing.assert_array_equal(to_host(_run(ck, A, B, M, N, K, 0, 0, NO_PACK)), want)


def test_noalloc_falls_back_to_the_unpacked_plan(ck, orc, dev):
    """A packed plan whose copies exceed the no-alloc scratch: the
    allocation-free entry point runs the unpacked plan, bit for bit the same
    as mi_gemm_f32 with MI_PLAN_NO_PACK."""
    L = ck.abi.lib()
    M, N, K = 6001, 3001, 2049      # A' + B' = 9002 x 2080 floats: 75 MB > 64 MiB
    p = _plan(ck, M, N, K, 0, 0, PACK)
    assert p.packed == 1 and p.workspace_bytes > ck.abi.NOALLOC_SCRATCH_BYTES
    a_st, b_st, a, b = _operands(orc, M, N, K, 0, 0, seed=5500)
    A, B = to_dev(a_st), to_dev(b_st)
    want = to_host(_run(ck, A, B, M, N, K, 0, 0, NO_PACK))
    C = torch.full((M, N), float("nan"), device="cuda")
    args = gemm_args(ck, A, B, C, M, N, K, override=PACK)
    ck.abi.check(L.mi_gemm_f32_noalloc(ctypes.byref(args), cur_stream()), "mi_gemm_f32_noalloc")
    np.testing.assert_array_equal(to_host(C), want)
    rows = [0, M // 3, M - 1]
    assert_close(orc, want[rows], orc.gemm(a, b, rows=rows), K, what="noalloc unpacked rows")
