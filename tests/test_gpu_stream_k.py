"""Stream-K schedule on the GPU, through the C ABI: parity with the fp64 oracle
in every layout on the direct-staged 256 and 128 tiles (16-byte and, on the
128 tile, 4-byte staging with a partial last slice) and the k-split 64 tile, tiles split over many workgroups
and ragged edges, a data-parallel wave ahead of the stream-K tiles, bitwise
repeatability (the fixup adds partials in a fixed order), and agreement with
the data-parallel plan of the same problem -- each under both schedules the
planner deals K-slices with (phases, where they apply, and contiguous ranges).

Bar: normalised max error <= 1e-4 against fp64; bitwise equality across runs.
"""
import numpy as np
import pytest
import torch

import freivalds as fv
from gpu_util import assert_close, gemm_args, run_gemm, to_dev, to_host, workspace

pytestmark = pytest.mark.gpu

SK_FORCE, SK_NEVER = 0x10, 0x20
SK_RANGES = 0x40000000  # contiguous K-slice ranges instead of the phased schedule
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
    rc, p = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40,
                        plan_override=override)
    assert rc == 0
    return p


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("M,N,K,cfg", [
    (1280, 1280, 2048, 3),   # 25 tiles of 256 over 256 workgroups: ~10 segments per tile
    (1000, 1000, 4096, 3),   # ragged edges on the 256 tile
    (640, 640, 2048, 2),     # 25 tiles of 128 over 768 workgroups
    (1000, 1100, 1024, 2),   # ragged edges on the 128 tile
    (640, 640, 2048, 10),    # 100 tiles of 64 over 256 workgroups (the k-split 64 tile)
    (1000, 1100, 1024, 10),  # ragged edges: 288 tiles, one data-parallel wave + 32 stream-K
    (1000, 1100, 1021, 2),   # 4-byte staging (K % 16 != 0): each tile's last slice partial
    (640, 643, 2047, 2),     # 4-byte staging, N and K odd
])
@pytest.mark.parametrize("ranges", [False, True])
def test_stream_k_parity(ck, orc, dev, op_a, op_b, M, N, K, cfg, ranges):
    ov = cfg | SK_FORCE | (SK_RANGES if ranges else 0)
    p = _plan(ck, M, N, K, op_a, op_b, ov)
    assert p.stream_k == 1 and p.plan_id == cfg
    if ranges:
        assert p.sk_phases == 0
    a_st, b_st, a, b = _operands(orc, M, N, K, op_a, op_b, seed=4100 + cfg)
    A, B = to_dev(a_st), to_dev(b_st)
    C = _run(ck, A, B, M, N, K, op_a, op_b, ov)
    assert_close(orc, to_host(C), orc.gemm(a, b), K,
                 what=f"stream-K {op_a}{op_b} {M}x{N}x{K} cfg{cfg} phases {p.sk_phases}")


@pytest.mark.parametrize("M,N,K,cfg,ops", [
    (5760, 5120, 256, 2, (0, 0)),    # 1800 tiles: one data-parallel wave (768) + 1032 stream-K
    (5120, 5120, 2048, 3, (1, 1)),   # 400 tiles of 256: 1.56 tiles per workgroup
    (3584, 3584, 1024, 3, (0, 1)),   # 196 tiles < 256 workgroups
    (1536, 1536, 2048, 10, (1, 0)),  # 576 tiles of 64: 256 data-parallel + 320 stream-K
    (8205, 2949, 5921, 2, (0, 0)),   # 4-byte staging: two data-parallel waves + 24 stream-K tiles
    (3001, 3001, 3001, 2, (1, 1)),   # 4-byte staging: 576 tiles, every one stream-K
])
@pytest.mark.parametrize("ranges", [False, True])
def test_stream_k_larger_every_element(ck, orc, dev, M, N, K, cfg, ops, ranges):
    """Bigger stream-K schedules, every element through fp64 row and column
    checksums, plus exact fp64 rows."""
    op_a, op_b = ops
    ov = cfg | SK_FORCE | (SK_RANGES if ranges else 0)
    p = _plan(ck, M, N, K, op_a, op_b, ov)
    assert p.stream_k == 1 and p.plan_id == cfg
    a_st, b_st, a, b = _operands(orc, M, N, K, op_a, op_b, seed=4200 + cfg)
    A, B = to_dev(a_st), to_dev(b_st)
    Cd = _run(ck, A, B, M, N, K, op_a, op_b, ov)
    C = to_host(Cd)
    rows = sorted({0, 1, 255, 256, 257, M // 2, M - 1})
    assert_close(orc, C[rows], orc.gemm(a, b, rows=rows), K, what="stream-K rows")
    v, u = fv.signs(N, 9), fv.signs(M, 10)
    fv.check(orc, *orc.checksums(C, v, u), *fv.reference(orc, a, b, v, u), K, 1.0, 1.0,
             f"stream-K {M}x{N}x{K} every element")


@pytest.mark.parametrize("M,N,K,cfg", [(1280, 1280, 2048, 3), (640, 640, 2048, 2), (640, 640, 2048, 10),
                                       (1000, 1100, 1021, 2)])
@pytest.mark.parametrize("ranges", [False, True])
def test_stream_k_bitwise_repeatable(ck, orc, dev, M, N, K, cfg, ranges):
    """20 runs, bitwise identical: every partial tile is added in slot order."""
    ov = cfg | SK_FORCE | (SK_RANGES if ranges else 0)
    a_st, b_st, _, _ = _operands(orc, M, N, K, 0, 0, seed=4300)
    A, B = to_dev(a_st), to_dev(b_st)
    first = to_host(_run(ck, A, B, M, N, K, 0, 0, ov))
    for _ in range(19):
        np.testing.assert_array_equal(to_host(_run(ck, A, B, M, N, K, 0, 0, ov)), first)


@pytest.mark.parametrize("M,N,K,cfg", [(1280, 1280, 2048, 3), (640, 640, 2048, 2), (640, 640, 2048, 10),
                                       (1000, 1100, 1021, 2)])
def test_stream_k_integer_inputs_exact(ck, orc, dev, M, N, K, cfg):
    """Integer-valued inputs: every partial sum is an exact integer, so the
    stream-K result equals the data-parallel one bit for bit."""
    a = orc.integers((M, K), 4400)
    b = orc.integers((K, N), 4401)
    A, B = to_dev(a), to_dev(b)
    sk = to_host(_run(ck, A, B, M, N, K, 0, 0, cfg | SK_FORCE))
    skr = to_host(_run(ck, A, B, M, N, K, 0, 0, cfg | SK_FORCE | SK_RANGES))
    dp = to_host(_run(ck, A, B, M, N, K, 0, 0, cfg | SK_NEVER))
    np.testing.assert_array_equal(sk, dp)
    np.testing.assert_array_equal(skr, dp)
    np.testing.assert_array_equal(sk, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


def test_stream_k_matches_data_parallel_within_tolerance(ck, orc, dev):
    M, N, K = 1280, 1280, 2048
    a_st, b_st, a, b = _operands(orc, M, N, K, 0, 0, seed=4500)
    A, B = to_dev(a_st), to_dev(b_st)
    sk = to_host(_run(ck, A, B, M, N, K, 0, 0, 3 | SK_FORCE))
    dp = to_host(_run(ck, A, B, M, N, K, 0, 0, 3 | SK_NEVER))
    assert orc.norm_err(sk, dp.astype(np.float64), K, 1.0, 1.0) <= 2 * orc.TOL


def _random_sk_shapes(n, seed):
    """Seeded shapes over the stream-K region of each tile config (16-byte
    rows, K a multiple of 64), the same generator as the CPU schedule test."""
    import random
    rnd = random.Random(seed)
    out = []
    for _ in range(n):
        cfg = rnd.choice([3, 3, 2, 9, 10])
        out.append((16 * rnd.randint(8, 480), 16 * rnd.randint(8, 480), 64 * rnd.randint(16, 96), cfg))
    return out


@pytest.mark.parametrize("M,N,K,cfg", _random_sk_shapes(12, 2027))
def test_stream_k_random_shapes_every_element(ck, orc, dev, M, N, K, cfg):
    """Seeded random shapes with stream-K forced on their config, under the
    planner's schedule (phases where they apply): every element through fp64
    row and column checksums, plus exact rows."""
    p = _plan(ck, M, N, K, 0, 0, cfg | SK_FORCE)
    if p.stream_k != 1:
        pytest.skip("the config takes no stream-K plan for this shape")
    a = orc.uniform((M, K), 4600 + cfg)
    b = orc.uniform((K, N), 4601 + cfg)
    C = to_host(_run(ck, to_dev(a), to_dev(b), M, N, K, 0, 0, cfg | SK_FORCE))
    rows = sorted({0, M // 3, M - 1})
    assert_close(orc, C[rows], orc.gemm(a, b, rows=rows), K,
                 what=f"stream-K {M}x{N}x{K} cfg{cfg} phases {p.sk_phases} rows")
    v, u = fv.signs(N, 11), fv.signs(M, 12)
    fv.check(orc, *orc.checksums(C, v, u), *fv.reference(orc, a, b, v, u), K, 1.0, 1.0,
             f"stream-K {M}x{N}x{K} cfg{cfg} phases {p.sk_phases} every element")
