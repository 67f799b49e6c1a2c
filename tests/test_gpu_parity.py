"""GPU parity of the HIP kernels, called through the C ABI (libmi355gemm.so),
against the fp64 CPU oracle on the same seeded inputs.

Bar: normalised max error <= 1e-4 (max|C - C64| / (sqrt(K) max|A| max|B|))
for real-valued inputs; bitwise equality for integer-valued inputs (every
partial sum is an integer below 2^24, so any summation order is exact), for
diag(a).B (one fp32 multiply) and for the structural zeros of the triangular
products; bitwise equality across repeated runs (determinism).
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import (assert_close, cur_stream, dev_uniform, gemm_args, run_gemm, to_dev, to_host,
                      vp, workspace)

pytestmark = pytest.mark.gpu

LAYOUTS = [(0, 0), (1, 0), (0, 1), (1, 1)]  # (op_a, op_b): NN, TN, NT, TT
SHAPES = [  # (M, N, K) -- tile multiples, ragged edges, degenerate extents
    (1024, 1024, 1024), (256, 256, 16), (128, 64, 48), (1023, 517, 2049), (1, 1, 1),
    (65, 129, 31), (7, 63, 65), (300, 4, 257), (4, 300, 8), (333, 333, 1),
]


def _host_operands(orc, M, N, K, op_a, op_b, seed):
    """Stored (not logical) operands, as the kernels see them."""
    a_st = orc.uniform((K, M) if op_a else (M, K), seed)
    b_st = orc.uniform((N, K) if op_b else (K, N), seed + 1)
    return a_st, b_st


def _logical(x_st, op):
    return x_st.T if op else x_st


@pytest.mark.parametrize("n", [1, 3, 1000, 65537])
@pytest.mark.parametrize("seed", [0, 17, 2 ** 20 + 5])
def test_device_generator_matches_host(ck, orc, dev, n, seed):
    got = to_host(dev_uniform(ck, (n,), seed))
    np.testing.assert_array_equal(got, orc.uniform((n,), seed))
    off = to_host(dev_uniform(ck, (n,), seed, offset=12345))
    np.testing.assert_array_equal(off, orc.uniform((n,), seed, offset=12345))


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_layouts_auto_plan(ck, orc, dev, op_a, op_b, M, N, K):
    a_st, b_st = _host_operands(orc, M, N, K, op_a, op_b, seed=7)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.full((M, N), float("nan"), device="cuda")
    args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b)
    ws = workspace(ck, args)
    args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, ws=ws)
    ck.abi.check(run_gemm(ck, args), "mi_gemm_f32")
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    assert_close(orc, to_host(C), ref, K, np.abs(a_st).max(), np.abs(b_st).max(),
                 f"layout {op_a}{op_b} {M}x{N}x{K}")


def _random_shapes(n, seed):
    """Seeded small-to-mid problems whose plans the planner picks freely:
    16-byte rows, K a multiple of 64 (so the k-split tile, split-K and
    stream-K all compete), random layouts."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M, N = (int(4 * rng.integers(16, 250)) for _ in range(2))
        K = int(64 * rng.integers(1, 48))
        out.append((M, N, K, int(rng.integers(0, 2)), int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("M,N,K,op_a,op_b", _random_shapes(12, 2026))
def test_random_shapes_auto_plan(ck, orc, dev, M, N, K, op_a, op_b):
    """Whatever the planner picks for these (data-parallel, split-K or
    stream-K, on any tile), the result matches the oracle."""
    rc, p = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40)
    assert rc == 0
    a_st, b_st = _host_operands(orc, M, N, K, op_a, op_b, seed=M + N + K)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.full((M, N), float("nan"), device="cuda")
    ws = workspace(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b))
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, ws=ws)))
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    assert_close(orc, to_host(C), ref, K, np.abs(a_st).max(), np.abs(b_st).max(),
                 f"auto plan {p.plan_id}/{p.split_k}/{p.stream_k} {op_a}{op_b} {M}x{N}x{K}")


_SWEEP_OVERRIDES = [0, 0, 0x40, 0x80, 0x12, 0x19, 0x13, 0x2, 0x3, 0x9, 0xb, 0xa, 0x1, 0x22, 0x29,
                    0x203, 0x402]


def _sweep_cases(n, seed):
    """Seeded problems over the ABI's combinations: aligned or not, every
    layout, padded leading dimensions, batches, the row bias (N/N), and
    forced plans (tiles, split-K, stream-K, packing on or off; a plan the
    problem cannot take is ignored by the planner)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        align = rng.random() < 0.5
        ext = lambda lo, hi: max(1, (int(rng.integers(lo, hi)) // 4) * 4 if align else int(rng.integers(lo, hi)))
        M, N, K = ext(1, 700), ext(1, 700), ext(1, 1500)
        op_a, op_b = int(rng.integers(0, 2)), int(rng.integers(0, 2))
        batch = int(rng.choice([1, 1, 2, 3]))
        pad = int(rng.choice([0, 0, 3, 4]))
        bias = bool(op_a == 0 and op_b == 0 and rng.random() < 0.3)
        ov = int(rng.choice(_SWEEP_OVERRIDES))
        out.append((M, N, K, op_a, op_b, batch, pad, bias, ov))
    return out


@pytest.mark.parametrize("M,N,K,op_a,op_b,batch,pad,bias,ov", _sweep_cases(40, 2041))
def test_random_abi_combinations(ck, orc, dev, M, N, K, op_a, op_b, batch, pad, bias, ov):
    lda, ldb, ldc = (M if op_a else K) + pad, (K if op_b else N) + pad, N + pad
    a_st = orc.uniform((batch,) + ((K, M) if op_a else (M, K)), 191)
    b_st = orc.uniform((batch,) + ((N, K) if op_b else (K, N)), 192)
    bi = orc.uniform((M,), 193)
    a_pad = np.zeros((batch, a_st.shape[1], lda), np.float32)
    a_pad[:, :, :a_st.shape[2]] = a_st
    b_pad = np.zeros((batch, b_st.shape[1], ldb), np.float32)
    b_pad[:, :, :b_st.shape[2]] = b_st
    A, B, Bi = to_dev(a_pad), to_dev(b_pad), to_dev(bi)
    C = torch.full((batch, M, ldc), float("nan"), device="cuda")
    args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch, lda=lda, ldb=ldb, ldc=ldc,
                     sa=a_pad[0].size, sb=b_pad[0].size, sc=M * ldc, override=ov)
    if bias:
        args.bias_m = Bi.data_ptr()
    ws = workspace(ck, args)
    args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch, lda=lda, ldb=ldb, ldc=ldc,
                     sa=a_pad[0].size, sb=b_pad[0].size, sc=M * ldc, override=ov, ws=ws)
    if bias:
        args.bias_m = Bi.data_ptr()
    ck.abi.check(run_gemm(ck, args))
    la = np.swapaxes(a_st, 1, 2) if op_a else a_st
    lb = np.swapaxes(b_st, 1, 2) if op_b else b_st
    ref = orc.gemm(la, lb) + (bi.astype(np.float64)[None, :, None] if bias else 0.0)
    got = to_host(C)
    assert_close(orc, got[:, :, :N], ref, K,
                 what=f"{M}x{N}x{K}x{batch} {op_a}{op_b} pad={pad} bias={bias} override={ov:#x}")
    if pad:
        assert np.isnan(got[:, :, N:]).all(), "a store landed in the ldc padding"

def _random_unaligned_shapes(n, seed):
    """Seeded problems with at least one extent not a multiple of 4 floats
    (rows the 16-byte loaders cannot stage): the planner then chooses
    between the 4-byte direct staging, the register-staged tiles, split-K
    and packing the operands into 16-byte rows (offered from K = 256)."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M, N = (int(rng.integers(200, 1400)) for _ in range(2))
        K = int(rng.integers(256, 2000))
        if M % 4 == 0 and N % 4 == 0 and K % 4 == 0:
            continue
        out.append((M, N, K, int(rng.integers(0, 2)), int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("M,N,K,op_a,op_b", _random_unaligned_shapes(12, 2040))
def test_random_unaligned_shapes_auto_plan(ck, orc, dev, M, N, K, op_a, op_b):
    """Whatever the planner picks for unaligned operands (packed or not, any
    tile, split-K), the result matches the oracle."""
    rc, p = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40)
    assert rc == 0
    a_st, b_st = _host_operands(orc, M, N, K, op_a, op_b, seed=M + 2 * N + 3 * K)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.full((M, N), float("nan"), device="cuda")
    ws = workspace(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b))
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, ws=ws)))
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    assert_close(orc, to_host(C), ref, K, np.abs(a_st).max(), np.abs(b_st).max(),
                 f"auto plan {p.plan_id}/{p.split_k}/{p.stream_k} packed={p.packed} "
                 f"{op_a}{op_b} {M}x{N}x{K}")


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5, 6, 7])
@pytest.mark.parametrize("M,N,K", [(512, 512, 512), (300, 200, 100), (64, 640, 37), (700, 520, 31),
                                   (130, 1030, 64), (1000, 999, 17), (513, 1027, 1)])
def test_gemm_every_tile_config(ck, orc, dev, op_a, op_b, cfg, M, N, K):
    a_st, b_st = _host_operands(orc, M, N, K, op_a, op_b, seed=11)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.full((M, N), float("nan"), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=cfg)))
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    assert_close(orc, to_host(C), ref, K, np.abs(a_st).max(), np.abs(b_st).max(),
                 f"cfg {cfg} layout {op_a}{op_b} {M}x{N}x{K}")


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5, 6, 7])
def test_integer_inputs_bitwise(ck, orc, dev, op_a, op_b, cfg):
    M, N, K = 200, 136, {4: 32, 5: 64, 6: 32, 7: 64}.get(cfg, 1000)
    a_st = orc.integers((K, M) if op_a else (M, K), seed=21)
    b_st = orc.integers((N, K) if op_b else (K, N), seed=22)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.empty((M, N), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=cfg)))
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    assert np.all(ref == np.round(ref))
    np.testing.assert_array_equal(to_host(C), ref.astype(np.float32))


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("M,N,K,extra", [(512, 512, 512, 0), (300, 200, 96, 0), (700, 520, 32, 0),
                                         (132, 1028, 64, 0), (1000, 996, 1024, 0),
                                         (260, 128, 2048, 2 << 8), (1280, 1280, 2048, 0x10)])
def test_b32_tile_config(ck, orc, dev, op_a, op_b, M, N, K, extra):
    """The 32-deep direct-staged 128 tile (config 9): plain, split-K and
    stream-K schedules, ragged edges, every layout."""
    ov = 9 | extra
    rc, p = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40, plan_override=ov)
    assert rc == 0 and p.plan_id == 9 and p.block_k == 32
    assert p.stream_k == (1 if extra & 0x10 else 0) and p.split_k == (extra >> 8 or 1)
    a_st, b_st = _host_operands(orc, M, N, K, op_a, op_b, seed=13)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.full((M, N), float("nan"), device="cuda")
    ws = workspace(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=ov))
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=ov, ws=ws)))
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    assert_close(orc, to_host(C), ref, K, np.abs(a_st).max(), np.abs(b_st).max(),
                 f"cfg 9 layout {op_a}{op_b} {M}x{N}x{K} override {ov:#x}")


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
def test_b32_integer_inputs_bitwise(ck, orc, dev, op_a, op_b):
    M, N, K = 200, 136, 992
    a_st = orc.integers((K, M) if op_a else (M, K), seed=23)
    b_st = orc.integers((N, K) if op_b else (K, N), seed=24)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.empty((M, N), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=9)))
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    np.testing.assert_array_equal(to_host(C), ref.astype(np.float32))


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("M,N,K,batch,pad,split", [(1024, 1024, 1024, 1, 0, 1), (300, 520, 1088, 1, 0, 1),
                                                   (260, 252, 2048, 1, 4, 1), (516, 260, 1024, 3, 0, 1),
                                                   (264, 300, 512, 2, 4, 1), (64, 64, 64, 1, 0, 1),
                                                   (20, 36, 192, 1, 0, 1), (132, 68, 128, 1, 4, 1),
                                                   (256, 192, 4096, 1, 0, 4), (200, 136, 640, 2, 0, 2)])
def test_ksplit_tile_config(ck, orc, dev, op_a, op_b, M, N, K, batch, pad, split):
    """The 64 x 64 tile whose eight waves split each 64-deep slice (config 10):
    every layout, edge rows and columns (loaded from the last valid row /
    column, never stored), padded leading dimensions, batched, split-K, row
    bias (N/N only); a 1-, 2- or 3-slice K range runs the ring's first steps
    only."""
    a_st = orc.uniform((batch,) + ((K, M) if op_a else (M, K)), 141)
    b_st = orc.uniform((batch,) + ((N, K) if op_b else (K, N)), 142)
    bias = orc.uniform((M,), 143)
    lda, ldb, ldc = (M if op_a else K) + pad, (K if op_b else N) + pad, N + pad
    a_pad = np.zeros((batch, a_st.shape[1], lda), np.float32)
    a_pad[:, :, :a_st.shape[2]] = a_st
    b_pad = np.zeros((batch, b_st.shape[1], ldb), np.float32)
    b_pad[:, :, :b_st.shape[2]] = b_st
    A, B, Bi = to_dev(a_pad), to_dev(b_pad), to_dev(bias)
    la = np.swapaxes(a_st, 1, 2) if op_a else a_st
    lb = np.swapaxes(b_st, 1, 2) if op_b else b_st
    ov = 10 | (split << 8)
    rc, p = ck.abi.plan(M, N, K, batch=batch, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40,
                        plan_override=ov)
    assert rc == 0 and p.plan_id == 10 and p.block_k == 64 and p.split_k == split
    for with_bias in ((False, True) if (op_a, op_b) == (0, 0) else (False,)):
        C = torch.full((batch, M, ldc), float("nan"), device="cuda")
        args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch, lda=lda, ldb=ldb, ldc=ldc,
                         sa=a_pad[0].size, sb=b_pad[0].size, sc=M * ldc, override=ov)
        ws = workspace(ck, args)
        args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch, lda=lda, ldb=ldb, ldc=ldc,
                         sa=a_pad[0].size, sb=b_pad[0].size, sc=M * ldc, override=ov, ws=ws)
        if with_bias:
            args.bias_m = Bi.data_ptr()
        ck.abi.check(run_gemm(ck, args))
        ref = orc.gemm(la, lb) + (bias.astype(np.float64)[None, :, None] if with_bias else 0.0)
        got = to_host(C)
        assert_close(orc, got[:, :, :N], ref, K,
                     what=f"cfg 10 {op_a}{op_b} {M}x{N}x{K}x{batch} pad={pad} split={split} bias={with_bias}")
        if pad:
            assert np.isnan(got[:, :, N:]).all(), "a store landed in the ldc padding"


@pytest.mark.parametrize("op_b", [0, 1])
@pytest.mark.parametrize("M,N,K,batch,pad,split", [(2048, 2048, 2048, 1, 0, 1), (300, 520, 1088, 1, 0, 1),
                                                   (260, 252, 2048, 1, 4, 1), (516, 260, 1024, 3, 0, 1),
                                                   (128, 128, 32, 1, 0, 1), (1000, 900, 4096, 1, 4, 2)])
def test_eight_wave_128_tile_config(ck, orc, dev, op_b, M, N, K, batch, pad, split):
    """The 32-deep 128 tile on 8 waves of 32 x 64 (config 11; A K-contiguous
    only): edge rows and columns, padded leading dimensions, batched,
    split-K, row bias (N/N)."""
    op_a = 0
    a_st = orc.uniform((batch, M, K), 151)
    b_st = orc.uniform((batch,) + ((N, K) if op_b else (K, N)), 152)
    bias = orc.uniform((M,), 153)
    lda, ldb, ldc = K + pad, (K if op_b else N) + pad, N + pad
    a_pad = np.zeros((batch, M, lda), np.float32)
    a_pad[:, :, :K] = a_st
    b_pad = np.zeros((batch, b_st.shape[1], ldb), np.float32)
    b_pad[:, :, :b_st.shape[2]] = b_st
    A, B, Bi = to_dev(a_pad), to_dev(b_pad), to_dev(bias)
    lb = np.swapaxes(b_st, 1, 2) if op_b else b_st
    ov = 11 | (split << 8)
    rc, p = ck.abi.plan(M, N, K, batch=batch, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40,
                        plan_override=ov)
    assert rc == 0 and p.plan_id == 11 and p.block_k == 32 and p.split_k == split
    for with_bias in ((False, True) if op_b == 0 else (False,)):
        C = torch.full((batch, M, ldc), float("nan"), device="cuda")
        args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch, lda=lda, ldb=ldb, ldc=ldc,
                         sa=a_pad[0].size, sb=b_pad[0].size, sc=M * ldc, override=ov)
        ws = workspace(ck, args)
        args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch, lda=lda, ldb=ldb, ldc=ldc,
                         sa=a_pad[0].size, sb=b_pad[0].size, sc=M * ldc, override=ov, ws=ws)
        if with_bias:
            args.bias_m = Bi.data_ptr()
        ck.abi.check(run_gemm(ck, args))
        ref = orc.gemm(a_st, lb) + (bias.astype(np.float64)[None, :, None] if with_bias else 0.0)
        got = to_host(C)
        assert_close(orc, got[:, :, :N], ref, K,
                     what=f"cfg 11 0{op_b} {M}x{N}x{K}x{batch} pad={pad} split={split} bias={with_bias}")
        if pad:
            assert np.isnan(got[:, :, N:]).all(), "a store landed in the ldc padding"


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
def test_ksplit_integer_inputs_bitwise_and_repeatable(ck, orc, dev, op_a, op_b):
    """Config 10 on small-integer operands is exact, and its fixed-order
    reduction of the eight waves' partial tiles repeats bit for bit on
    uniform inputs."""
    M, N, K = 200, 136, 1024
    a_st = orc.integers((K, M) if op_a else (M, K), seed=25)
    b_st = orc.integers((N, K) if op_b else (K, N), seed=26)
    C = torch.empty((M, N), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, to_dev(a_st), to_dev(b_st), C, M, N, K, op_a, op_b,
                                        override=10)))
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    np.testing.assert_array_equal(to_host(C), ref.astype(np.float32))
    a_st, b_st = _host_operands(orc, M, N, K, op_a, op_b, seed=27)
    A, B = to_dev(a_st), to_dev(b_st)
    outs = []
    for _ in range(3):
        C = torch.full((M, N), float("nan"), device="cuda")
        ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=10)))
        outs.append(to_host(C))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_closed_forms_identity_ones_rank1(ck, orc, dev):
    n = 384
    I = np.eye(n, dtype=np.float32)
    X = orc.uniform((n, n), seed=31)
    for a, b, want in [(I, X, X), (X, I, X),
                       (np.ones((n, 700), np.float32), np.ones((700, n), np.float32),
                        np.full((n, n), 700, np.float32))]:
        C = torch.empty((a.shape[0], b.shape[1]), device="cuda")
        ck.abi.check(run_gemm(ck, gemm_args(ck, to_dev(a), to_dev(b), C, a.shape[0], b.shape[1],
                                            a.shape[1])))
        np.testing.assert_array_equal(to_host(C), want)
    u = orc.integers((n, 1), seed=32, lo=-3, hi=3)
    v = orc.integers((1, n), seed=33, lo=-3, hi=3)
    C = torch.empty((n, n), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, to_dev(u), to_dev(v), C, n, n, 1)))
    np.testing.assert_array_equal(to_host(C), u * v)


@pytest.mark.parametrize("split", [2, 3, 8, 64])
@pytest.mark.parametrize("cfg", [1, 2, 3])
def test_split_k_partition_and_determinism(ck, orc, dev, split, cfg):
    M, N, K = 160, 96, 20000
    a_st, b_st = orc.uniform((M, K), 41), orc.uniform((K, N), 42)
    A, B = to_dev(a_st), to_dev(b_st)
    ov = cfg | (split << 8)
    C = torch.empty((M, N), device="cuda")
    probe = gemm_args(ck, A, B, C, M, N, K, override=ov)
    ws = workspace(ck, probe)
    outs = []
    for _ in range(3):
        C = torch.full((M, N), float("nan"), device="cuda")
        ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, override=ov, ws=ws)))
        outs.append(to_host(C))
    assert_close(orc, outs[0], orc.gemm(a_st, b_st), K, what=f"split {split} cfg {cfg}")
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


@pytest.mark.parametrize("cfg", [3, 2])
@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("M,N,K,batch,pad", [(300, 520, 1056, 1, 0), (260, 252, 2048, 1, 4),
                                             (257, 255, 2048, 1, 0), (516, 260, 1024, 3, 0),
                                             (256, 256, 4096, 1, 8), (264, 300, 512, 2, 4),
                                             (300, 264, 256, 1, 0), (130, 132, 272, 1, 0),
                                             (200, 196, 80, 2, 4)])
def test_direct_staging(ck, orc, dev, cfg, op_a, op_b, M, N, K, batch, pad):
    """The 256- and 128-tile paths with direct global->LDS loads (K a multiple
    of the slice depth, 32 / 16; for the 256 tile K >= 256 per split, and >=
    512 in the layouts other than N/N; 16-byte operands -- other shapes take the
    register-staged kernel, as do contiguous extents that are not multiples
    of 4): edge rows and columns are loaded from the last valid row / column
    and must not leak into stored outputs; padded leading dimensions; batched;
    row bias (N/N only)."""
    a_st = orc.uniform((batch,) + ((K, M) if op_a else (M, K)), 131)
    b_st = orc.uniform((batch,) + ((N, K) if op_b else (K, N)), 132)
    bias = orc.uniform((M,), 133)
    lda = (M if op_a else K) + pad
    ldb = (K if op_b else N) + pad
    ldc = N + pad
    # padded storage: the logical operands sit in the leading columns
    a_pad = np.zeros((batch, a_st.shape[1], lda), np.float32)
    a_pad[:, :, :a_st.shape[2]] = a_st
    b_pad = np.zeros((batch, b_st.shape[1], ldb), np.float32)
    b_pad[:, :, :b_st.shape[2]] = b_st
    A, B, Bi = to_dev(a_pad), to_dev(b_pad), to_dev(bias)
    la = np.swapaxes(a_st, 1, 2) if op_a else a_st
    lb = np.swapaxes(b_st, 1, 2) if op_b else b_st
    for with_bias in ((False, True) if (op_a, op_b) == (0, 0) else (False,)):
        C = torch.full((batch, M, ldc), float("nan"), device="cuda")
        args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch, lda=lda, ldb=ldb, ldc=ldc,
                         sa=a_pad[0].size, sb=b_pad[0].size, sc=M * ldc, override=cfg)
        if with_bias:
            args.bias_m = Bi.data_ptr()
        ck.abi.check(run_gemm(ck, args))
        ref = orc.gemm(la, lb) + (bias.astype(np.float64)[None, :, None] if with_bias else 0.0)
        got = to_host(C)
        assert_close(orc, got[:, :, :N], ref, K,
                     what=f"direct cfg {cfg} {op_a}{op_b} {M}x{N}x{K}x{batch} pad={pad} bias={with_bias}")
        if pad:
            assert np.isnan(got[:, :, N:]).all(), "a store landed in the ldc padding"


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("M,N,K,batch,pad,split", [(301, 299, 517, 1, 0, 1), (130, 129, 37, 2, 1, 1),
                                                   (257, 263, 1000, 1, 0, 1), (260, 264, 48, 1, 3, 1),
                                                   (129, 250, 2001, 1, 0, 2), (5, 7, 19, 1, 0, 1)])
def test_direct_staging_unaligned(ck, orc, dev, op_a, op_b, M, N, K, batch, pad, split):
    """The 128-tile path with 4-byte direct loads: operands that are not
    16-byte aligned or K not a multiple of 16.  The last slice of each K
    range is partial: its loads are clamped into the operand and its
    fragments past the range zeroed; with split-K only the last chunk has
    one.  Edge rows / columns, padded leading dimensions, batched, row bias."""
    a_st = orc.uniform((batch,) + ((K, M) if op_a else (M, K)), 171)
    b_st = orc.uniform((batch,) + ((N, K) if op_b else (K, N)), 172)
    bias = orc.uniform((M,), 173)
    lda = (M if op_a else K) + pad
    ldb = (K if op_b else N) + pad
    ldc = N + pad
    a_pad = np.zeros((batch, a_st.shape[1], lda), np.float32)
    a_pad[:, :, :a_st.shape[2]] = a_st
    b_pad = np.zeros((batch, b_st.shape[1], ldb), np.float32)
    b_pad[:, :, :b_st.shape[2]] = b_st
    # a NaN in the padding would poison any product that read past the K range
    if pad:
        a_pad[:, :, a_st.shape[2]:] = np.nan
        b_pad[:, :, b_st.shape[2]:] = np.nan
    A, B, Bi = to_dev(a_pad), to_dev(b_pad), to_dev(bias)
    la = np.swapaxes(a_st, 1, 2) if op_a else a_st
    lb = np.swapaxes(b_st, 1, 2) if op_b else b_st
    ov = 2 | (split << 8)
    for with_bias in ((False, True) if (op_a, op_b) == (0, 0) and split == 1 else (False,)):
        C = torch.full((batch, M, ldc), float("nan"), device="cuda")
        kw = dict(batch=batch, lda=lda, ldb=ldb, ldc=ldc, sa=a_pad[0].size, sb=b_pad[0].size,
                  sc=M * ldc, override=ov)
        args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, **kw)
        if split > 1:
            args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, ws=workspace(ck, args), **kw)
        if with_bias:
            args.bias_m = Bi.data_ptr()
        ck.abi.check(run_gemm(ck, args))
        ref = orc.gemm(la, lb) + (bias.astype(np.float64)[None, :, None] if with_bias else 0.0)
        got = to_host(C)
        assert_close(orc, got[:, :, :N], ref, K,
                     what=f"direct4 {op_a}{op_b} {M}x{N}x{K}x{batch} pad={pad} split={split} bias={with_bias}")
        if pad:
            assert np.isnan(got[:, :, N:]).all(), "a store landed in the ldc padding"


@pytest.mark.parametrize("cfg", [3, 2])
@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
def test_direct_staging_split_k(ck, orc, dev, cfg, op_a, op_b):
    """Split-K over the direct path: two 1024-deep chunks per tile, partials
    reduced in fixed order."""
    M, N, K = 260, 264, 2048
    a_st, b_st = _host_operands(orc, M, N, K, op_a, op_b, 141)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.full((M, N), float("nan"), device="cuda")
    args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=cfg | (2 << 8))
    ws = workspace(ck, args)
    args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=cfg | (2 << 8), ws=ws)
    ck.abi.check(run_gemm(ck, args))
    assert_close(orc, to_host(C), orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b)), K,
                 what=f"direct split cfg {cfg} {op_a}{op_b}")


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("K,cfg", [(32, 6), (64, 7), (30, 6), (24, 6), (5, 6), (40, 7), (64, 8), (40, 8),
                                   (16, 8), (64, 12), (40, 12), (33, 12)])
def test_panel_fast_path(ck, orc, dev, op_a, op_b, K, cfg):
    """The panel kernel's fast path (interior tiles, runs of >= 2 streamed
    tiles: 4096 x 4096 gives 16 (32) row panels x 16 (8) runs of 2 (4); the
    B-resident panel 16 column panels x 16 runs of 2 row tiles): stores of
    one tile overlap the next tile's MFMAs; the 32-deep and the 128-row
    panels stage each 32 x 32 block through LDS to store whole rows.  With
    and without the row bias (N/N; the B-resident panel takes none)."""
    M = N = 4096
    rc, p = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, plan_override=cfg)
    assert rc == 0 and p.plan_id == cfg
    a_st, b_st = _host_operands(orc, M, N, K, op_a, op_b, 151)
    bias = orc.uniform((M,), 153)
    A, B, Bi = to_dev(a_st), to_dev(b_st), to_dev(bias)
    ref = orc.gemm(_logical(a_st, op_a), _logical(b_st, op_b))
    for with_bias in ((False, True) if (op_a, op_b) == (0, 0) and cfg != 12 else (False,)):
        C = torch.full((M, N), float("nan"), device="cuda")
        args = gemm_args(ck, A, B, C, M, N, K, op_a, op_b, override=cfg)
        if with_bias:
            args.bias_m = Bi.data_ptr()
        ck.abi.check(run_gemm(ck, args))
        want = ref + (bias.astype(np.float64)[:, None] if with_bias else 0.0)
        assert_close(orc, to_host(C), want, K, what=f"panel {op_a}{op_b} K={K} bias={with_bias}")


@pytest.mark.parametrize("M,batch", [(128, 2), (384, 1)])
def test_panel_128_rows_auto(ck, orc, dev, M, batch):
    """M an odd multiple of 128 with a large output and K <= 64 (the 1x1
    convolution's shape) is planned on 128-row panels; the weight is
    broadcast over the batch (stride_a = 0) and the row bias added."""
    N, K = 65536, 64
    rc, p = ck.abi.plan(M, N, K, batch=batch)
    assert p.plan_id == 8
    w = orc.uniform((M, K), 161)
    x = orc.uniform((batch, K, N), 162)
    bias = orc.uniform((M,), 163)
    W, X, Bi = to_dev(w), to_dev(x), to_dev(bias)
    C = torch.full((batch, M, N), float("nan"), device="cuda")
    args = gemm_args(ck, W, X, C, M, N, K, batch=batch, sa=0, sb=K * N, sc=M * N)
    args.bias_m = Bi.data_ptr()
    ck.abi.check(run_gemm(ck, args))
    got = to_host(C)
    cols = np.r_[0:300, N - 300:N]  # sampled columns keep the fp64 oracle cheap
    for b in range(batch):
        ref = orc.gemm(w, np.ascontiguousarray(x[b][:, cols])) + bias.astype(np.float64)[:, None]
        assert_close(orc, got[b][:, cols], ref, K, what=f"panel128 b={b}")
    assert not np.isnan(got).any()


def test_split_k_without_workspace_is_rejected(ck, dev):
    M, N, K = 64, 64, 8192
    A = torch.zeros((M, K), device="cuda")
    B = torch.zeros((K, N), device="cuda")
    C = torch.zeros((M, N), device="cuda")
    rc = run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, override=2 | (4 << 8)))
    assert rc == ck.abi.MI_ERR_WORKSPACE


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
def test_strided_batched_and_broadcast(ck, orc, dev, op_a, op_b):
    batch, M, N, K = 5, 96, 80, 72
    a_st = orc.uniform((batch,) + ((K, M) if op_a else (M, K)), 51)
    b_st = orc.uniform((batch,) + ((N, K) if op_b else (K, N)), 52)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.empty((batch, M, N), device="cuda")
    sa, sb = a_st[0].size, b_st[0].size
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch, sa=sa,
                                        sb=sb, sc=M * N)))
    la = np.swapaxes(a_st, 1, 2) if op_a else a_st
    lb = np.swapaxes(b_st, 1, 2) if op_b else b_st
    assert_close(orc, to_host(C), orc.gemm(la, lb), K, what="batched")
    # stride_b = 0 broadcasts B[0] to every batch
    C2 = torch.empty((batch, M, N), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C2, M, N, K, op_a, op_b, batch=batch, sa=sa,
                                        sb=0, sc=M * N)))
    assert_close(orc, to_host(C2), orc.gemm(la, np.ascontiguousarray(lb[:1])), K,
                 what="broadcast")


@pytest.mark.parametrize("N,pad_c", [(60, 5), (61, 3), (64, 4)])
@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 7])
def test_leading_dimensions_larger_than_rows(ck, orc, dev, N, pad_c, cfg):
    # ldc = N + pad_c covers the 16-byte store path (ldc % 4 == 0) with a
    # ragged last column group, and the element-store path (ldc % 4 != 0)
    M, K = 300, 50
    big_a = orc.uniform((M, K + 13), 61)
    big_b = orc.uniform((K, N + 7), 62)
    C_big = torch.full((M, N + pad_c), -7.0, device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, to_dev(big_a), to_dev(big_b), C_big, M, N, K,
                                        lda=K + 13, ldb=N + 7, ldc=N + pad_c, override=cfg)))
    got = to_host(C_big)
    assert_close(orc, got[:, :N], orc.gemm(big_a[:, :K], big_b[:, :N]), K, what="ld")
    assert np.all(got[:, N:] == -7.0), "wrote outside the ldc window"


@pytest.mark.parametrize("structure", [1, 2])
@pytest.mark.parametrize("n", [1, 5, 64, 100, 257, 640])
@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4, 5])
def test_triangular_products(ck, orc, dev, structure, n, cfg):
    tri = np.tril if structure == 1 else np.triu
    a = tri(orc.uniform((n, n), 71))
    b = tri(orc.uniform((n, n), 72))
    C = torch.full((n, n), float("nan"), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, to_dev(a), to_dev(b), C, n, n, n,
                                        structure=structure, override=cfg)))
    got = to_host(C)
    ref = orc.gemm(a, b, structure)
    assert_close(orc, got, ref, n, what=f"tri {structure} n={n} cfg={cfg}")
    zero = np.triu(np.ones((n, n), bool), 1) if structure == 1 else np.tril(np.ones((n, n), bool), -1)
    z = got[zero]
    assert np.all(z == 0.0) and not np.any(np.signbit(z)), "structural zeros must be +0.0"


@pytest.mark.parametrize("structure", [1, 2])
@pytest.mark.parametrize("n,override", [(1024, 3), (1536, 3 | (1 << 8)), (2048, 3 | (5 << 8)),
                                        (2048, 3 | (8 << 8)), (768, 3)])
@pytest.mark.parametrize("triangular_inputs", [True, False])
def test_triangular_chunked_direct(ck, orc, dev, structure, n, override, triangular_inputs):
    """The 256-tile direct kernel on the chunked longest-first work list: long
    tiles are cut in two, the second chunk's partial parked in the mirror tile
    of the zero triangle and added by the finishing pass.  Checks parity,
    +0.0 structural zeros (the parked partials must be gone), the masking of
    non-triangular inputs, the ldc padding, and run-to-run bitwise equality."""
    tri = np.tril if structure == 1 else np.triu
    a, b = orc.uniform((n, n), 75), orc.uniform((n, n), 76)
    if triangular_inputs:
        a, b = tri(a), tri(b)
    ldc = n + 4
    A, B = to_dev(a), to_dev(b)
    outs = []
    for _ in range(2):
        C = torch.full((n, ldc), float("nan"), device="cuda")
        args = gemm_args(ck, A, B, C, n, n, n, ldc=ldc, structure=structure, override=override)
        rc, p = ck.abi.plan(n, n, n, structure=structure, plan_override=override, ldc=ldc)
        assert p.plan_id == 3 and p.num_tiles != p.tiles_m ** 2, "expected the chunked work list"
        ck.abi.check(run_gemm(ck, args))
        outs.append(to_host(C))
    got = outs[0]
    assert np.isnan(got[:, n:]).all(), "a store landed in the ldc padding"
    got = got[:, :n]
    assert_close(orc, got, orc.gemm(a, b, structure), n, what=f"tri-direct {structure} n={n}")
    zero = np.triu(np.ones((n, n), bool), 1) if structure == 1 else np.tril(np.ones((n, n), bool), -1)
    z = got[zero]
    assert np.all(z == 0.0) and not np.any(np.signbit(z)), "structural zeros must be +0.0"
    np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("structure", [1, 2])
def test_triangular_masks_non_triangular_input(ck, orc, dev, structure):
    # The operator is tril(tril(A) tril(B)) / triu(triu(A) triu(B)): entries of
    # the inputs outside the triangle must not leak into the result.
    n = 300
    a, b = orc.uniform((n, n), 73), orc.uniform((n, n), 74)
    C = torch.empty((n, n), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, to_dev(a), to_dev(b), C, n, n, n, structure=structure)))
    assert_close(orc, to_host(C), orc.gemm(a, b, structure), n, what="masked inputs")


@pytest.mark.parametrize("M,K", [(1, 1), (7, 5), (1000, 4096), (4097, 8192), (33, 65536),
                                 (300, 1023), (64, 1 << 18), (5000, 4)])
@pytest.mark.parametrize("with_ws", [True, False])
def test_gemv(ck, orc, dev, M, K, with_ws):
    a = orc.uniform((M, K), 81)
    x = orc.uniform((K,), 82)
    A, X = to_dev(a), to_dev(x)
    y = torch.full((M,), float("nan"), device="cuda")
    L = ck.abi.lib()
    nws = L.mi_gemv_workspace_bytes(M, K)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda") if (with_ws and nws) else None
    ck.abi.check(L.mi_gemv_f32(vp(A), vp(X), vp(y), M, K, vp(ws) if ws is not None else None,
                               nws if ws is not None else 0, cur_stream()), "gemv")
    assert_close(orc, to_host(y), orc.gemv(a, x), K, np.abs(a).max(), np.abs(x).max(), "gemv")


def test_gemv_unaligned_pointer(ck, orc, dev):
    M, K = 129, 2048
    a = orc.uniform((M * K + 1,), 83)
    x = orc.uniform((K + 1,), 84)
    A, X = to_dev(a), to_dev(x)
    y = torch.empty((M,), device="cuda")
    L = ck.abi.lib()
    ck.abi.check(L.mi_gemv_f32(ctypes.c_void_p(A.data_ptr() + 4), ctypes.c_void_p(X.data_ptr() + 4),
                               vp(y), M, K, None, 0, cur_stream()))
    assert_close(orc, to_host(y), orc.gemv(a[1:].reshape(M, K), x[1:]), K, what="gemv unaligned")


@pytest.mark.parametrize("N,M", [(1, 1), (3, 5), (8192, 8), (100, 1027), (513, 4096)])
def test_diag_mult_bitwise(ck, orc, dev, N, M):
    a = orc.uniform((N,), 91)
    b = orc.uniform((N, M), 92)
    out = torch.empty((N, M), device="cuda")
    da, db = to_dev(a), to_dev(b)  # keep the device buffers alive across the launch
    ck.abi.check(ck.abi.lib().mi_diag_mult_f32(vp(da), vp(db), vp(out), N, M, cur_stream()))
    np.testing.assert_array_equal(to_host(out), orc.diag_mult(a, b))


@pytest.mark.parametrize("n,misalign", [(n, m) for n in (1, 3, 4, 5, 2047, 8192, 8192 * 4 + 3, (1 << 22) + 7)
                                         for m in (0, 1)] + [(16384 * 4096, 0)])
def test_matrix_scalar_bitwise(ck, orc, dev, n, misalign):
    """C = A * s (mi_matrix_scalar_mult_f32): one fp32 multiply per element, so
    bitwise equal to the oracle, on the float4 path (chunk multiples, a partial
    chunk, an n % 4 tail) and, with both pointers one float off 16-byte
    alignment, on the scalar path."""
    a = orc.uniform((n + misalign,), 93)
    da = to_dev(a)
    out = torch.empty((n + misalign,), device="cuda")
    L = ck.abi.lib()
    for s in (3.14159, -0.0, 2.0 ** -3):
        out.fill_(7.0)
        ck.abi.check(L.mi_matrix_scalar_mult_f32(ctypes.c_void_p(da.data_ptr() + 4 * misalign),
                                                 ctypes.c_void_p(out.data_ptr() + 4 * misalign),
                                                 n, s, cur_stream()))
        got = to_host(out)
        ref = orc.scale(a[misalign:], s)
        np.testing.assert_array_equal(got[misalign:].view(np.uint32), ref.view(np.uint32),
                                      err_msg=f"n={n} s={s}")
        if misalign:
            assert got[0] == 7.0  # nothing written before the array


def test_matrix_scalar_zero_and_errors(ck, dev):
    L = ck.abi.lib()
    assert L.mi_matrix_scalar_mult_f32(None, None, 0, 2.0, cur_stream()) == 0
    assert L.mi_matrix_scalar_mult_f32(None, None, -1, 2.0, cur_stream()) != 0
    assert L.mi_matrix_scalar_mult_f32(None, None, 5, 2.0, cur_stream()) != 0


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5, 6, 7])
def test_row_bias_every_config(ck, orc, dev, cfg):
    """mi_gemm_args.bias_m: C = A.B + bias[row], one add after the full sum, in
    every tile config's epilogue (ragged M and N, so edge tiles too)."""
    M, N, K = 300, 260, 32
    a, b, bias = orc.uniform((M, K), 94), orc.uniform((K, N), 95), orc.uniform((M,), 96)
    A, B, Bi = to_dev(a), to_dev(b), to_dev(bias)
    C = torch.empty((M, N), device="cuda")
    args = gemm_args(ck, A, B, C, M, N, K, override=cfg)
    args.bias_m = Bi.data_ptr()
    ck.abi.check(run_gemm(ck, args))
    ref = orc.gemm(a, b) + bias.astype(np.float64)[:, None]
    assert_close(orc, to_host(C), ref, K, what=f"bias cfg {cfg}")


def test_row_bias_split_k_zero_k_and_batched(ck, orc, dev):
    """bias with split-K (added once, in the reduction), with K = 0 (C = bias),
    on a batched call, and rejected for triangular structure."""
    M, N, K = 64, 48, 65536
    a, b, bias = orc.uniform((M, K), 97), orc.uniform((K, N), 98), orc.uniform((M,), 99)
    A, B, Bi = to_dev(a), to_dev(b), to_dev(bias)
    C = torch.empty((M, N), device="cuda")
    args = gemm_args(ck, A, B, C, M, N, K, override=3 | (16 << 8))
    args.bias_m = Bi.data_ptr()
    ws = workspace(ck, args)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    ck.abi.check(run_gemm(ck, args))
    assert_close(orc, to_host(C), orc.gemm(a, b) + bias.astype(np.float64)[:, None], K,
                 what="bias split-K")

    C0 = torch.full((M, N), 5.0, device="cuda")
    args0 = gemm_args(ck, A, B, C0, M, N, 0)
    args0.bias_m = Bi.data_ptr()
    ck.abi.check(run_gemm(ck, args0))
    np.testing.assert_array_equal(to_host(C0), np.broadcast_to(bias[:, None], (M, N)))

    nb, Mb, Nb, Kb = 3, 70, 90, 40
    a3, b3 = orc.uniform((nb, Mb, Kb), 100), orc.uniform((nb, Kb, Nb), 101)
    bias3 = orc.uniform((Mb,), 102)
    A3, B3, Bi3 = to_dev(a3), to_dev(b3), to_dev(bias3)
    C3 = torch.empty((nb, Mb, Nb), device="cuda")
    args3 = gemm_args(ck, A3, B3, C3, Mb, Nb, Kb, batch=nb, sa=Mb * Kb, sb=Kb * Nb, sc=Mb * Nb)
    args3.bias_m = Bi3.data_ptr()
    ck.abi.check(run_gemm(ck, args3))
    assert_close(orc, to_host(C3), orc.gemm(a3, b3) + bias3.astype(np.float64)[None, :, None], Kb,
                 what="bias batched")

    T = torch.empty((64, 64), device="cuda")
    argst = gemm_args(ck, T, T, T, 64, 64, 64, structure=1)
    argst.bias_m = Bi.data_ptr()
    assert run_gemm(ck, argst) != 0
    for op_a, op_b in ((1, 0), (0, 1), (1, 1)):  # the bias epilogue is N/N only
        argsl = gemm_args(ck, T, T, T, 64, 64, 64, op_a=op_a, op_b=op_b)
        argsl.bias_m = Bi.data_ptr()
        assert run_gemm(ck, argsl) != 0


def test_symmetric_structure(ck, orc, dev):
    """mi_gemm_f32 with MI_SYMMETRIC equals the dense product of symmetric
    inputs (and the named symmetric entry point, bitwise)."""
    n = 300
    r1, r2 = orc.uniform((n, n), 141), orc.uniform((n, n), 142)
    a, b = (r1 + r1.T) / 2, (r2 + r2.T) / 2
    A, B = to_dev(a), to_dev(b)
    C = torch.empty((n, n), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, n, n, n, structure=3)))
    assert_close(orc, to_host(C), orc.gemm(a, b), n, what="MI_SYMMETRIC")
    C2 = torch.empty((n, n), device="cuda")
    ck.abi.check(ck.abi.lib().mi_symmetric_matmul_f32(vp(A), vp(B), vp(C2), n, None, 0, cur_stream()))
    np.testing.assert_array_equal(to_host(C), to_host(C2))


@pytest.mark.parametrize("n", [300, 1024])
def test_symmetric_operator_on_non_symmetric_inputs(ck, orc, dev, n):
    """PID 13 returns A.B for any input, as kernels/13_...:57,134-151 does
    (it loads B row-major and uses no symmetry): non-symmetric A and B through
    the C entry point, the ATen operator and MI_SYMMETRIC all match the fp64
    A.B, and not A.B^T."""
    a, b = orc.uniform((n, n), 143), orc.uniform((n, n), 144)
    A, B = to_dev(a), to_dev(b)
    ref = orc.gemm(a, b)
    C = torch.empty((n, n), device="cuda")
    ck.abi.check(ck.abi.lib().mi_symmetric_matmul_f32(vp(A), vp(B), vp(C), n, None, 0, cur_stream()))
    got = to_host(C)
    assert_close(orc, got, ref, n, what="mi_symmetric_matmul_f32, non-symmetric")
    wrong = orc.gemm(a, b.T)
    assert orc.norm_err(got, wrong, n, 1.0, 1.0) > 1e-2   # it is not A.B^T
    assert_close(orc, to_host(ck.p13.symmetric_matmul_cuda(A, B)), ref, n,
                 what="p13.symmetric_matmul_cuda, non-symmetric")
    C3 = torch.empty((n, n), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C3, n, n, n, structure=3)))
    np.testing.assert_array_equal(to_host(C3), got)


def test_named_entry_points(ck, orc, dev):
    """Every per-operator C entry point against the oracle on a moderate shape."""
    L = ck.abi.lib()
    s = cur_stream()
    M, K, N = 192, 160, 224
    a, b = orc.uniform((M, K), 101), orc.uniform((K, N), 102)
    A, B = to_dev(a), to_dev(b)

    keep = []

    def d(x):  # device copy that stays alive until the test ends
        t = to_dev(x)
        keep.append(t)
        return vp(t)

    def run(fn, *args):
        ck.abi.check(fn(*args, s), fn.__name__)

    C = torch.empty((M, N), device="cuda")
    run(L.mi_matmul_f32, vp(A), vp(B), vp(C), M, K, N, None, 0)
    assert_close(orc, to_host(C), orc.gemm(a, b), K, what="mi_matmul_f32")
    nws = L.mi_matmul_workspace_bytes(M, K, N)
    wsm = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
    run(L.mi_matmul_f32, vp(A), vp(B), vp(C), M, K, N, vp(wsm), nws)
    assert_close(orc, to_host(C), orc.gemm(a, b), K, what="mi_matmul_f32 with workspace")
    run(L.mi_gemm_small_k_f32, vp(A), vp(B), vp(C), M, K, N)
    assert_close(orc, to_host(C), orc.gemm(a, b), K, what="mi_gemm_small_k_f32")

    sq = orc.uniform((N, N), 103)
    S = to_dev(sq)
    C2 = torch.empty((N, N), device="cuda")
    run(L.mi_square_matmul_f32, vp(S), vp(S), vp(C2), N, None, 0)
    assert_close(orc, to_host(C2), orc.gemm(sq, sq), N, what="square")

    at = orc.uniform((K, M), 104)  # A stored K x M
    bt = orc.uniform((N, K), 105)  # B stored N x K
    At, Bt = to_dev(at), to_dev(bt)
    run(L.mi_matmul_transposed_a_f32, vp(At), vp(B), vp(C), M, K, N, None, 0)
    assert_close(orc, to_host(C), orc.gemm(at.T, b), K, what="transposed_a")
    run(L.mi_matmul_transposed_b_f32, vp(A), vp(Bt), vp(C), M, K, N, None, 0)
    assert_close(orc, to_host(C), orc.gemm(a, bt.T), K, what="transposed_b")
    run(L.mi_matmul_transposed_both_f32, vp(At), vp(Bt), vp(C), M, K, N, None, 0)
    assert_close(orc, to_host(C), orc.gemm(at.T, bt.T), K, what="transposed_both")

    bb, m3, k3, n3 = 3, 40, 56, 72
    a3, b3 = orc.uniform((bb, m3, k3), 106), orc.uniform((bb, k3, n3), 107)
    C3 = torch.empty((bb, m3, n3), device="cuda")
    run(L.mi_batched_matmul_f32, d((a3)), d((b3)), vp(C3), bb, m3, k3, n3, None, 0)
    assert_close(orc, to_host(C3), orc.gemm(a3, b3), k3, what="batched")

    t3 = orc.uniform((4, 33, k3), 108)
    w = orc.uniform((k3, n3), 109)
    O3 = torch.empty((4, 33, n3), device="cuda")
    run(L.mi_tensor3d_matmul_f32, d((t3)), d((w)), vp(O3), 4, 33, k3, n3, None, 0)
    assert_close(orc, to_host(O3).reshape(-1, n3), orc.gemm(t3.reshape(-1, k3), w), k3, what="3d")

    t4 = orc.uniform((2, 3, 5, k3), 110)
    O4 = torch.empty((2, 3, 5, n3), device="cuda")
    run(L.mi_tensor4d_matmul_f32, d((t4)), d((w)), vp(O4), 2, 3, 5, k3, n3, None, 0)
    assert_close(orc, to_host(O4).reshape(-1, n3), orc.gemm(t4.reshape(-1, k3), w), k3, what="4d")

    ta = orc.uniform((300, 24), 111)
    tb = orc.uniform((24, 300), 112)
    O = torch.empty((300, 300), device="cuda")
    run(L.mi_tall_skinny_matmul_f32, d((ta)), d((tb)), vp(O), 300, 24)
    assert_close(orc, to_host(O), orc.gemm(ta, tb), 24, what="tall_skinny")

    r1, r2 = orc.uniform((N, N), 113), orc.uniform((N, N), 114)
    sa, sb = (r1 + r1.T) / 2, (r2 + r2.T) / 2
    run(L.mi_symmetric_matmul_f32, d((sa)), d((sb)), vp(C2), N, None, 0)
    assert_close(orc, to_host(C2), orc.gemm(sa, sb), N, what="symmetric")

    lo_a, lo_b = np.tril(r1), np.tril(r2)
    run(L.mi_lower_tri_mul_f32, d((lo_a)), d((lo_b)), vp(C2), N)
    assert_close(orc, to_host(C2), orc.gemm(lo_a, lo_b, orc.LOWER), N, what="lower")
    up_a, up_b = np.triu(r1), np.triu(r2)
    run(L.mi_upper_tri_matmul_f32, d((up_a)), d((up_b)), vp(C2), N)
    assert_close(orc, to_host(C2), orc.gemm(up_a, up_b, orc.UPPER), N, what="upper")

    Ml, Kl, Nl = 64, 100000, 48
    al, bl = orc.uniform((Ml, Kl), 115), orc.uniform((Kl, Nl), 116)
    nws = L.mi_matmul_large_k_workspace_bytes(Ml, Kl, Nl)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
    Cl = torch.empty((Ml, Nl), device="cuda")
    run(L.mi_matmul_large_k_f32, d((al)), d((bl)), vp(Cl), Ml, Kl, Nl, vp(ws), nws)
    assert_close(orc, to_host(Cl), orc.gemm(al, bl), Kl, what="large_k")


def test_zero_sizes(ck, dev):
    L = ck.abi.lib()
    s = cur_stream()
    C = torch.full((4, 5), 3.0, device="cuda")
    A = torch.ones((4, 0), device="cuda")
    B = torch.ones((0, 5), device="cuda")
    ck.abi.check(L.mi_matmul_f32(vp(A), vp(B), vp(C), 4, 0, 5, None, 0, s))
    assert torch.all(C == 0)
    for M, N in [(0, 5), (4, 0)]:
        assert L.mi_matmul_f32(None, None, None, M, 3, N, None, 0, s) == 0


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5, 6, 7])
def test_repeatability_bitwise(ck, orc, dev, cfg):
    M, N, K = 512, 384, {4: 32, 5: 64, 6: 32, 7: 64}.get(cfg, 1536)
    A, B = dev_uniform(ck, (M, K), 121), dev_uniform(ck, (K, N), 122)
    first = None
    for _ in range(20):
        C = torch.empty((M, N), device="cuda")
        ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, override=cfg)))
        h = to_host(C)
        if first is None:
            first = h
        else:
            np.testing.assert_array_equal(h, first)


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("cfg", [6, 7, 12])
def test_panel_kernel_batched_and_many_column_runs(ck, orc, dev, op_a, op_b, cfg):
    # several batches, several resident panels, ragged last panel and
    # streamed tile
    batch, M, N, K = 3, 600, 2100, 30 if cfg == 6 else 61
    a_st = orc.uniform((batch,) + ((K, M) if op_a else (M, K)), 131)
    b_st = orc.uniform((batch,) + ((N, K) if op_b else (K, N)), 132)
    A, B = to_dev(a_st), to_dev(b_st)
    C = torch.full((batch, M, N), float("nan"), device="cuda")
    ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch,
                                        sa=a_st[0].size, sb=b_st[0].size, sc=M * N, override=cfg)))
    la = np.swapaxes(a_st, 1, 2) if op_a else a_st
    lb = np.swapaxes(b_st, 1, 2) if op_b else b_st
    assert_close(orc, to_host(C), orc.gemm(la, lb), K, what=f"panel cfg {cfg}")


@pytest.mark.parametrize("op_a,op_b", LAYOUTS)
@pytest.mark.parametrize("M,N,K,batch", [(4096, 4096, 64, 1), (1000, 3000, 50, 1), (2048, 1536, 64, 2),
                                         (8192, 2048, 37, 1)])
def test_b_panel_equals_a_panel_bitwise(ck, orc, dev, op_a, op_b, M, N, K, batch):
    """The B-resident panel (config 12) runs the same MFMA sequence per
    output element as the A-resident one (config 7): equal bits, fast and
    ragged paths, batched; and within tolerance of the oracle."""
    a_st = orc.uniform(((batch,) if batch > 1 else ()) + ((K, M) if op_a else (M, K)), 171)
    b_st = orc.uniform(((batch,) if batch > 1 else ()) + ((N, K) if op_b else (K, N)), 172)
    A, B = to_dev(a_st), to_dev(b_st)
    outs = []
    for cfg in (7, 12):
        rc, p = ck.abi.plan(M, N, K, batch=batch, op_a=op_a, op_b=op_b, plan_override=cfg)
        assert rc == 0 and p.plan_id == cfg
        C = torch.full(((batch,) if batch > 1 else ()) + (M, N), float("nan"), device="cuda")
        ck.abi.check(run_gemm(ck, gemm_args(ck, A, B, C, M, N, K, op_a, op_b, batch=batch,
                                            sa=M * K if batch > 1 else 0, sb=K * N if batch > 1 else 0,
                                            sc=M * N if batch > 1 else 0, override=cfg)))
        outs.append(to_host(C))
    np.testing.assert_array_equal(outs[1], outs[0])
    if batch > 1:
        la = np.swapaxes(a_st, 1, 2) if op_a else a_st
        lb = np.swapaxes(b_st, 1, 2) if op_b else b_st
    else:
        la, lb = _logical(a_st, op_a), _logical(b_st, op_b)
    assert_close(orc, outs[1], orc.gemm(la, lb), K, what=f"B panel {op_a}{op_b} {M}x{N}x{K}")
