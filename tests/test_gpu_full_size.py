"""Parity at BASELINE.json's full sizes, on the GPU, through the drop-in operators.

Inputs come from the device generator with the BASELINE seeds (16*cfg + tensor);
the host regenerates or copies them for the fp64 oracle.  Where a dense fp64
reference of the whole output would not fit the test budget, the check is on
sampled rows (including tile-boundary rows) and sampled entries, plus
size-independent properties: exact structural zeros, symmetry of the inputs,
bitwise repeatability of split-K.  Tolerance: the north-star bound 1e-4.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, dev_uniform, to_host

pytestmark = pytest.mark.gpu


def _rows(M, extra=8, seed=0):
    rng = np.random.default_rng(seed)
    fixed = [0, 1, 63, 64, 127, 128, 255, 256, M // 2, M - 1]
    rows = sorted({r for r in fixed if 0 <= r < M} | set(rng.integers(0, M, extra).tolist()))
    return rows


def _entries(M, N, count=1024, seed=1):
    rng = np.random.default_rng(seed)
    return np.stack([np.zeros(count, np.int64), rng.integers(0, M, count),
                     rng.integers(0, N, count)], axis=1)


def test_cfg0_square_1024_full(ck, orc):
    A = dev_uniform(ck, (1024, 1024), 0)
    B = dev_uniform(ck, (1024, 1024), 1)
    C = to_host(ck.p01.matmul_cuda(A, B))
    assert_close(orc, C, orc.gemm(to_host(A), to_host(B)), 1024, what="cfg0 1024^3")


@pytest.mark.parametrize("layout", ["NN", "TN", "NT", "TT"])
def test_cfg1_8192_four_layouts(ck, orc, layout):
    n = 8192
    A = dev_uniform(ck, (n, n), 16)   # stored operand (K x M when A is transposed)
    B = dev_uniform(ck, (n, n), 17)
    fn = {"NN": ck.p01.matmul_cuda, "TN": ck.p16.matmul_transposed_cuda,
          "NT": ck.p17.matmul_cuda, "TT": ck.p18.matmul_transposed_cuda}[layout]
    C = fn(A, B)
    a, b = to_host(A), to_host(B)
    la = a.T if layout[0] == "T" else a
    lb = b.T if layout[1] == "T" else b
    rows = _rows(n, extra=4)
    got_rows = to_host(C[rows])
    assert_close(orc, got_rows, orc.gemm(la, lb, rows=rows), n, what=f"8192 {layout} rows")
    bij = _entries(n, n, 2048)
    got = to_host(C)[bij[:, 1], bij[:, 2]]
    assert_close(orc, got, orc.gemm_entries(la, lb, bij), n, what=f"8192 {layout} entries")


def test_cfg2_batched(ck, orc):
    bsz, M, K, N = 128, 512, 1024, 768
    A = dev_uniform(ck, (bsz, M, K), 32)
    B = dev_uniform(ck, (bsz, K, N), 33)
    C = ck.p03.batched_matmul_cuda(A, B)
    for bi in (0, 77, 127):
        a, b = to_host(A[bi]), to_host(B[bi])
        assert_close(orc, to_host(C[bi]), orc.gemm(a, b), K, what=f"batched b={bi}")


def test_cfg2_tensor3d(ck, orc):
    n, M, K, L = 16, 1024, 2048, 768
    A = dev_uniform(ck, (n, M, K), 34)
    B = dev_uniform(ck, (K, L), 35)
    out = ck.p10.batched_matmul_cuda(A, B)
    assert tuple(out.shape) == (n, M, L)
    flat = to_host(A).reshape(-1, K)
    rows = _rows(n * M, extra=16)
    assert_close(orc, to_host(out.reshape(-1, L)[rows]), orc.gemm(flat, to_host(B), rows=rows), K,
                 what="3d")


def test_cfg2_tensor4d(ck, orc):
    b, i, j, l, k = 8, 64, 128, 256, 512
    A = dev_uniform(ck, (b, i, j, l), 36)
    B = dev_uniform(ck, (l, k), 37)
    out = ck.p11.tensor_matmul_cuda(A, B)
    assert tuple(out.shape) == (b, i, j, k)
    flat = to_host(A).reshape(-1, l)
    rows = _rows(b * i * j, extra=16)
    assert_close(orc, to_host(out.reshape(-1, k)[rows]), orc.gemm(flat, to_host(B), rows=rows), l,
                 what="4d")


def test_cfg3_gemv_full_size(ck, orc):
    M, K = 32768, 65536
    A = dev_uniform(ck, (M, K), 48)
    x = dev_uniform(ck, (K, 1), 50)
    y = to_host(ck.p04.gemv_cuda(A, x))[:, 0]
    rows = _rows(M, extra=64)
    ref = orc.gemv_generated(48, to_host(x)[:, 0], rows)   # A regenerated row by row on the host
    assert_close(orc, y[rows], ref, K, what="gemv rows")
    assert np.all(np.isfinite(y))


def test_cfg3_small_k_full_output(ck, orc):
    M = N = 16384
    K = 32
    A = dev_uniform(ck, (M, K), 51)
    B = dev_uniform(ck, (K, N), 52)
    C = to_host(ck.p07.gemm_cuda(A, B))
    assert_close(orc, C, orc.gemm(to_host(A), to_host(B)), K, what="small-K full")


def test_cfg3_diag_bitwise(ck, orc):
    a = dev_uniform(ck, (8192,), 53)
    B = dev_uniform(ck, (8192, 8192), 54)
    out = to_host(ck.p12.diag_mult_cuda(a, B))
    np.testing.assert_array_equal(out, orc.diag_mult(to_host(a), to_host(B)))


def test_cfg4_large_k_split_deterministic(ck, orc):
    M = N = 256
    K = 1 << 20
    A = dev_uniform(ck, (M, K), 64)
    B = dev_uniform(ck, (K, N), 65)
    C1 = to_host(ck.p06.matmul_cuda(A, B))
    C2 = to_host(ck.p06.matmul_cuda(A, B))
    np.testing.assert_array_equal(C1, C2)
    bij = _entries(M, N, 512)
    assert_close(orc, C1[bij[:, 1], bij[:, 2]], orc.gemm_entries(to_host(A), to_host(B), bij), K,
                 what="large-K entries")


def test_cfg4_tall_skinny(ck, orc):
    M, K = 65536, 64
    A = dev_uniform(ck, (M, K), 66)
    B = dev_uniform(ck, (K, M), 67)
    C = ck.p09.tall_skinny_matmul_cuda(A, B)
    assert tuple(C.shape) == (M, M)
    rows = _rows(M, extra=6)
    a, b = to_host(A), to_host(B)
    assert_close(orc, to_host(C[rows]), orc.gemm(a, b, rows=rows), K, what="tall-skinny rows")
    cols = [0, 255, 256, 40000, M - 1]
    got = to_host(C[:, cols])
    ref = orc.gemm(a, np.ascontiguousarray(b[:, cols]))
    assert_close(orc, got, ref, K, what="tall-skinny cols")


@pytest.mark.parametrize("structure", ["lower", "upper"])
def test_cfg4_triangular(ck, orc, structure):
    n = 8192
    tri = torch.tril if structure == "lower" else torch.triu
    A = tri(dev_uniform(ck, (n, n), 68))
    B = tri(dev_uniform(ck, (n, n), 69))
    fn = ck.p15.lower_tri_mul_cuda if structure == "lower" else ck.p14.upper_tri_matmul_cuda
    C = fn(A, B)
    s = orc.LOWER if structure == "lower" else orc.UPPER
    rows = _rows(n, extra=6)
    got = to_host(C[rows])
    assert_close(orc, got, orc.gemm(to_host(A), to_host(B), s, rows=rows), n, what=structure)
    # every element on the wrong side of the diagonal is exactly +0.0
    Ch = to_host(C)
    wrong = np.triu(np.ones((n, n), bool), 1) if structure == "lower" else np.tril(np.ones((n, n), bool), -1)
    z = Ch[wrong]
    assert np.all(z == 0.0) and not np.any(np.signbit(z))


def test_cfg4_symmetric(ck, orc):
    n = 8192
    R1 = dev_uniform(ck, (n, n), 70)
    R2 = dev_uniform(ck, (n, n), 71)
    A = (R1 + R1.t()) / 2
    B = (R2 + R2.t()) / 2
    assert torch.equal(A, A.t()) and torch.equal(B, B.t())
    C = ck.p13.symmetric_matmul_cuda(A, B)
    rows = _rows(n, extra=4)
    assert_close(orc, to_host(C[rows]), orc.gemm(to_host(A), to_host(B), rows=rows), n,
                 what="symmetric")
