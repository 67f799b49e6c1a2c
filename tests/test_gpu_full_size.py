"""Parity at BASELINE.json's full sizes, on the GPU, through the drop-in operators.

Inputs come from the device generator with the BASELINE seeds (16*cfg + tensor);
the host regenerates or copies them for the fp64 oracle.  Every output element
of every config is checked:
  * outputs small enough for an fp64 reference of the whole product (1024^3,
    small-K, diag, GEMV) are compared element by element;
  * the others enter fp64 row and column checksums, C.v against A.(B.v) and
    u^T.C against (u^T.A).B with random +-1 vectors (tests/freivalds.py gives
    the bounds), reduced on the host in row blocks, plus exact fp64 values of
    sampled rows (tile-boundary rows included) and entries;
plus size-independent properties: exact structural zeros, symmetry of the
inputs, bitwise repeatability of split-K.  Tolerance: the north-star bound 1e-4.
"""
import numpy as np
import pytest
import torch

import freivalds as fv
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


def _dev_checksums(orc, C, v, u, block_bytes=1 << 29):
    """fp64 C.v and u^T.C of a 2-D device tensor, copied to the host in row
    blocks of at most block_bytes."""
    M, N = C.shape
    rows = max(1, block_bytes // (4 * N))
    cv = np.empty(M, dtype=np.float64)
    utc = np.zeros(N, dtype=np.float64)
    for r0 in range(0, M, rows):
        blk = to_host(C[r0:r0 + rows])
        cv[r0:r0 + rows], utc = orc.checksums(blk, v, u[r0:r0 + rows], utc)
    return cv, utc


def _whole(orc, C, a, b, K, seed, what):
    """Every element of device output C (M x N) against the fp64 a.b (host
    fp32 operands or views) through row and column checksums."""
    M, N = C.shape
    v, u = fv.signs(N, seed), fv.signs(M, seed + 1)
    ref = fv.reference(orc, a, b, v, u)
    return fv.check(orc, *_dev_checksums(orc, C, v, u), *ref, K, 1.0, 1.0, what)


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
    _whole(orc, C, la, lb, n, 100, f"8192 {layout} every element")


def test_cfg2_batched(ck, orc):
    bsz, M, K, N = 128, 512, 1024, 768
    A = dev_uniform(ck, (bsz, M, K), 32)
    B = dev_uniform(ck, (bsz, K, N), 33)
    C = ck.p03.batched_matmul_cuda(A, B)
    Ah, Bh = to_host(A), to_host(B)
    for bi in (0, 77, 127):
        assert_close(orc, to_host(C[bi]), orc.gemm(Ah[bi], Bh[bi]), K, what=f"batched b={bi}")
    for bi in range(bsz):   # every batch, every element
        _whole(orc, C[bi], Ah[bi], Bh[bi], K, 200 + 2 * bi, f"batched b={bi} every element")


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
    _whole(orc, out.reshape(-1, L), flat, to_host(B), K, 300, "3d every element")


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
    _whole(orc, out.reshape(-1, k), flat, to_host(B), l, 400, "4d every element")


def test_cfg3_gemv_full_size(ck, orc):
    M, K = 32768, 65536
    A = dev_uniform(ck, (M, K), 48)
    x = dev_uniform(ck, (K, 1), 50)
    y = to_host(ck.p04.gemv_cuda(A, x))[:, 0]
    # every row; A (8 GiB) is regenerated row by row on the host
    ref = orc.gemv_generated(48, to_host(x)[:, 0], np.arange(M))
    assert_close(orc, y, ref, K, what="gemv every row")
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
    Cd = ck.p06.matmul_cuda(A, B)
    C1 = to_host(Cd)
    C2 = to_host(ck.p06.matmul_cuda(A, B))
    np.testing.assert_array_equal(C1, C2)
    a, b = to_host(A), to_host(B)
    bij = _entries(M, N, 512)
    assert_close(orc, C1[bij[:, 1], bij[:, 2]], orc.gemm_entries(a, b, bij), K,
                 what="large-K entries")
    _whole(orc, Cd, a, b, K, 500, "large-K every element")


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
    # the 16 GiB output, every element, reduced in 512 MiB row blocks
    _whole(orc, C, a, b, K, 600, "tall-skinny every element")


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
    a, b = to_host(A), to_host(B)
    got = to_host(C[rows])
    assert_close(orc, got, orc.gemm(a, b, s, rows=rows), n, what=structure)
    # tril(A).tril(B) is itself lower triangular (triu likewise), so the
    # whole C equals a.b with the masked inputs
    _whole(orc, C, a, b, n, 700, f"{structure} every element")
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
    a, b = to_host(A), to_host(B)
    assert_close(orc, to_host(C[rows]), orc.gemm(a, b, rows=rows), n, what="symmetric")
    _whole(orc, C, a, b, n, 800, "symmetric every element")


def test_sdpa_bench_shape_every_chunk(ck, orc, dev):
    """PID 97 at the bench shape (32, 32, 512, 1024): 1,024 heads, i.e. eight
    chunks of 128 heads through the workspace.  One head of every chunk (at a
    different position in each) is checked against the fp64 oracle to the
    attention bound (one binary16 spacing + 2^-17 max|V|); every head is
    checked for the convexity of softmax weights: each output lies within the
    [min, max] of its V column (plus one fp16 spacing), with no NaN."""
    shape = (32, 32, 512, 1024)
    Q, K, V = (dev_uniform(ck, shape, 970 + i).half() for i in range(3))
    O = ck.p97.fused_attention_cuda(Q, K, V)
    torch.cuda.synchronize()
    assert not torch.isnan(O).any()
    Of, Vf = O.float().view(1024, 512, 1024), V.float().view(1024, 512, 1024)
    lo, hi = Vf.amin(dim=1, keepdim=True), Vf.amax(dim=1, keepdim=True)
    slack = 2.0 ** -10 * torch.maximum(lo.abs(), hi.abs())
    assert bool(((Of >= lo - slack) & (Of <= hi + slack)).all())
    qh, kh, vh = (t.view(1024, 512, 1024) for t in (Q, K, V))
    for c in range(8):
        h = 128 * c + (37 * c + 5) % 128
        q, k, v = (to_host(t[h]) for t in (qh, kh, vh))
        ref = orc.sdpa(q, k, v)
        err = np.abs(to_host(Of[h]).astype(np.float64) - ref)
        bound = orc.half_ulp(ref) + 2.0 ** -17 * float(np.max(np.abs(v.astype(np.float64))))
        assert float(np.max(err / bound)) <= 1.0, f"head {h}: error {float(np.max(err / bound)):.2f} x bound"


def test_pointwise_conv_bench_shape(ck, orc, dev):
    """PID 87 at the bench shape (16, 64, 128, 256, 256) with bias: the
    128-row A-resident panel over 16 images of 65,536 pixels.  Every output
    element enters per-image fp64 row and column checksums (the conv is
    out[n] = W . X[n] + bias, tests/freivalds.py), and sampled pixels of every
    image are compared with the fp64 oracle element by element."""
    n, cin, cout, hw = 16, 64, 128, 256 * 256
    X = dev_uniform(ck, (n, cin, 256, 256), 980)
    W = dev_uniform(ck, (cout, cin, 1, 1), 981)
    bias = dev_uniform(ck, (cout,), 982)
    out = ck.p87.pointwise_conv_cuda(X, W, bias)
    assert tuple(out.shape) == (n, cout, 256, 256)
    w = to_host(W).reshape(cout, cin)
    b64 = to_host(bias).astype(np.float64)
    cols = np.r_[0:200, 32768 - 100:32768 + 100, hw - 200:hw]
    for i in range(n):
        x = to_host(X[i]).reshape(cin, hw)
        got = to_host(out[i]).reshape(cout, hw)
        v, u = fv.signs(hw, 990 + i), fv.signs(cout, 1990 + i)
        ref_cv, ref_utc = fv.reference(orc, w, x, v, u)
        ref_cv = ref_cv + b64 * v.sum()
        ref_utc = ref_utc + float(u @ b64)
        fv.check(orc, got.astype(np.float64) @ v, u @ got.astype(np.float64), ref_cv, ref_utc, cin,
                 1.0, 1.0, what=f"conv image {i}")
        ref = orc.gemm(w, np.ascontiguousarray(x[:, cols])) + b64[:, None]
        assert_close(orc, got[:, cols], ref, cin, what=f"conv image {i} sampled pixels")
