"""CPU tests that pin the fp64 oracle before it is trusted as the checker.

Pins, in the order the oracle's header lists them:
  * the generator against splitmix64's published output vector;
  * every operator semantic against the committed integer fixtures
    (tests/golden, built with numpy int64 arithmetic -- an independent path);
  * numpy float64 matmul (an independent implementation) on random inputs in
    every layout, batched and triangular;
  * closed forms: identity, permutation, all-ones (C = K), rank-1;
  * brute force from the textbook definition on tiny shapes, including the
    triangular k-range sum_{k=j}^{i};
  * planted mistakes (transposed operand, dropped K term, wrong triangle,
    off-by-one row) that the tolerance check must reject.
"""
import itertools
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "gemm_family_int.npz")


# ---- generator ---------------------------------------------------------------

def test_splitmix64_published_vector(orc):
    # splitmix64 seeded with 1234567 (the sequence in Vigna's reference
    # implementation's test output): state advances by the golden gamma.
    gamma = 0x9E3779B97F4A7C15
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    state = 1234567
    for w in want:
        assert orc.splitmix64(state) == w
        state = (state + gamma) % 2 ** 64
    assert orc.splitmix64(0) == 0xE220A8397B1DCDAF


def test_uniform_generator_is_exact_and_in_range(orc):
    x = orc.uniform((1 << 20,), seed=3).astype(np.float64)
    assert x.min() >= -1.0 and x.max() < 1.0
    assert np.all(x * 2 ** 23 == np.round(x * 2 ** 23))  # multiples of 2^-23
    assert abs(x.mean()) < 5e-3 and abs(x.var() - 1 / 3) < 5e-3
    # counter-based: an offset window equals the tail of the full stream
    np.testing.assert_array_equal(orc.uniform((100,), 3, offset=1000), x[1000:1100].astype(np.float32))
    # value i is a fixed function of (seed, i): recompute two entries by hand
    for i in (0, 777):
        z = orc.splitmix64((3 << 40) + i)
        assert x[i] == (z >> 40) * 2.0 ** -23 - 1.0


def test_integer_generator_range(orc):
    v = orc.integers((100000,), seed=5, lo=-2, hi=2)
    assert set(np.unique(v).tolist()) == {-2.0, -1.0, 0.0, 1.0, 2.0}


# ---- golden fixtures -------------------------------------------------------------

def _golden():
    z = np.load(GOLDEN)  # allow_pickle defaults to False
    names = sorted({k.split(".")[0] for k in z.files})
    return z, names


def _oracle_for(orc, name, A, B):
    """The oracle call for one reference operator semantic."""
    if name == "p03_batched":
        return orc.gemm(A, B)
    if name == "p04_gemv":
        return orc.gemv(A, B[:, 0])[:, None]
    if name == "p10_tensor3d":
        return orc.gemm(A.reshape(-1, A.shape[-1]), B).reshape(A.shape[0], A.shape[1], -1)
    if name == "p11_tensor4d":
        return orc.gemm(A.reshape(-1, A.shape[-1]), B).reshape(A.shape[:-1] + (B.shape[1],))
    if name == "p12_diag":
        return orc.diag_mult(A, B)
    if name == "p05_scalar":
        return orc.scale(A, float(B[0]))
    if name == "p14_upper":
        return orc.gemm(A, B, orc.UPPER)
    if name == "p15_lower":
        return orc.gemm(A, B, orc.LOWER)
    if name == "p16_transposed_a":
        return orc.gemm(A.T, B)
    if name == "p17_transposed_b":
        return orc.gemm(A, B.T)
    if name == "p18_transposed_both":
        return orc.gemm(A.T, B.T)
    return orc.gemm(A, B)


def test_golden_fixtures_cover_every_pid():
    _, names = _golden()
    pids = sorted(int(n[1:3]) for n in names)
    assert pids == list(range(1, 19)) + [87]


@pytest.mark.parametrize("name", _golden()[1])
def test_oracle_matches_golden_exactly(orc, name):
    z, _ = _golden()
    A, B, C = z[f"{name}.A"], z[f"{name}.B"], z[f"{name}.C"]
    if name == "p87_pointwise":
        got = orc.pointwise_conv(A, B, z[f"{name}.bias"])
    else:
        got = _oracle_for(orc, name, A, B)
    np.testing.assert_array_equal(np.asarray(got, dtype=np.float64), C.astype(np.float64))


# ---- independent implementation: numpy float64 -------------------------------------

@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
def test_oracle_matches_numpy_float64(orc, ta, tb):
    M, N, K = 37, 53, 129
    a_st = orc.uniform((K, M) if ta else (M, K), 11)
    b_st = orc.uniform((N, K) if tb else (K, N), 12)
    a = a_st.T if ta else a_st
    b = b_st.T if tb else b_st
    ref = a.astype(np.float64) @ b.astype(np.float64)
    got = orc.gemm(a, b)
    assert np.max(np.abs(got - ref)) <= 1e-12 * K


def test_oracle_batched_and_broadcast(orc):
    a = orc.uniform((4, 9, 17), 13)
    b = orc.uniform((4, 17, 6), 14)
    ref = np.einsum("bik,bkj->bij", a.astype(np.float64), b.astype(np.float64))
    assert np.max(np.abs(orc.gemm(a, b) - ref)) <= 1e-12
    ref0 = np.einsum("bik,kj->bij", a.astype(np.float64), b[0].astype(np.float64))
    assert np.max(np.abs(orc.gemm(a, b[:1]) - ref0)) <= 1e-12


@pytest.mark.parametrize("structure", [1, 2])
def test_oracle_triangular_vs_numpy(orc, structure):
    n = 70
    a, b = orc.uniform((n, n), 15), orc.uniform((n, n), 16)  # not triangular: inputs get masked
    tri = np.tril if structure == 1 else np.triu
    ref = tri(tri(a).astype(np.float64) @ tri(b).astype(np.float64))
    got = orc.gemm(a, b, structure)
    assert np.max(np.abs(got - ref)) <= 1e-12
    assert np.all(got[tri(np.ones((n, n), bool)) == 0] == 0.0)


def test_oracle_rows_and_entries(orc):
    a, b = orc.uniform((40, 30), 17), orc.uniform((30, 20), 18)
    full = orc.gemm(a, b)
    rows = [0, 7, 39]
    np.testing.assert_array_equal(orc.gemm(a, b, rows=rows), full[rows])
    bij = np.array([[0, 3, 4], [0, 39, 19], [0, 0, 0]])
    np.testing.assert_array_equal(orc.gemm_entries(a, b, bij), full[bij[:, 1], bij[:, 2]])


def test_gemv_and_generated_rows(orc):
    M, K = 50, 333
    a, x = orc.uniform((M, K), 19), orc.uniform((K,), 20)
    ref = a.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(orc.gemv(a, x) - ref)) <= 1e-12
    rows = [0, 13, 49]
    np.testing.assert_array_equal(orc.gemv_generated(19, x, rows), orc.gemv(a, x)[rows])


def test_diag_is_one_fp32_multiply(orc):
    a, b = orc.uniform((33,), 21), orc.uniform((33, 19), 22)
    np.testing.assert_array_equal(orc.diag_mult(a, b), a[:, None] * b)


def test_scale_pins(orc):
    """C = A * s (kernels/5_...:10-42): powers of two are exact (ldexp), s = 1
    is the identity, s = -1 flips every sign bit, s = 0 gives zeros carrying
    the sign of A, and a non-finite A stays non-finite.  A planted mistake (s
    applied twice, an off-by-one element) fails these."""
    a = orc.uniform((1001,), 24)
    bits = lambda x: np.asarray(x, dtype=np.float32).view(np.uint32)
    for e in (-3, 0, 5):
        np.testing.assert_array_equal(orc.scale(a, 2.0 ** e), np.ldexp(a, e).astype(np.float32))
    np.testing.assert_array_equal(bits(orc.scale(a, 1.0)), bits(a))
    np.testing.assert_array_equal(bits(orc.scale(a, -1.0)), bits(a) ^ np.uint32(0x80000000))
    z = orc.scale(a, 0.0)
    np.testing.assert_array_equal(np.signbit(z), np.signbit(a))
    assert not np.any(z)
    special = np.array([np.inf, -np.inf, np.nan, 1.0], dtype=np.float32)
    out = orc.scale(special, 0.0)
    assert np.isnan(out[:3]).all() and out[3] == 0.0
    # shape-preserving, 2-D input (the operator's output is empty_like(A))
    m = orc.uniform((17, 9), 25)
    assert orc.scale(m, 3.0).shape == (17, 9)
    wrong = orc.scale(orc.scale(m, 3.0), 3.0)  # planted: s applied twice
    assert not np.array_equal(wrong, orc.scale(m, 3.0))


def test_pointwise_conv_pins(orc):
    """1x1 convolution (kernels/87_...:451-492) against numpy float64 einsum
    (independent), the identity weight (out = x + bias exactly), a zero weight
    (out = bias broadcast), and planted mistakes: weight transposed, bias
    dropped, bias added per input channel instead of once."""
    x = orc.uniform((3, 7, 5, 6), 26)
    w = orc.uniform((9, 7, 1, 1), 27)
    b = orc.uniform((9,), 28)
    ref = np.einsum("oc,nchw->nohw", w[:, :, 0, 0].astype(np.float64), x.astype(np.float64))
    ref += b.astype(np.float64)[None, :, None, None]
    got = orc.pointwise_conv(x, w, b)
    assert got.shape == (3, 9, 5, 6)
    assert np.max(np.abs(got - ref)) <= 1e-12
    # a Cout x Cin weight and its Cout x Cin x 1 x 1 form are the same operator
    np.testing.assert_array_equal(orc.pointwise_conv(x, w[:, :, 0, 0], None),
                                  orc.pointwise_conv(x, w, None))
    eye = np.eye(7, dtype=np.float32)
    bi = orc.uniform((7,), 29)
    np.testing.assert_array_equal(orc.pointwise_conv(x, eye, bi),
                                  x.astype(np.float64) + bi.astype(np.float64)[None, :, None, None])
    z = orc.pointwise_conv(x, np.zeros((9, 7), np.float32), b)
    np.testing.assert_array_equal(z, np.broadcast_to(b.astype(np.float64)[None, :, None, None], z.shape))
    sq = orc.uniform((7, 7), 30)
    planted = [
        orc.pointwise_conv(x, sq.T.copy(), None),                 # transposed weight
        orc.pointwise_conv(x, sq, None),                          # bias dropped
        orc.pointwise_conv(x, sq, bi) + 6 * bi.astype(np.float64)[None, :, None, None],  # bias per channel
    ]
    want = np.einsum("oc,nchw->nohw", sq.astype(np.float64), x.astype(np.float64)) + \
        bi.astype(np.float64)[None, :, None, None]
    for bad in planted:
        assert np.max(np.abs(bad - want)) > 1e-3


def test_half_decoder_exhaustive(orc):
    """orc_half_to_double on all 65536 binary16 patterns equals numpy's
    float16 -> float64 conversion (NaN patterns decode to NaN)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float64)
    f = orc.lib().orc_half_to_double
    got = np.array([f(int(b)) for b in bits], dtype=np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan], want[~nan])


def _np_sdpa(q, k, v, scale):
    q, k, v = (x.astype(np.float64) for x in (q, k, v))
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    s -= s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=-1, keepdims=True)
    return np.matmul(w, v)


def test_sdpa_pins(orc):
    """Attention (kernels/97_...:136-296) against an independent numpy float64
    implementation, the closed forms of identical keys (uniform weights: the
    mean of V) and of one dominant key (its V row), and planted mistakes
    (no scale, softmax over queries, V transposed per head)."""
    shape = (2, 3, 9, 16)
    q = orc.uniform(shape, 31).astype(np.float16)
    k = orc.uniform(shape, 32).astype(np.float16)
    v = orc.uniform(shape, 33).astype(np.float16)
    scale = 1.0 / 4.0
    got = orc.sdpa(q, k, v)
    ref = _np_sdpa(q, k, v, scale)
    assert got.shape == shape and np.max(np.abs(got - ref)) <= 1e-12
    same_k = np.broadcast_to(k[:, :, :1, :], shape).copy()
    np.testing.assert_allclose(orc.sdpa(q, same_k, v), np.broadcast_to(
        v.astype(np.float64).mean(axis=-2, keepdims=True), shape), rtol=0, atol=1e-12)
    # one key aligned with every query and 8x longer: its weight -> 1
    k1 = np.zeros((1, 1, 4, 16), np.float16)
    k1[0, 0, 2, 0] = 8.0
    q1 = np.zeros((1, 1, 4, 16), np.float16)
    q1[..., 0] = 8.0
    v1 = orc.uniform((1, 1, 4, 16), 34).astype(np.float16)
    o1 = orc.sdpa(q1, k1, v1, scale=1.0)
    np.testing.assert_allclose(o1, np.broadcast_to(v1[0, 0, 2].astype(np.float64), o1.shape), atol=1e-12)
    planted = [_np_sdpa(q, k, v, 1.0),
               np.swapaxes(_np_sdpa(np.swapaxes(q, -1, -2), np.swapaxes(k, -1, -2),
                                    np.swapaxes(v, -1, -2), scale), -1, -2),
               _np_sdpa(q, k, np.swapaxes(v[..., :9, :9], -1, -2).copy(), scale)]
    for bad in planted:
        assert bad.shape != got.shape or np.max(np.abs(bad - got)) > 1e-3


def test_half_ulp(orc):
    np.testing.assert_array_equal(orc.half_ulp(np.array([1.0, 1.5, 2.0, 0.04, 0.0, 2.0 ** -20])),
                                  [2.0 ** -10, 2.0 ** -10, 2.0 ** -9, 2.0 ** -15, 2.0 ** -24, 2.0 ** -24])


# ---- closed forms ------------------------------------------------------------------

def test_closed_forms(orc):
    n = 48
    X = orc.uniform((n, n), 23)
    I = np.eye(n, dtype=np.float32)
    np.testing.assert_array_equal(orc.gemm(I, X), X.astype(np.float64))
    np.testing.assert_array_equal(orc.gemm(X, I), X.astype(np.float64))
    perm = np.random.default_rng(0).permutation(n)
    P = I[perm]
    np.testing.assert_array_equal(orc.gemm(P, X), X[perm].astype(np.float64))
    ones_a, ones_b = np.ones((5, 1000), np.float32), np.ones((1000, 3), np.float32)
    np.testing.assert_array_equal(orc.gemm(ones_a, ones_b), np.full((5, 3), 1000.0))
    u = orc.integers((n, 1), 24, -3, 3)
    v = orc.integers((1, n), 25, -3, 3)
    np.testing.assert_array_equal(orc.gemm(u, v), (u * v).astype(np.float64))


# ---- brute force from the definition ------------------------------------------------

def _brute(a, b, structure=0):
    M, K = a.shape
    N = b.shape[1]
    out = np.zeros((M, N))
    for i in range(M):
        for j in range(N):
            if structure == 1:      # C[i][j] = sum_{k=j}^{i} A[i][k] B[k][j], 0 above
                ks = range(j, i + 1)
            elif structure == 2:    # C[i][j] = sum_{k=i}^{j} A[i][k] B[k][j], 0 below
                ks = range(i, j + 1)
            else:
                ks = range(K)
            out[i, j] = math.fsum(float(a[i, k]) * float(b[k, j]) for k in ks)
    return out


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (2, 3, 4), (5, 1, 7), (6, 6, 6)])
def test_brute_force_dense(orc, M, N, K):
    a, b = orc.uniform((M, K), 26), orc.uniform((K, N), 27)
    assert np.max(np.abs(orc.gemm(a, b) - _brute(a, b))) <= 1e-14


@pytest.mark.parametrize("structure", [1, 2])
@pytest.mark.parametrize("n", [1, 2, 5, 8])
def test_brute_force_triangular(orc, structure, n):
    tri = np.tril if structure == 1 else np.triu
    a, b = tri(orc.uniform((n, n), 28)), tri(orc.uniform((n, n), 29))
    assert np.max(np.abs(orc.gemm(a, b, structure) - _brute(a, b, structure))) <= 1e-14


# ---- the tolerance check rejects plausible mistakes ----------------------------------

def test_planted_mistakes_are_caught(orc):
    M = N = K = 128  # square, so a transposed operand has the right shape
    a, b = orc.uniform((M, K), 30), orc.uniform((K, N), 31)
    ref = orc.gemm(a, b)
    ok = ref.astype(np.float32)
    assert orc.norm_err(ok, ref, K, 1, 1) <= orc.TOL
    wrong = {
        "transposed operand": orc.gemm(a, np.ascontiguousarray(b.T)),
        "dropped last K term": orc.gemm(a[:, :-1], b[:-1]),
        "off-by-one row": np.roll(ref, 1, axis=0),
        "sign flip": -ref,
    }
    for what, bad in wrong.items():
        err = orc.norm_err(bad.astype(np.float32), ref, K, 1, 1)
        assert err > orc.TOL, f"{what} slipped through ({err:.2e})"
    # wrong triangle for the structured products
    n = 32
    la, lb = np.tril(orc.uniform((n, n), 32)), np.tril(orc.uniform((n, n), 33))
    good = orc.gemm(la, lb, orc.LOWER)
    bad = orc.gemm(la, lb, orc.UPPER)
    assert orc.norm_err(bad.astype(np.float32), good, n, 1, 1) > orc.TOL
    # NaN is never within tolerance
    nan = ok.copy()
    nan[3, 3] = np.nan
    assert orc.norm_err(nan, ref, K, 1, 1) == math.inf


def test_fp32_accumulation_error_is_far_below_tolerance(orc):
    # sanity of the bar itself: a plain fp32 sequential sum at K = 8192 lands
    # orders of magnitude below 1e-4 normalised, so the tolerance is not loose
    # enough to hide a wrong algorithm yet not tight enough to reject fp32.
    K = 8192
    a, b = orc.uniform((8, K), 34), orc.uniform((K, 8), 35)
    ref = orc.gemm(a, b)
    acc = np.zeros((8, 8), np.float32)
    for k in range(K):
        acc += np.outer(a[:, k], b[k, :]).astype(np.float32)
    err = orc.norm_err(acc, ref, K, 1, 1)
    assert err < 1e-5


# ---- whole-output checksums (full-size tests) ------------------------------------

def test_matvec_and_checksums_vs_numpy(orc):
    a = orc.uniform((300, 200), 901)
    v = np.random.default_rng(0).standard_normal(200)
    u = np.random.default_rng(1).standard_normal(300)
    np.testing.assert_allclose(orc.matvec(a, v), a.astype(np.float64) @ v, rtol=1e-13, atol=1e-12)
    # a transposed view is read in place through its strides
    np.testing.assert_allclose(orc.matvec(a.T, u), a.astype(np.float64).T @ u, rtol=1e-13, atol=1e-12)
    cv, utc = orc.checksums(a, v, u)
    np.testing.assert_allclose(cv, a.astype(np.float64) @ v, rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose(utc, u @ a.astype(np.float64), rtol=1e-13, atol=1e-12)
    # block by block (row slices, a padded row stride) accumulates the same
    # column checksums
    big = orc.uniform((300, 256), 902)
    blk = big[:, :200]
    acc = np.zeros(200)
    parts = []
    for r0 in range(0, 300, 64):
        c, acc = orc.checksums(blk[r0:r0 + 64], v, u[r0:r0 + 64], acc)
        parts.append(c)
    np.testing.assert_allclose(np.concatenate(parts), blk.astype(np.float64) @ v, rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose(acc, u @ blk.astype(np.float64), rtol=1e-12, atol=1e-11)


def test_freivalds_accepts_fp32_products_and_catches_planted_mistakes(orc):
    import freivalds as fv
    M, K, N = 512, 1024, 384
    a, b = orc.uniform((M, K), 903), orc.uniform((K, N), 904)
    v, u = fv.signs(N, 5), fv.signs(M, 6)
    ref_cv, ref_utc = fv.reference(orc, a, b, v, u)
    np.testing.assert_allclose(ref_cv, orc.gemm(a, b) @ v, rtol=1e-10, atol=1e-8)
    np.testing.assert_allclose(ref_utc, u @ orc.gemm(a, b), rtol=1e-10, atol=1e-8)
    c = (a @ b).astype(np.float32)             # an fp32-accumulated product passes
    fv.check(orc, *orc.checksums(c, v, u), ref_cv, ref_utc, K, 1.0, 1.0, "fp32 product")
    # transposed-operand layouts through views
    at = np.ascontiguousarray(a.T)
    cv_t, utc_t = fv.reference(orc, at.T, b, v, u)
    np.testing.assert_allclose(cv_t, ref_cv, rtol=1e-13, atol=1e-10)
    plants = {
        "one 32x32 block zero": lambda x: x.__setitem__((slice(64, 96), slice(32, 64)), 0.0),
        "one tile from the wrong K range": lambda x: x.__setitem__(
            (slice(0, 128), slice(0, 128)), (a[:128, :512] @ b[:512, :128]).astype(np.float32)),
        "one row shifted": lambda x: x.__setitem__(7, np.roll(x[7], 1)),
        "one element off by 1": lambda x: x.__setitem__((100, 200), x[100, 200] + 1.0),
        "sign flip of one column": lambda x: x.__setitem__((slice(None), 5), -x[:, 5]),
    }
    for name, plant in plants.items():
        bad = c.copy()
        plant(bad)
        with pytest.raises(AssertionError):
            fv.check(orc, *orc.checksums(bad, v, u), ref_cv, ref_utc, K, 1.0, 1.0, name)
