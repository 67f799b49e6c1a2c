"""Writes tests/golden/gemm_family_int.npz: small known-answer cases for every
operator semantic of the GEMM-family path (reference kernels/1..18 and the
pointwise convolution of kernels/87).

The reference ships no tests, fixtures or golden vectors, so these are built
from closed forms: integer-valued fp32 inputs in [-3, 3] whose products and
sums are exact in fp32 and fp64, with the expected outputs computed here in
numpy *int64* arithmetic -- an implementation independent of the fp64 oracle
(oracle/oracle.c) and of the kernels, both of which are checked against it.

Shapes follow the reference wrappers' shape logic (file:line per case).
Run:  python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "gemm_family_int.npz")


def ints(rng, shape):
    return rng.integers(-3, 4, size=shape).astype(np.int64)


def main():
    rng = np.random.default_rng(20261201)
    cases = {}

    def add(name, **arrays):
        for k, v in arrays.items():
            cases[f"{name}.{k}"] = v.astype(np.float32) if v.dtype != np.float32 else v

    # kernels/1_...:190 square, N x N
    a, b = ints(rng, (9, 9)), ints(rng, (9, 9))
    add("p01_square", A=a, B=b, C=a @ b)
    # kernels/2_...:122-124 and 8_...:156-160 rectangular / irregular
    a, b = ints(rng, (7, 13)), ints(rng, (13, 5))
    add("p02_matmul", A=a, B=b, C=a @ b)
    a, b = ints(rng, (33, 17)), ints(rng, (17, 65))
    add("p08_irregular", A=a, B=b, C=a @ b)
    # kernels/3_...:126-131 batched
    a, b = ints(rng, (3, 4, 6)), ints(rng, (3, 6, 5))
    add("p03_batched", A=a, B=b, C=np.einsum("bik,bkj->bij", a, b))
    # kernels/4_...:85-92 GEMV: B is K x 1, output M x 1
    a, x = ints(rng, (11, 37)), ints(rng, (37, 1))
    add("p04_gemv", A=a, B=x, C=a @ x)
    # kernels/6_...:131-134 large K
    a, b = ints(rng, (3, 4097)), ints(rng, (4097, 2))
    add("p06_large_k", A=a, B=b, C=a @ b)
    # kernels/7_...:81-85 small K
    a, b = ints(rng, (8, 2)), ints(rng, (2, 9))
    add("p07_small_k", A=a, B=b, C=a @ b)
    # kernels/9_...:146-148 tall-skinny: A M x N, B N x M, C M x M
    a, b = ints(rng, (12, 3)), ints(rng, (3, 12))
    add("p09_tall_skinny", A=a, B=b, C=a @ b)
    # kernels/10_...:181-186 3-D tensor x matrix
    a, b = ints(rng, (2, 5, 7)), ints(rng, (7, 4))
    add("p10_tensor3d", A=a, B=b, C=np.einsum("nmk,kl->nml", a, b))
    # kernels/11_...:136-146,165 4-D tensor x matrix
    a, b = ints(rng, (2, 3, 2, 5)), ints(rng, (5, 4))
    add("p11_tensor4d", A=a, B=b, C=np.einsum("bijl,lk->bijk", a, b))
    # kernels/12_...:46-54 diag(a) . B
    d, b = ints(rng, (6,)), ints(rng, (6, 7))
    add("p12_diag", A=d, B=b, C=d[:, None] * b)
    # kernels/13_...:135-136 symmetric
    r1, r2 = ints(rng, (8, 8)), ints(rng, (8, 8))
    s1, s2 = r1 + r1.T, r2 + r2.T
    add("p13_symmetric", A=s1, B=s2, C=s1 @ s2)
    # kernels/14_...:57,74-75,84-85,123-128 upper triangular
    u1, u2 = np.triu(ints(rng, (10, 10))), np.triu(ints(rng, (10, 10)))
    add("p14_upper", A=u1, B=u2, C=np.triu(u1 @ u2))
    # kernels/15_...:155-206 lower triangular
    l1, l2 = np.tril(ints(rng, (10, 10))), np.tril(ints(rng, (10, 10)))
    add("p15_lower", A=l1, B=l2, C=np.tril(l1 @ l2))
    # kernels/16_...:127-132 A stored K x M
    a, b = ints(rng, (6, 4)), ints(rng, (6, 5))
    add("p16_transposed_a", A=a, B=b, C=a.T @ b)
    # kernels/17_...:268-272 B stored N x K
    a, b = ints(rng, (4, 6)), ints(rng, (5, 6))
    add("p17_transposed_b", A=a, B=b, C=a @ b.T)
    # kernels/18_...:156-160 both stored transposed
    a, b = ints(rng, (6, 4)), ints(rng, (5, 6))
    add("p18_transposed_both", A=a, B=b, C=a.T @ b.T)

    # kernels/5_...:47-71 matrix-scalar: C = A * s (B holds s); s = -5/2 keeps
    # every product exact, the expected value is (-5 * A) / 2 in int64 first
    a = ints(rng, (5, 7))
    add("p05_scalar", A=a, B=np.array([-2.5], dtype=np.float32),
        C=((-5 * a).astype(np.float64) / 2.0))

    # kernels/87_...:451-492 pointwise (1x1) convolution, with bias:
    # out[n,o,h,w] = sum_c weight[o,c] * input[n,c,h,w] + bias[o]
    x, w, bias = ints(rng, (2, 5, 3, 4)), ints(rng, (6, 5, 1, 1)), ints(rng, (6,))
    add("p87_pointwise", A=x, B=w, bias=bias,
        C=np.einsum("oc,nchw->nohw", w[:, :, 0, 0], x) + bias[None, :, None, None])

    np.savez_compressed(OUT, **cases)
    print(f"wrote {OUT}: {len(cases) // 3} cases")


if __name__ == "__main__":
    main()
