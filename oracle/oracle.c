/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the mathematics of the reference's GEMM-family operators
 * (champloo2878/cuPilot-Kernels, kernels/1..18 except 5), accumulated in fp64.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker.  The product path never calls it.
 *
 * The reference computes in fp16/bf16/tf32 on tensor cores; the operators it
 * stands for are exact real-number contractions, so the oracle restates the
 * operator, not the reference's rounding.  Each function cites the reference
 * wrapper whose shape logic it follows:
 *
 *   orc_gemm_f64      C[b] = op(A[b]) . op(B[b])  (dense / batched / transposed)
 *                     kernels/1_...:190, 2_...:122-124, 3_...:126-131,
 *                     6_...:131-134, 7_...:81-85, 8_...:156-160, 9_...:146-148,
 *                     10_...:181-186, 11_...:136-146, 13_...:135-136,
 *                     16_...:127-132 (A stored KxM), 17_...:268-272 (B stored NxK),
 *                     18_...:156-160 (both)
 *   orc_gemm_f64 with structure LOWER / UPPER
 *                     tril(tril(A).tril(B)) -- kernels/15_...:155-206 (k-range
 *                     [bx,by], zero store above the diagonal);
 *                     triu(triu(A).triu(B)) -- kernels/14_...:57,74-75,84-85 (input
 *                     masks), 123-128 (masked store)
 *   orc_gemv_f64      y = A.x -- kernels/4_...:84-92 (B is Kx1, output Mx1)
 *   orc_diag_f32      out[i,j] = a[i]*B[i,j] -- kernels/12_...:43-62 (one fp32
 *                     multiply per element, so bitwise-exact)
 *   orc_scale_f32     C[i] = A[i]*s -- kernels/5_...:10-42 (kernel: float4 body
 *                     at :24-35, scalar tail at :36-40), :47-71 (wrapper: C is
 *                     empty_like(A), n = A.numel()); one fp32 multiply per element
 *   orc_pointwise_conv_f64
 *                     out[n][o][p] = sum_c w[o][c]*x[n][c][p] + bias[o] --
 *                     kernels/87_...:451-492 (wrapper: output N x Cout x H x W,
 *                     weight indexed out_c * in_channels + c at :308,:321, bias
 *                     optional at :452) and :373-388 (bias added once after the
 *                     channel sum)
 *   orc_half_to_double / orc_sdpa_f64
 *                     out = softmax(q.k^T * scale) . v per head, in fp64 from
 *                     binary16 inputs -- kernels/97_...:256-296 (wrapper: Q, K, V
 *                     batch x heads x seq x embed fp16, scale 1/sqrt(embed)
 *                     at :275, output empty_like(Q)) and :136-250 (scores, row
 *                     softmax with max subtraction, weighted sum of V rows)
 *   orc_matvec_f64 / orc_checksums_f32
 *                     fp64 y = A.v of a strided fp32 matrix, and fp64 row / column
 *                     checksums C.v, u^T.C of an fp32 output block: the
 *                     whole-output (Freivalds) checks of the full-size tests
 *                     compare C.v with A.(B.v) and u^T.C with (u^T.A).B.
 *   orc_fill_uniform_f32 / orc_fill_int_f32
 *                     counter-based splitmix64 input generator shared with the
 *                     device fill kernel, so any element can be regenerated on
 *                     the host without copying a multi-GiB operand back.
 *
 * Pins (tests/test_oracle.py): published splitmix64 vectors, committed integer
 * fixtures (exact), numpy float64 matmul (independent implementation),
 * identity/permutation/all-ones/rank-1 closed forms, brute force on tiny shapes,
 * planted-mistake checks (transposed operand, dropped term, wrong triangle).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_EXPORT __attribute__((visibility("default")))

/* ---- generator -------------------------------------------------------- */

/* splitmix64 output function (S. Vigna, public domain algorithm): the value
 * the sequential generator returns for state x. */
ORC_EXPORT uint64_t orc_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* Element i of stream `seed`: x = splitmix64((seed << 40) + i);
 * v = float(x >> 40) * 2^-23 - 1, exact in fp32, uniform on [-1, 1 - 2^-23]. */
ORC_EXPORT void orc_fill_uniform_f32(float* out, int64_t n, uint64_t seed, int64_t offset) {
    const uint64_t base = (seed << 40) + (uint64_t)offset;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint64_t z = orc_splitmix64(base + (uint64_t)i);
        out[i] = (float)(z >> 40) * 0x1p-23f - 1.0f;
    }
}

/* Integer-valued variant: v = lo + (x >> 32) % (hi - lo + 1). */
ORC_EXPORT void orc_fill_int_f32(float* out, int64_t n, uint64_t seed, int64_t offset,
                                 int32_t lo, int32_t hi) {
    const uint64_t base = (seed << 40) + (uint64_t)offset;
    const uint64_t span = (uint64_t)(hi - lo + 1);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint64_t z = orc_splitmix64(base + (uint64_t)i);
        out[i] = (float)(lo + (int64_t)((z >> 32) % span));
    }
}

/* ---- dense / structured contraction ------------------------------------ */

enum { ORC_DENSE = 0, ORC_LOWER = 1, ORC_UPPER = 2 };

/* Element (r, c) of a logical matrix held with row stride rs and column
 * stride cs (the transposed layouts are just swapped strides). */
static inline double at2(const float* p, int64_t r, int64_t c, int64_t rs, int64_t cs) {
    return (double)p[r * rs + c * cs];
}

/*
 * C[b][i][j] = sum_k opA[b][i][k] * opB[b][k][j], fp64 accumulation, written
 * as double.  Logical opA is MxK with element (i,k) at A[b*sa + i*a_rs + k*a_cs];
 * logical opB is KxN with (k,j) at B[b*sb + k*b_rs + j*b_cs]; C is dense
 * batch x M x N (row-major).
 * structure LOWER: inputs masked to their lower triangles, output to its
 *   lower triangle (exact zeros above); UPPER symmetric.  Square only.
 * rows: if non-NULL, only rows rows[0..nrows) of every batch are produced and
 *   C is batch x nrows x N.
 */
ORC_EXPORT void orc_gemm_f64(const float* A, const float* B, double* C,
                             int64_t batch, int64_t M, int64_t N, int64_t K,
                             int64_t sa, int64_t a_rs, int64_t a_cs,
                             int64_t sb, int64_t b_rs, int64_t b_cs,
                             int32_t structure, const int64_t* rows, int64_t nrows) {
    const int64_t R = rows ? nrows : M;
    for (int64_t b = 0; b < batch; ++b) {
        const float* Ab = A + b * sa;
        const float* Bb = B + b * sb;
        /* opB materialised as a dense KxN double panel so the inner loop is unit stride */
        double* Bd = (double*)malloc((size_t)(K * N > 0 ? K * N : 1) * sizeof(double));
#pragma omp parallel for schedule(static)
        for (int64_t k = 0; k < K; ++k) {
            for (int64_t j = 0; j < N; ++j) {
                double v = at2(Bb, k, j, b_rs, b_cs);
                if (structure == ORC_LOWER && k < j) v = 0.0;
                if (structure == ORC_UPPER && k > j) v = 0.0;
                Bd[k * N + j] = v;
            }
        }
        double* Cb = C + b * R * N;
#pragma omp parallel for schedule(dynamic, 4)
        for (int64_t r = 0; r < R; ++r) {
            const int64_t i = rows ? rows[r] : r;
            double* crow = Cb + r * N;
            for (int64_t j = 0; j < N; ++j) crow[j] = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                double a = at2(Ab, i, k, a_rs, a_cs);
                if (structure == ORC_LOWER && k > i) a = 0.0;
                if (structure == ORC_UPPER && k < i) a = 0.0;
                if (a == 0.0) continue;
                const double* brow = Bd + k * N;
                for (int64_t j = 0; j < N; ++j) crow[j] += a * brow[j];
            }
            if (structure == ORC_LOWER)
                for (int64_t j = i + 1; j < N; ++j) crow[j] = 0.0;
            if (structure == ORC_UPPER)
                for (int64_t j = 0; j < i && j < N; ++j) crow[j] = 0.0;
        }
        free(Bd);
    }
}

/* Sparse sampling: out[t] = sum_k opA[b_t][i_t][k] * opB[b_t][k][j_t] for the
 * listed (b, i, j) triples; used at full BASELINE sizes where a dense fp64
 * reference would not fit the test budget. Dense structure only. */
ORC_EXPORT void orc_gemm_entries_f64(const float* A, const float* B, double* out,
                                     const int64_t* bij, int64_t count, int64_t K,
                                     int64_t sa, int64_t a_rs, int64_t a_cs,
                                     int64_t sb, int64_t b_rs, int64_t b_cs) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < count; ++t) {
        const int64_t b = bij[3 * t], i = bij[3 * t + 1], j = bij[3 * t + 2];
        const float* Ab = A + b * sa;
        const float* Bb = B + b * sb;
        double s = 0.0;
        for (int64_t k = 0; k < K; ++k) s += at2(Ab, i, k, a_rs, a_cs) * at2(Bb, k, j, b_rs, b_cs);
        out[t] = s;
    }
}

/* y[i] = sum_k A[i*lda + k] * x[k] for the listed rows (all rows if rows == NULL). */
ORC_EXPORT void orc_gemv_f64(const float* A, const float* x, double* y, int64_t M, int64_t K,
                             int64_t lda, const int64_t* rows, int64_t nrows) {
    const int64_t R = rows ? nrows : M;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < R; ++r) {
        const int64_t i = rows ? rows[r] : r;
        const float* a = A + i * lda;
        double s = 0.0;
        for (int64_t k = 0; k < K; ++k) s += (double)a[k] * (double)x[k];
        y[r] = s;
    }
}

/* GEMV over a generated A: row i of A is stream seed_a at offset i*K, so an
 * 8 GiB operand can be checked row by row without holding it. */
ORC_EXPORT void orc_gemv_generated_f64(uint64_t seed_a, const float* x, double* y, int64_t K,
                                       const int64_t* rows, int64_t nrows) {
#pragma omp parallel
    {
        float* buf = (float*)malloc((size_t)K * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < nrows; ++r) {
            const uint64_t base = (seed_a << 40) + (uint64_t)(rows[r] * K);
            for (int64_t k = 0; k < K; ++k) {
                uint64_t z = orc_splitmix64(base + (uint64_t)k);
                buf[k] = (float)(z >> 40) * 0x1p-23f - 1.0f;
            }
            double s = 0.0;
            for (int64_t k = 0; k < K; ++k) s += (double)buf[k] * (double)x[k];
            y[r] = s;
        }
        free(buf);
    }
}

/* out[i*M + j] = a[i] * B[i*M + j] in fp32: a single rounding, so the device
 * result must match bitwise. */
ORC_EXPORT void orc_diag_f32(const float* a, const float* B, float* out, int64_t N, int64_t M) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; ++i)
        for (int64_t j = 0; j < M; ++j) out[i * M + j] = a[i] * B[i * M + j];
}

ORC_EXPORT void orc_scale_f32(const float* A, float* C, int64_t n, float s) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) C[i] = A[i] * s;
}

ORC_EXPORT void orc_pointwise_conv_f64(const float* x, const float* w, const float* bias,
                                       double* out, int64_t n, int64_t cin, int64_t cout,
                                       int64_t hw) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < n; ++b)
        for (int64_t o = 0; o < cout; ++o) {
            double* dst = out + (b * cout + o) * hw;
            for (int64_t p = 0; p < hw; ++p) dst[p] = 0.0;
            for (int64_t c = 0; c < cin; ++c) {
                const double wv = (double)w[o * cin + c];
                const float* src = x + (b * cin + c) * hw;
                for (int64_t p = 0; p < hw; ++p) dst[p] += wv * (double)src[p];
            }
            if (bias)
                for (int64_t p = 0; p < hw; ++p) dst[p] += (double)bias[o];
        }
}

/* IEEE binary16 bit pattern -> double (normal, subnormal, zero, inf, NaN). */
ORC_EXPORT double orc_half_to_double(uint16_t h) {
    const int sign = h >> 15, exp = (h >> 10) & 0x1F, frac = h & 0x3FF;
    double v;
    if (exp == 0) v = ldexp((double)frac, -24);
    else if (exp == 31) v = frac ? NAN : INFINITY;
    else v = ldexp((double)(frac | 0x400), exp - 25);
    return sign ? -v : v;
}

ORC_EXPORT void orc_sdpa_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, double* out,
                             int64_t heads, int64_t seq, int64_t embed, double scale) {
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
    for (int64_t h = 0; h < heads; ++h)
        for (int64_t i = 0; i < seq; ++i) {
            const uint16_t* qi = q + (h * seq + i) * embed;
            double* s = (double*)malloc((size_t)seq * sizeof(double));
            double mx = -INFINITY;
            for (int64_t j = 0; j < seq; ++j) {
                const uint16_t* kj = k + (h * seq + j) * embed;
                double d = 0.0;
                for (int64_t e = 0; e < embed; ++e) d += orc_half_to_double(qi[e]) * orc_half_to_double(kj[e]);
                s[j] = d * scale;
                if (s[j] > mx) mx = s[j];
            }
            double sum = 0.0;
            for (int64_t j = 0; j < seq; ++j) {
                s[j] = exp(s[j] - mx);
                sum += s[j];
            }
            double* o = out + (h * seq + i) * embed;
            for (int64_t e = 0; e < embed; ++e) o[e] = 0.0;
            for (int64_t j = 0; j < seq; ++j) {
                const double w = s[j] / sum;
                const uint16_t* vj = v + (h * seq + j) * embed;
                for (int64_t e = 0; e < embed; ++e) o[e] += w * orc_half_to_double(vj[e]);
            }
            free(s);
        }
}

/* y[r] = sum_c A(r, c) * v[c] in fp64, A(r, c) = A[r * rs + c * cs]: a
 * strided fp32 matrix (a transposed view is the same data with rs and cs
 * swapped).  Used for the whole-output checksums of the full-size tests:
 * A.(B.v) needs two of these, O(MK + KN) instead of the O(MNK) product. */
ORC_EXPORT void orc_matvec_f64(const float* A, int64_t rows, int64_t cols, int64_t rs, int64_t cs,
                               const double* v, double* y) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        double s = 0.0;
        const float* a = A + r * rs;
        for (int64_t c = 0; c < cols; ++c) s += (double)a[c * cs] * v[c];
        y[r] = s;
    }
}

/* Row and column checksums of an fp32 block C (rows x cols, row stride ldc),
 * in fp64: cv[r] = sum_c C[r][c] * v[c] (written) and utc[c] += sum_r u[r] *
 * C[r][c] (accumulated, so a large output can be reduced block by block).
 * Every element of the block enters both. */
ORC_EXPORT void orc_checksums_f32(const float* C, int64_t rows, int64_t cols, int64_t ldc,
                                  const double* v, const double* u, double* cv, double* utc) {
#pragma omp parallel
    {
        double* acc = (double*)calloc((size_t)cols, sizeof(double));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const float* c = C + r * ldc;
            const double ur = u[r];
            double s = 0.0;
            for (int64_t j = 0; j < cols; ++j) {
                const double x = (double)c[j];
                s += x * v[j];
                acc[j] += ur * x;
            }
            cv[r] = s;
        }
#pragma omp critical
        for (int64_t j = 0; j < cols; ++j) utc[j] += acc[j];
        free(acc);
    }
}

/* max_t |got[t] - ref[t]| over n elements (fp32 result vs fp64 reference). */
ORC_EXPORT double orc_max_abs_diff(const float* got, const double* ref, int64_t n) {
    double m = 0.0;
#pragma omp parallel for reduction(max : m)
    for (int64_t t = 0; t < n; ++t) {
        double d = fabs((double)got[t] - ref[t]);
        if (d != d) d = INFINITY; /* NaN counts as failure */
        if (d > m) m = d;
    }
    return m;
}

ORC_EXPORT int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
