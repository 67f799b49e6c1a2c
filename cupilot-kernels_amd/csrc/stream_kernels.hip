// stream_kernels.hip -- HBM-bound kernels of the GEMM family on gfx950, plus
// the split-K reduction and the fills.
//
//   gemv_kernel    y = A.x (kernels/4_Matrix_vector_multiplication_best_kernel.cu:6-80
//                  is the reference's version).  Every wave owns ROWS rows and
//                  walks K with 16-byte non-temporal loads of A (A is read
//                  exactly once, so it should not evict x from L2; plain
//                  loads measured 13 % slower); each x float4 it loads is
//                  used for all ROWS rows, cutting the x traffic to 1/ROWS of
//                  A's.  The per-lane partial sums are
//                  reduced across the wave with xor shuffles at the end.
//                  Optional split over K writes per-split partial sums that a
//                  second pass adds in fixed order.
//   diag_kernel    out[i,j] = a[i] * B[i,j]
//                  (kernels/12_Matmul_with_diagonal_matrices_best_kernel.cu:9-38):
//                  a pure 16-byte streaming copy-scale, one row per iteration.
//   scale_kernel   C[i] = A[i] * s over a flat array
//                  (kernels/5_Matrix_scalar_multiplication_best_kernel.cu:10-42):
//                  the same stream over fixed 32 KiB chunks of the array.
//   splitk_reduce  C = sum over splits of the partial tiles, in split order.
//   fill kernels   zero fill and the counter-based uniform generator.
#include <type_traits>

#include "mi_device.hpp"
#include "mi_internal.hpp"

namespace mi {

// ---------------------------------------------------------------------------
// GEMV
// ---------------------------------------------------------------------------
constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / 64;

template <int ROWS, int UNROLL, bool VEC>
__global__ void __launch_bounds__(kGemvThreads)
    gemv_kernel(const float* __restrict__ A, const float* __restrict__ x, float* __restrict__ y,
                float* __restrict__ ws, int M, int K, int64_t lda, int k_chunk, int split_k) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kGemvWaves + wave) * ROWS;
    if (row0 >= M) return;
    const int split = blockIdx.y;
    const int kb = split * k_chunk;
    const int ke = min(K, kb + k_chunk);
    const int nrows = min(ROWS, M - row0);

    const float* arow[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) arow[r] = A + (int64_t)(row0 + min(r, nrows - 1)) * lda;

    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.f;

    if (VEC) {
        constexpr int STEP = 64 * 4 * UNROLL;  // floats per wave iteration
        // Full iterations cover [kb, full_end): every load is in range, so all
        // UNROLL*ROWS loads of an iteration can be in flight together.
        const int full_end = ke > kb ? kb + ((ke - kb) / STEP) * STEP : kb;
        int k = kb + lane * 4;
        for (; k < full_end; k += STEP) {
            f4 xv[UNROLL];
            f4 av[UNROLL][ROWS];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                xv[u] = *reinterpret_cast<const f4*>(x + k + u * 256);
#pragma unroll
                for (int r = 0; r < ROWS; ++r)
                    av[u][r] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(arow[r] + k + u * 256));
            }
            // all UNROLL * ROWS loads are issued before the first FMA waits on
            // one (left to itself the scheduler may pair each load with its
            // FMAs, which serialises the loads on their latency)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    acc[r] = fmaf(av[u][r][0], xv[u][0], acc[r]);
                    acc[r] = fmaf(av[u][r][1], xv[u][1], acc[r]);
                    acc[r] = fmaf(av[u][r][2], xv[u][2], acc[r]);
                    acc[r] = fmaf(av[u][r][3], xv[u][3], acc[r]);
                }
        }
        // Remainder, 256 floats per step (K is a multiple of 4 here).
        for (; k < ke; k += 256) {
            const f4 xv = *reinterpret_cast<const f4*>(x + k);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const f4 av = __builtin_nontemporal_load(reinterpret_cast<const f4*>(arow[r] + k));
                acc[r] = fmaf(av[0], xv[0], acc[r]);
                acc[r] = fmaf(av[1], xv[1], acc[r]);
                acc[r] = fmaf(av[2], xv[2], acc[r]);
                acc[r] = fmaf(av[3], xv[3], acc[r]);
            }
        }
    } else {
        for (int k = kb + lane; k < ke; k += 64) {
            const float xv = x[k];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] = fmaf(arow[r][k], xv, acc[r]);
        }
    }

#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        float v = acc[r];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[r] = v;
    }
    if (lane == 0) {
        float* out = split_k > 1 ? ws + (int64_t)split * M : y;
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            if (r < nrows) out[row0 + r] = acc[r];
    }
}

__global__ void gemv_reduce_kernel(const float* __restrict__ ws, float* __restrict__ y, int M,
                                   int split_k) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= M) return;
    float s = 0.f;
    for (int t = 0; t < split_k; ++t) s += ws[(int64_t)t * M + i];
    y[i] = s;
}

constexpr int kGemvUnroll = 2;

GemvPlan gemv_plan(int64_t M, int64_t K, bool aligned) {
    GemvPlan p;
    // Rows per wave: each x float4 a wave loads serves all its rows, so more
    // rows mean less x traffic; measured on MI355X at 32768 x 65536 with
    // 16-byte non-temporal A loads: 16 rows 7.04 TB/s, 8 rows 6.89 TB/s,
    // 4 rows 6.87 TB/s (2 and 1 rows lose to the x re-reads).  Fewer rows for
    // smaller M keep >= 2048 waves in flight.
    const int rows = M >= 16 * 2048 ? 16 : M >= 8 * 2048 ? 8 : 4;
    p.rows_per_wg = kGemvWaves * rows;
    p.vec = aligned ? 4 : 1;
    const int64_t wgs = (M + p.rows_per_wg - 1) / p.rows_per_wg;
    // Split K only when the rows alone give fewer than 2 workgroups per CU
    // (256 CUs) and each split still streams >= 16 KiB per row: measured on
    // MI355X, A = 32768 x 65536 streams at 6.46 TB/s unsplit (4 workgroups per
    // CU) and 5.85 TB/s split in two.
    int split = 1;
    while (wgs * split < 512 && K / (split * 2) >= 4096) split *= 2;
    p.split_k = split;
    int64_t chunk = (K + split - 1) / split;
    chunk = (chunk + 255) / 256 * 256;
    p.k_chunk = (int)chunk;
    p.ws_bytes = split > 1 ? (size_t)split * (size_t)M * sizeof(float) : 0;
    return p;
}

hipError_t launch_gemv(const GemvPlan& p, const float* A, const float* x, float* y, float* ws,
                       int M, int K, int64_t lda, hipStream_t s) {
    const int wgs = (M + p.rows_per_wg - 1) / p.rows_per_wg;
    dim3 grid(wgs, p.split_k);
    const int rows = p.rows_per_wg / kGemvWaves;
#define MI_GEMV_LAUNCH(R, V)                                                                      \
    hipLaunchKernelGGL((gemv_kernel<R, kGemvUnroll, V>), grid, dim3(kGemvThreads), 0, s, A, x, y, \
                       ws, M, K, lda, p.k_chunk, p.split_k)
    if (p.vec == 4) {
        if (rows == 16) MI_GEMV_LAUNCH(16, true);
        else if (rows == 8) MI_GEMV_LAUNCH(8, true);
        else MI_GEMV_LAUNCH(4, true);
    } else {
        if (rows == 16) MI_GEMV_LAUNCH(16, false);
        else if (rows == 8) MI_GEMV_LAUNCH(8, false);
        else MI_GEMV_LAUNCH(4, false);
    }
#undef MI_GEMV_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.split_k == 1) return e;
    hipLaunchKernelGGL(gemv_reduce_kernel, dim3((M + 255) / 256), dim3(256), 0, s, ws, y, M, p.split_k);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// diag(a) . B
// ---------------------------------------------------------------------------
constexpr int kDiagThreads = 256;

template <bool VEC>
__global__ void __launch_bounds__(kDiagThreads)
    diag_kernel(const float* __restrict__ a, const float* __restrict__ B, float* __restrict__ out,
                int64_t N, int64_t M) {
    for (int64_t i = blockIdx.x; i < N; i += gridDim.x) {
        const float s = a[i];
        const float* src = B + i * M;
        float* dst = out + i * M;
        if (VEC) {
            const int64_t m4 = M / 4;
            const f4* s4 = reinterpret_cast<const f4*>(src);
            f4* d4 = reinterpret_cast<f4*>(dst);
            // 8 independent 16-byte loads in flight per thread before the
            // stores, then a remainder loop
            constexpr int U = 8;
            int64_t c = threadIdx.x;
            for (; c + (U - 1) * kDiagThreads < m4; c += U * kDiagThreads) {
                f4 v[U];
#pragma unroll
                for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(s4 + c + u * kDiagThreads);
#pragma unroll
                for (int u = 0; u < U; ++u) __builtin_nontemporal_store(v[u] * s, d4 + c + u * kDiagThreads);
            }
            for (; c < m4; c += kDiagThreads)
                __builtin_nontemporal_store(__builtin_nontemporal_load(s4 + c) * s, d4 + c);
        } else {
            for (int64_t c = threadIdx.x; c < M; c += kDiagThreads)
                __builtin_nontemporal_store(__builtin_nontemporal_load(src + c) * s, dst + c);
        }
    }
}

hipError_t launch_diag(const float* a, const float* B, float* out, int64_t N, int64_t M,
                       hipStream_t s) {
    const bool vec = (M % 4 == 0) && ((uintptr_t)B % 16 == 0) && ((uintptr_t)out % 16 == 0);
    const int64_t grid = N < 65536 ? N : 65536;
    if (vec)
        hipLaunchKernelGGL((diag_kernel<true>), dim3((unsigned)grid), dim3(kDiagThreads), 0, s, a, B, out, N, M);
    else
        hipLaunchKernelGGL((diag_kernel<false>), dim3((unsigned)grid), dim3(kDiagThreads), 0, s, a, B, out, N, M);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// C = s * A over a flat array
// ---------------------------------------------------------------------------
constexpr int kScaleThreads = 256;
constexpr int kScaleUnroll = 8;  // 16-byte loads in flight per thread
constexpr int64_t kScaleChunk = (int64_t)kScaleUnroll * kScaleThreads;  // float4s per chunk

// Workgroup b streams chunks b, b + grid, ... of kScaleChunk float4s: all 8
// loads of a thread are issued before its 8 stores.  The one partial chunk at
// the end of the float4 range belongs to exactly one workgroup, which finishes
// it element by element; workgroup 0 also does the last n % 4 floats.
template <bool VEC>
__global__ void __launch_bounds__(kScaleThreads)
    scale_kernel(const float* __restrict__ A, float* __restrict__ C, float s, int64_t n) {
    if (VEC) {
        const int64_t n4 = n / 4;
        const f4* a4 = reinterpret_cast<const f4*>(A);
        f4* c4 = reinterpret_cast<f4*>(C);
        int64_t base = (int64_t)blockIdx.x * kScaleChunk;
        for (; base + kScaleChunk <= n4; base += (int64_t)gridDim.x * kScaleChunk) {
            f4 v[kScaleUnroll];
#pragma unroll
            for (int u = 0; u < kScaleUnroll; ++u)
                v[u] = __builtin_nontemporal_load(a4 + base + threadIdx.x + u * kScaleThreads);
#pragma unroll
            for (int u = 0; u < kScaleUnroll; ++u)
                __builtin_nontemporal_store(v[u] * s, c4 + base + threadIdx.x + u * kScaleThreads);
        }
        for (int64_t i = base + threadIdx.x; i < n4; i += kScaleThreads) c4[i] = a4[i] * s;
        const int64_t tail = n - n4 * 4;
        if (blockIdx.x == 0 && threadIdx.x < tail) C[n4 * 4 + threadIdx.x] = A[n4 * 4 + threadIdx.x] * s;
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kScaleThreads + threadIdx.x; i < n;
             i += (int64_t)gridDim.x * kScaleThreads)
            C[i] = A[i] * s;
    }
}

hipError_t launch_scale(const float* A, float* C, int64_t n, float s, hipStream_t st) {
    const bool vec = ((uintptr_t)A % 16 == 0) && ((uintptr_t)C % 16 == 0);
    if (vec) {
        int64_t grid = (n / 4 + kScaleChunk - 1) / kScaleChunk;
        grid = grid < 1 ? 1 : (grid > 65536 ? 65536 : grid);
        hipLaunchKernelGGL((scale_kernel<true>), dim3((unsigned)grid), dim3(kScaleThreads), 0, st, A, C, s, n);
    } else {
        int64_t grid = (n + kScaleThreads - 1) / kScaleThreads;
        grid = grid > 65536 ? 65536 : grid;
        hipLaunchKernelGGL((scale_kernel<false>), dim3((unsigned)grid), dim3(kScaleThreads), 0, st, A, C, s, n);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// split-K reduction and fills
// ---------------------------------------------------------------------------
// Each output element's split_k partials are summed by kReduceGroups threads,
// each over a fixed contiguous range of splits (sequentially, 4 loads in
// flight), and the group sums are added in group order: a fixed partition and
// order, so the result is the same on every call.  32 elements (VEC: 32
// float4s) per workgroup of 256 threads.
constexpr int kReduceGroups = 8;

template <bool VEC>
__global__ void __launch_bounds__(256)
    splitk_reduce_kernel(const float* __restrict__ ws, float* __restrict__ C, int M, int N, int split_k,
                         int64_t ldc, int64_t sc, int64_t split_stride, const float* __restrict__ bias) {
    using V = typename std::conditional<VEC, f4, float>::type;
    constexpr int W = VEC ? 4 : 1;
    __shared__ V part[kReduceGroups][32];
    const int64_t per_batch = (int64_t)M * N;
    const int lane32 = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int64_t q = (int64_t)blockIdx.x * 32 + lane32;  // element (VEC: float4) index
    const int b = blockIdx.y;
    const bool live = q * W < per_batch;
    V acc = V{};
    if (live) {
        const V* src = reinterpret_cast<const V*>(ws + (int64_t)b * per_batch) + q;
        const int64_t stride = split_stride / W;
        const int t0 = (int)((int64_t)g * split_k / kReduceGroups);
        const int t1 = (int)((int64_t)(g + 1) * split_k / kReduceGroups);
        int t = t0;
        for (; t + 4 <= t1; t += 4) {
            V v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = src[(int64_t)(t + u) * stride];
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += v[u];
        }
        for (; t < t1; ++t) acc += src[(int64_t)t * stride];
    }
    part[g][lane32] = acc;
    __syncthreads();
    if (g != 0 || !live) return;
    V s = part[0][lane32];
#pragma unroll
    for (int h = 1; h < kReduceGroups; ++h) s += part[h][lane32];
    const int64_t e = q * W;
    const int64_t row = e / N, col = e % N;
    if (bias) s += bias[row];
    float* dst = C + (int64_t)b * sc + row * ldc + col;
    if constexpr (VEC) *reinterpret_cast<f4*>(dst) = s;
    else *dst = s;
}

hipError_t launch_splitk_reduce(const float* ws, float* C, int M, int N, int batch, int split_k,
                                int64_t ldc, int64_t sc, const float* bias, hipStream_t s) {
    const int64_t per_batch = (int64_t)M * N;
    const bool vec = N % 4 == 0 && ldc % 4 == 0 && sc % 4 == 0 && ((uintptr_t)C & 15u) == 0 &&
                     ((uintptr_t)ws & 15u) == 0;
    const int64_t items = vec ? per_batch / 4 : per_batch;
    dim3 grid((unsigned)((items + 31) / 32), (unsigned)batch);
    if (vec)
        hipLaunchKernelGGL((splitk_reduce_kernel<true>), grid, dim3(256), 0, s, ws, C, M, N, split_k, ldc,
                           sc, per_batch * batch, bias);
    else
        hipLaunchKernelGGL((splitk_reduce_kernel<false>), grid, dim3(256), 0, s, ws, C, M, N, split_k,
                           ldc, sc, per_batch * batch, bias);
    return hipGetLastError();
}

// Stream-K fixup: one workgroup per (stream-K tile, band of rows).  The tile's
// head segment (k from 0) is already in C; its other segments sit in their
// workspace slots (tile-local, bm x bn) and are added in slot order, i.e. in
// k order -- a fixed order, so the result is the same on every call.  A slot
// whose workgroup had an empty range (contiguous ranges only) holds nothing
// and is skipped.  The schedule (SkSched, by value) is the launch's.
struct SkSched {
    int n_dp, S, ipt, G, nph;
    SkPhase ph[kSkMaxPhases];
};

template <bool VEC>
__global__ void __launch_bounds__(256)
    sk_fixup_kernel(float* __restrict__ C, const float* __restrict__ ws, int64_t ldc, int M, int N,
                    int bm, int bn, int tiles_m, int tiles_n, int group_m, const SkSched sc,
                    int band_rows) {
    const int t = blockIdx.x;
    int64_t first, count;
    sk_tile_slots(t, sc.S, sc.ipt, sc.G, sc.ph, sc.nph, first, count);
    if (count == 0) return;
    const int n_dp = sc.n_dp;
    int tm, tn;
    raster(n_dp + t, tiles_m, tiles_n, group_m, tm, tn);
    constexpr int W = VEC ? 4 : 1;
    const int per_row = bn / W;
    const int r0 = (int)blockIdx.y * band_rows;
    const int64_t slot_elems = (int64_t)bm * bn;
    for (int e = threadIdx.x; e < band_rows * per_row; e += 256) {
        const int r = r0 + e / per_row, c = (e % per_row) * W;
        const int row = tm * bm + r, col = tn * bn + c;
        if (row >= M || col >= N) continue;
        float* const dst = C + (int64_t)row * ldc + col;
        const float* const src = ws + (int64_t)r * bn + c;
        if constexpr (VEC) {
            f4 v = *reinterpret_cast<const f4*>(dst);
            for (int64_t q = 0; q < count; ++q) {
                const int64_t slot = first + q;
                if (!sk_slot_used(slot, sc.S, sc.ipt, sc.G, sc.nph)) continue;
                v += *reinterpret_cast<const f4*>(src + slot * slot_elems);
            }
            *reinterpret_cast<f4*>(dst) = v;
        } else {
            float v = *dst;
            for (int64_t q = 0; q < count; ++q) {
                const int64_t slot = first + q;
                if (!sk_slot_used(slot, sc.S, sc.ipt, sc.G, sc.nph)) continue;
                v += src[slot * slot_elems];
            }
            *dst = v;
        }
    }
}

hipError_t launch_sk_fixup(const GemmLaunch& g, hipStream_t s) {
    const CfgInfo ci = cfg_info(g.cfg);
    const int band_rows = 4096 / ci.bn;  // 4096 floats of C per workgroup
    const dim3 grid((unsigned)g.sk_tiles, (unsigned)(ci.bm / band_rows));
    const bool vec = g.N % 4 == 0 && g.ldc % 4 == 0 && ((uintptr_t)g.C & 15u) == 0 &&
                     ((uintptr_t)g.ws & 15u) == 0;
    SkSched sc;
    sc.n_dp = g.sk_dp;
    sc.S = g.sk_tiles;
    sc.ipt = g.sk_ipt;
    sc.G = g.grid_x;
    sc.nph = g.sk_nph;
    for (int q = 0; q < kSkMaxPhases; ++q) sc.ph[q] = g.sk_ph[q];
    if (vec)
        hipLaunchKernelGGL(sk_fixup_kernel<true>, grid, dim3(256), 0, s, g.C, g.ws, g.ldc, g.M, g.N,
                           ci.bm, ci.bn, g.tiles_m, g.tiles_n, g.group_m, sc, band_rows);
    else
        hipLaunchKernelGGL(sk_fixup_kernel<false>, grid, dim3(256), 0, s, g.C, g.ws, g.ldc, g.M, g.N,
                           ci.bm, ci.bn, g.tiles_m, g.tiles_n, g.group_m, sc, band_rows);
    return hipGetLastError();
}

__global__ void fill_zero_kernel(float* __restrict__ C, int64_t rows, int64_t cols, int64_t ld,
                                 int64_t batch_stride, const float* __restrict__ bias) {
    const int64_t per = rows * cols;
    const int64_t b = blockIdx.y;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / cols, c = e % cols;
        C[b * batch_stride + r * ld + c] = bias ? bias[r] : 0.f;
    }
}

hipError_t launch_fill_zero_2d(float* C, int64_t rows, int64_t cols, int64_t ld, int64_t batch,
                               int64_t batch_stride, hipStream_t s, const float* bias) {
    const int64_t per = rows * cols;
    if (per == 0 || batch == 0) return hipSuccess;
    int64_t blocks = (per + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks, (unsigned)batch), dim3(256), 0, s, C,
                       rows, cols, ld, batch_stride, bias);
    return hipGetLastError();
}

// One workgroup per (zero-triangle tile, quarter of its 256 rows).  Zero
// tile (a, b) is the mirror of compute tile (b, a); when that tile was longer
// than cap K units its second chunk's partial sum sits here and is added to
// the first chunk's result (one fixed-order fp32 add).
template <bool VEC>
__global__ void __launch_bounds__(256)
    tri_finish_kernel(float* __restrict__ C, int64_t ldc, int nt, int cap, int lower, int zeroed) {
    int a, b;
    tri_tile(nt * (nt + 1) / 2 + (int)blockIdx.x, nt, lower != 0, a, b);
    const bool add = (a > b ? a - b : b - a) + 1 > cap;
    // zeroed: the main kernel wrote every zero tile but the mirrors and the
    // item counter's tile (zero-triangle tile 0, (0, 1) / (1, 0))
    if (zeroed && !add && blockIdx.x != 0) return;
    // 16 rows of the tile per workgroup, four 16-byte groups per thread, all
    // of a thread's loads issued before its stores (one memory round trip
    // per workgroup instead of one per group: the mirror and its tile never
    // overlap, but the compiler cannot know that and would not reorder them)
    const int64_t row0 = (int64_t)blockIdx.y * 16;
    float* const z0 = C + ((int64_t)a * 256 + row0) * ldc + (int64_t)b * 256;
    float* const d0 = C + ((int64_t)b * 256 + row0) * ldc + (int64_t)a * 256;
    if (VEC) {
        f4 zv[4], dv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = threadIdx.x + 256 * q, r = e >> 6, c = (e & 63) * 4;
            if (add) {
                zv[q] = *reinterpret_cast<const f4*>(z0 + (int64_t)r * ldc + c);
                dv[q] = *reinterpret_cast<const f4*>(d0 + (int64_t)r * ldc + c);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = threadIdx.x + 256 * q, r = e >> 6, c = (e & 63) * 4;
            if (add) *reinterpret_cast<f4*>(d0 + (int64_t)r * ldc + c) = dv[q] + zv[q];
            *reinterpret_cast<f4*>(z0 + (int64_t)r * ldc + c) = f4{0.f, 0.f, 0.f, 0.f};
        }
    } else {
        for (int e = threadIdx.x; e < 16 * 64; e += 256) {
            const int r = e >> 6, c = (e & 63) * 4;
            float* const z = z0 + (int64_t)r * ldc + c;
            float* const d = d0 + (int64_t)r * ldc + c;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (add) d[q] += z[q];
                z[q] = 0.f;
            }
        }
    }
}

hipError_t launch_tri_finish(float* C, int64_t ldc, int nt, int cap, bool lower, bool zeroed,
                             hipStream_t s) {
    const int zero_tiles = nt * (nt - 1) / 2;
    if (zero_tiles == 0) return hipSuccess;
    const dim3 grid((unsigned)zero_tiles, 16);
    if (ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(C) & 15u) == 0)
        hipLaunchKernelGGL(tri_finish_kernel<true>, grid, dim3(256), 0, s, C, ldc, nt, cap, (int)lower,
                           (int)zeroed);
    else
        hipLaunchKernelGGL(tri_finish_kernel<false>, grid, dim3(256), 0, s, C, ldc, nt, cap, (int)lower,
                           (int)zeroed);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Operand packing for the 16-byte staging path.  dst is R rows of kp floats
// (kp a multiple of 32, dst 16-byte aligned): dst[r][k] = src(r, k) for
// k < K and 0 for K <= k < kp.  K-contiguous sources, src(r, k) = src[r*ld + k],
// are copied row by row (each thread one 16-byte group of dst); MN-contiguous
// ones, src(r, k) = src[k*ld + r], are transposed through a 64 x 64 LDS tile
// so that both the reads (along r) and the writes (along k) are coalesced.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
    pack_rows_kernel(const float* __restrict__ src, int64_t ld, int64_t R, int K, float* __restrict__ dst,
                     int kp) {
    const int g4 = kp / 4;  // 16-byte groups per dst row
    const int64_t total = R * g4;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / g4;
        const int k = (int)(e - r * g4) * 4;
        const float* const row = src + r * ld;
        f4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = k + q < K ? row[k + q] : 0.f;
        *reinterpret_cast<f4*>(dst + r * kp + k) = v;
    }
}

__global__ void __launch_bounds__(256)
    pack_transpose_kernel(const float* __restrict__ src, int64_t ld, int64_t R, int K, float* __restrict__ dst,
                          int kp) {
    __shared__ float t[64][65];  // [k][r]
    const int64_t r0 = (int64_t)blockIdx.x * 64;
    const int k0 = blockIdx.y * 64;
    const int tid = threadIdx.x;
    // read: lane r = tid % 64 along the source's contiguous r, 16 k-rows each
    const int rr = tid & 63;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int kk = (tid >> 6) + 4 * i;
        const int64_t r = r0 + rr;
        const int k = k0 + kk;
        t[kk][rr] = (r < R && k < K) ? src[(int64_t)k * ld + r] : 0.f;
    }
    __syncthreads();
    // write: 64 rows x 16 groups of 4 k.  Each wave covers 4 rows: lanes
    // 8 q .. 8 q + 7 take groups 0-7 (lanes 32 + 8 q .. : 8-15) of row q, so
    // 8 lanes store 128 contiguous bytes and the LDS reads t[4 g + c][wr] of a
    // half-wave hit 32 distinct banks (with groups 0-15 of one row per 16
    // lanes, groups g and g + 8 shared a bank: 33 % of its LDS cycles were
    // conflict stalls)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid + 256 * i, lane = idx & 63;
        const int wr = 4 * (idx >> 6) + ((lane >> 3) & 3);
        const int g = (lane & 7) | (((lane >> 5) & 1) << 3);
        const int64_t r = r0 + wr;
        const int k = k0 + 4 * g;
        if (r < R && k < kp) {
            const f4 v = {t[4 * g][wr], t[4 * g + 1][wr], t[4 * g + 2][wr], t[4 * g + 3][wr]};
            *reinterpret_cast<f4*>(dst + r * kp + k) = v;
        }
    }
}

hipError_t launch_pack_rows(const float* src, int64_t ld, bool k_contig, int64_t R, int64_t K, float* dst,
                            int64_t kp, hipStream_t s) {
    if (R == 0 || kp == 0) return hipSuccess;
    if (k_contig) {
        int64_t blocks = (R * (kp / 4) + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(pack_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, ld, R, (int)K, dst,
                           (int)kp);
    } else {
        // (the planner packs only with kp / 64 <= 65535: grid.y's limit)
        const dim3 grid((unsigned)((R + 63) / 64), (unsigned)((kp + 63) / 64));
        hipLaunchKernelGGL(pack_transpose_kernel, grid, dim3(256), 0, s, src, ld, R, (int)K, dst, (int)kp);
    }
    return hipGetLastError();
}

__global__ void zero_word_kernel(int* w) {
    if (threadIdx.x == 0) *w = 0;
}

hipError_t launch_zero_word(void* w, hipStream_t s) {
    hipLaunchKernelGGL(zero_word_kernel, dim3(1), dim3(64), 0, s, static_cast<int*>(w));
    return hipGetLastError();
}

__global__ void fill_uniform_kernel(float* __restrict__ out, int64_t n, uint64_t base) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = uniform_from_bits(splitmix64(base + (uint64_t)i));
}

hipError_t launch_fill_uniform(float* out, int64_t n, uint64_t seed, int64_t offset, hipStream_t s) {
    if (n == 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 262144) blocks = 262144;
    hipLaunchKernelGGL(fill_uniform_kernel, dim3((unsigned)blocks), dim3(256), 0, s, out, n,
                       (seed << 40) + (uint64_t)offset);
    return hipGetLastError();
}

}  // namespace mi
