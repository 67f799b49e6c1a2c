// attention.hip -- scaled dot-product attention, fp16 in / fp16 out, for
// kernels/97_ScaledDotProductAttention_best_kernel.cu (reference kernel
// :136-250, wrapper :256-296): per (batch, head),
//     O = softmax(Q K^T / sqrt(E)) V,   Q, K, V, O: seq x E.
//
// MI355X design: attention with E = 1024 is two large contractions around a
// row softmax, so it runs as
//   1. S = (Q . K^T) / sqrt(E)           fp16 MFMA (v_mfma_f32_32x32x16_f16),
//                                        fp32 accumulation and output
//   2. P = softmax_rows(S)               fp32, written as two scaled fp16 terms
//                                        2^14 P = H + 2^-11 L, side by side
//   3. Vt = V^T                          E x Sp (zero padded to Sp keys)
//   4. O = 2^-14 (H.V + 2^-11 L.V)       fp16 MFMA over [H | L] . [Vt | Vt]^T
//                                        (the B operand wraps around Vt),
//                                        fp32 accumulation, fp16 out
// Step 4 is one contraction of depth 2*Sp whose accumulator is multiplied by
// 2^11 where the H half ends, so the attention weights keep ~22 bits
// (fp32-like) although the MFMA takes fp16.  The 2^14 and 2^11 scalings keep
// H and L in binary16's normal range: the MFMA treats subnormal fp16 inputs
// as zero, which unscaled would drop most of L and every weight below 2^-14.
// Products of fp16 values are exact in fp32, so every step except the final
// rounding to fp16 carries fp32-level error, as the reference's fp32 math does.
// Both contractions are "NT" (both operands contiguous along the reduction),
// so every operand fetch is a 16-byte row chunk: one ds_read_b128 feeds one
// MFMA operand (8 halves per lane).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "gemm_direct.hpp"
#include "mi_device.hpp"
#include "mi_internal.hpp"

namespace mi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// fp16 NT contraction: C[b] (M x N) = alpha * A[b] (M x K) . B[b]^T, with A
// row-major (lda) and B stored N x K row-major (ldb); K % 64 == 0 and 16-byte
// aligned rows (lda, ldb multiples of 8).  Output fp32 (OUT_HALF = false) or
// fp16.  128 x 128 tiles, 4 waves of 64 x 64 (2 x 2 blocks of 32 x 32), K in
// 64-deep slices through two LDS buffers (one barrier per slice, next slice's
// loads in flight during the MFMAs, as in the fp32 engine).
// ---------------------------------------------------------------------------
constexpr int kHgBM = 128, kHgBN = 128, kHgBK = 64, kHgThreads = 256;
constexpr int kHgLD = kHgBK + 8;  // halves per LDS row (+16 B: conflict-free b128 reads)

struct HgemmParams {
    const _Float16* A;
    const _Float16* B;
    void* C;
    int M, N, K;
    int n_store;          // columns that may be written (>= N; row padding of C)
    int tiles_n;
    int k_switch;         // slice index at which the accumulator is multiplied by switch_mul
    float switch_mul;
    int b_kwrap;          // > 0: B holds K / 2 columns, read twice (k -> k - b_kwrap past it)
    int64_t lda, ldb, ldc;
    int64_t sa, sb, sc;   // batch strides (elements)
    float alpha;
};

template <bool OUT_HALF>
__global__ void __launch_bounds__(kHgThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
    hgemm_nt_kernel(const HgemmParams p) {
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][kHgBM * kHgLD];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][kHgBN * kHgLD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31;
    const int tm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
    const int m0 = tm * kHgBM, n0 = tn * kHgBN;
    const _Float16* A = p.A + (int64_t)blockIdx.z * p.sa;
    const _Float16* B = p.B + (int64_t)blockIdx.z * p.sb;

    // 16-byte chunks: a tile is 128 rows x 8 chunks; 4 chunks per thread
    constexpr int NS = kHgBM * (kHgBK / 8) / kHgThreads;
    h8 ra[NS], rb[NS];
    auto load = [&](int k0) {
        const int kb0 = (p.b_kwrap > 0 && k0 >= p.b_kwrap) ? k0 - p.b_kwrap : k0;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int c = tid + s * kHgThreads;
            const int row = c >> 3, kc = (c & 7) * 8;
            const int am = m0 + row, bn = n0 + row;
            ra[s] = am < p.M ? *reinterpret_cast<const h8*>(A + (int64_t)am * p.lda + k0 + kc) : h8{};
            rb[s] = bn < p.N ? *reinterpret_cast<const h8*>(B + (int64_t)bn * p.ldb + kb0 + kc) : h8{};
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int c = tid + s * kHgThreads;
            const int row = c >> 3, kc = (c & 7) * 8;
            *reinterpret_cast<h8*>(&sA[buf][row * kHgLD + kc]) = ra[s];
            *reinterpret_cast<h8*>(&sB[buf][row * kHgLD + kc]) = rb[s];
        }
    };

    f16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = p.K / kHgBK;
    load(0);
    store(0);
    __syncthreads();
    for (int it = 0; it < nk; ++it) {
        const int cb = it & 1;
        if (it == p.k_switch) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] *= p.switch_mul;
        }
        // next slice's loads (the last iteration re-reads its own slice, unused)
        load((it + 1 < nk ? it + 1 : it) * kHgBK);
#pragma unroll
        for (int ks = 0; ks < kHgBK / 16; ++ks) {
            h8 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                fa[i] = *reinterpret_cast<const h8*>(
                    &sA[cb][(wm * 64 + i * 32 + l32) * kHgLD + ks * 16 + half * 8]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                fb[j] = *reinterpret_cast<const h8*>(
                    &sB[cb][(wn * 64 + j * 32 + l32) * kHgLD + ks * 16 + half * 8]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    // B fragment as the row operand: the block holds C^T, so
                    // lane l owns row l % 32 and 4 consecutive columns per
                    // register group
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[j], fa[i], acc[i][j], 0, 0, 0);
        }
        store(cb ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int row = m0 + wm * 64 + i * 32 + l32;
                const int col = n0 + wn * 64 + j * 32 + g * 8 + half * 4;
                if (row >= p.M || col + 3 >= p.n_store) continue;
                const int64_t off = (int64_t)blockIdx.z * p.sc + (int64_t)row * p.ldc + col;
                if (OUT_HALF) {
                    h4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = (_Float16)(acc[i][j][4 * g + e] * p.alpha);
                    *reinterpret_cast<h4*>(static_cast<_Float16*>(p.C) + off) = v;
                } else {
                    f4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e] * p.alpha;
                    *reinterpret_cast<f4*>(static_cast<float*>(p.C) + off) = v;
                }
            }
}

// ---------------------------------------------------------------------------
// The same NT contraction on 256 x 256 tiles with direct LDS staging, for
// the full-size shapes: 8 waves (2 x 4) of 128 x 64 (4 x 2 blocks), K in
// 64-half (128-byte) slices.  A 64-half row is 32 floats, so the fp32 direct
// loader stages both operands byte for byte (buffer_load_dwordx4 ... lds,
// [row][32 floats] with its chunk swizzle), and its fragment read -- 16 bytes
// of row r0 + lane % 32 at chunk 2 ks + lane / 32 -- is exactly the fp16
// MFMA's operand (8 halves: k = 16 ks + 8 (lane / 32) .. + 7).  Persistent
// over (batch, tile), XCD-remapped so the tiles of one batch entry share an
// L2; per slice: first fragment reads, the next slice's loads, then the
// MFMAs with the following k-step's reads issued ahead (as the fp32 kernel).
// With 64 x 64 wave tiles (hgemm_nt_kernel) every MFMA needed 2 KiB of
// fragment reads and the LDS read rate set the pace (~20 % of the MFMA peak).
// ---------------------------------------------------------------------------
template <bool OUT_HALF>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
    hgemm_direct_kernel(const HgemmParams p, int batch) {
    constexpr int BM = 256, BN = 256, WM = 128, WN = 64, TM = 4, TN = 2, BKH = 64;
    using L = DirectLoader<true, 8>;
    __shared__ __attribute__((aligned(16))) float sA0[L::ELEMS];
    __shared__ __attribute__((aligned(16))) float sA1[L::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB0[L::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB1[L::ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const int tiles_m = (p.M + BM - 1) / BM;
    const int per_b = tiles_m * p.tiles_n;
    const int total = per_b * batch;
    const int nk = p.K / BKH;
    const int64_t lda = p.lda / 2, ldb = p.ldb / 2;  // in floats

    struct Work {
        int b, tm, tn;
    };
    auto decode = [&](int t) {
        const int id = xcd_remap(t, total);
        Work w;
        w.b = id / per_b;
        const int r = id - w.b * per_b;
        w.tm = r / p.tiles_n;
        w.tn = r - w.tm * p.tiles_n;
        return w;
    };

    uint32_t voA[L::PER_WAVE], voB[L::PER_WAVE];
    auto set_offsets = [&](const Work& w) __attribute__((always_inline)) {
        L::offsets(lda, w.tm * BM, p.M, wave, lane, voA);
        L::offsets(ldb, w.tn * BN, p.N, wave, lane, voB);
    };
    auto issue = [&](const Work& w, int it, float* dA, float* dB) __attribute__((always_inline)) {
        const int k0 = it * BKH;
        const int kb = (p.b_kwrap > 0 && k0 >= p.b_kwrap) ? k0 - p.b_kwrap : k0;
        const float* A = reinterpret_cast<const float*>(p.A + (int64_t)w.b * p.sa);
        const float* B = reinterpret_cast<const float*>(p.B + (int64_t)w.b * p.sb);
        L::load(A, lda, w.tm * BM, k0 / 2, voA, dA, wave);
        L::load(B, ldb, w.tn * BN, kb / 2, voB, dB, wave);
    };

    f16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    h8 fa[2][TM], fb[2][TN];
    auto frags = [&](const float* As, const float* Bs, int ks) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float t[4];
            L::frag(As, wm * WM + i * 32, ks, lane, t);
            fa[ks & 1][i] = __builtin_bit_cast(h8, f4{t[0], t[1], t[2], t[3]});
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            float t[4];
            L::frag(Bs, wn * WN + j * 32, ks, lane, t);
            fb[ks & 1][j] = __builtin_bit_cast(h8, f4{t[0], t[1], t[2], t[3]});
        }
    };
    auto compute = [&](const float* As, const float* Bs, auto&& loads) __attribute__((always_inline)) {
        frags(As, Bs, 0);
        __builtin_amdgcn_sched_barrier(0);
        loads();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < BKH / 16; ++ks) {
            if (ks + 1 < BKH / 16) frags(As, Bs, ks + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    // B fragment as the row operand: the block holds C^T
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[ks & 1][j], fa[ks & 1][i],
                                                                       acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto store = [&](const Work& w) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = w.tm * BM + wm * WM + i * 32 + (lane & 31);
            if (row >= p.M) continue;
            const int64_t roff = (int64_t)w.b * p.sc + (int64_t)row * p.ldc;
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int col = w.tn * BN + wn * WN + j * 32 + g * 8 + (lane >> 5) * 4;
                    f4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e] * p.alpha;
                    if (OUT_HALF) {
                        _Float16* dst = static_cast<_Float16*>(p.C) + roff + col;
                        if (col + 3 < p.N) {
                            *reinterpret_cast<h4*>(dst) =
                                h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (col + e < p.N) dst[e] = (_Float16)v[e];
                        }
                    } else {
                        float* dst = static_cast<float*>(p.C) + roff + col;
                        if (col + 3 < p.N) {
                            *reinterpret_cast<f4*>(dst) = v;
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (col + e < p.N) dst[e] = v[e];
                        }
                    }
                }
        }
    };

    int t = blockIdx.x;
    if (t >= total) return;
    Work cur = decode(t);
    int it = 0;
    set_offsets(cur);
    issue(cur, 0, sA0, sB0);
    __syncthreads();
    auto slice = [&](auto cb_tag) __attribute__((always_inline)) -> bool {
        constexpr int CB = decltype(cb_tag)::value;
        const float* const curA = CB == 0 ? sA0 : sA1;
        const float* const curB = CB == 0 ? sB0 : sB1;
        float* const nxtA = CB == 0 ? sA1 : sA0;
        float* const nxtB = CB == 0 ? sB1 : sB0;
        const bool last = it + 1 >= nk;
        int nt = t;
        bool has_next = true;
        Work nw = cur;
        int nit = it + 1;
        if (last) {
            nt = t + gridDim.x;
            has_next = nt < total;
            nit = has_next ? 0 : it;
            if (has_next) {
                nw = decode(nt);
                set_offsets(nw);
            }
        }
        if (it == p.k_switch) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] *= p.switch_mul;
        }
        compute(curA, curB, [&]() __attribute__((always_inline)) { issue(nw, nit, nxtA, nxtB); });
        __syncthreads();
        if (!last) {
            ++it;
            return false;
        }
        store(cur);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
        if (!has_next) return true;
        t = nt;
        cur = nw;
        it = 0;
        return false;
    };
    for (;;) {
        if (slice(std::integral_constant<int, 0>{})) break;
        if (slice(std::integral_constant<int, 1>{})) break;
    }
}

// ---------------------------------------------------------------------------
// Row softmax with the two-term fp16 split.  One wave per row of S (n values,
// row stride lds floats); writes the P' row (2 * sp halves) [H | 0 pad | L | 0 pad]
// with 2^14 p = H + 2^-11 L.  Rows up to 64 * VPL values stay in registers
// (one read of S); longer rows take three passes over S.
// ---------------------------------------------------------------------------
template <int VPL>
__global__ void __launch_bounds__(256)
    softmax_split_kernel(const float* __restrict__ S, _Float16* __restrict__ P, int64_t rows, int n,
                         int sp, int64_t lds) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* s = S + row * lds;
    _Float16* out = P + row * (2 * (int64_t)sp);
    auto emit = [&](int c, float e, float scale) {
        const float pv = e * scale;  // 2^14 p <= 2^14
        const _Float16 hi = (_Float16)pv;
        out[c] = hi;
        out[sp + c] = (_Float16)((pv - (float)hi) * 2048.0f);
    };
    if (VPL > 0) {
        float x[VPL > 0 ? VPL : 1];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int c = lane + 64 * i;
            x[i] = c < n ? s[c] : -INFINITY;
            mx = fmaxf(mx, x[i]);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            x[i] = lane + 64 * i < n ? expf(x[i] - mx) : 0.f;
            sum += x[i];
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
        const float scale = 16384.0f / sum;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int c = lane + 64 * i;
            if (c < sp) emit(c, x[i], scale);
        }
        return;
    }
    float mx = -INFINITY;
    for (int c = lane; c < n; c += 64) mx = fmaxf(mx, s[c]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float sum = 0.f;
    for (int c = lane; c < n; c += 64) sum += expf(s[c] - mx);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float scale = 16384.0f / sum;
    for (int c = lane; c < sp; c += 64) emit(c, c < n ? expf(s[c] - mx) : 0.f, scale);
}

// ---------------------------------------------------------------------------
// Vt[b] (E x sp) = V[b]^T, zero for keys >= n.  64 x 64 tiles through LDS:
// 16-byte loads (8 halves along E) and 16-byte stores (8 halves along the
// keys), so both sides move whole 128-byte lines per 8 lanes; E % 8 == 0 and
// sp % 64 == 0 (16-byte aligned rows).  (Element-wise loads and stores ran at
// 2.5 TB/s.)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
    transpose_kernel(const _Float16* __restrict__ V, _Float16* __restrict__ Vt, int n, int E, int sp) {
    constexpr int LDH = 64 + 8;  // halves per LDS row (16-byte aligned rows)
    __shared__ __attribute__((aligned(16))) _Float16 tile[64 * LDH];
    const int b = blockIdx.z;
    const int k0 = blockIdx.y * 64, e0 = blockIdx.x * 64;
    const _Float16* v = V + (int64_t)b * n * E;
    _Float16* vt = Vt + (int64_t)b * E * (int64_t)sp;
    const int t = threadIdx.x;
    const int c = (t & 7) * 8;  // 8-half chunk within a 64-wide row
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const int r = pass * 32 + (t >> 3);  // key row of the tile
        const int k = k0 + r, e = e0 + c;
        h8 x = h8{};
        if (k < n && e < E) x = *reinterpret_cast<const h8*>(v + (int64_t)k * E + e);
        *reinterpret_cast<h8*>(&tile[r * LDH + c]) = x;
    }
    __syncthreads();
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const int r = pass * 32 + (t >> 3);  // E row of the output tile
        const int e = e0 + r, k = k0 + c;
        if (e >= E) continue;
        h8 y;
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = tile[(c + j) * LDH + r];
        *reinterpret_cast<h8*>(vt + (int64_t)e * sp + k) = y;
    }
}

// ---------------------------------------------------------------------------
// Host side: one chunk of heads at a time through the caller's workspace.
// ---------------------------------------------------------------------------
namespace {

int round_up(int x, int m) { return (x + m - 1) / m * m; }
// keys per half of a P' row (and per Vt row): whole 64-deep slices, so the switch from
// the H half to the L half falls between slices
constexpr int kSdpaKeyPad = 64;

template <bool OUT_HALF>
hipError_t launch_hgemm(const HgemmParams& p, int batch, hipStream_t s) {
    const int tiles_m = (p.M + kHgBM - 1) / kHgBM;
    dim3 grid((unsigned)(tiles_m * p.tiles_n), 1u, (unsigned)batch);
    hipLaunchKernelGGL((hgemm_nt_kernel<OUT_HALF>), grid, dim3(kHgThreads), 0, s, p);
    return hipGetLastError();
}

// The 256-tile direct kernel, persistent over (batch, tile): one workgroup per
// CU (its LDS holds two 64-deep slices of both 256-row operands).  p.tiles_n
// counts 256-wide tiles.  Byte offsets within a slice (256 rows) fit 32 bits
// for lda, ldb < 2^22 halves.
template <bool OUT_HALF>
hipError_t launch_hgemm_direct(HgemmParams p, int batch, hipStream_t s) {
    if (p.lda >= (INT64_C(1) << 22) || p.ldb >= (INT64_C(1) << 22))
        return launch_hgemm<OUT_HALF>(p, batch, s);
    p.tiles_n = (p.N + 255) / 256;
    const int total = ((p.M + 255) / 256) * p.tiles_n * batch;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
    }
    const int grid = total < cus ? total : cus;
    hipLaunchKernelGGL((hgemm_direct_kernel<OUT_HALF>), dim3((unsigned)grid), dim3(512), 0, s, p, batch);
    return hipGetLastError();
}

}  // namespace

int64_t sdpa_chunk_heads(int64_t heads) { return heads < kSdpaChunkHeads ? heads : kSdpaChunkHeads; }

size_t sdpa_workspace_bytes(int64_t heads, int seq, int embed) {
    if (heads <= 0 || seq <= 0 || embed <= 0) return 0;
    const int64_t hc = sdpa_chunk_heads(heads);
    const int64_t sp = round_up(seq, kSdpaKeyPad);
    return (size_t)hc * (seq * sp * 4       // S (fp32)
                         + seq * 2 * sp * 2  // P' (fp16)
                         + embed * sp * 2);     // Vt (fp16)
}

hipError_t launch_sdpa(const _Float16* Q, const _Float16* K, const _Float16* V, _Float16* O,
                       int64_t heads, int seq, int embed, void* ws, hipStream_t s) {
    const int sp = round_up(seq, kSdpaKeyPad);
    const int64_t hc_max = sdpa_chunk_heads(heads);
    float* S = static_cast<float*>(ws);
    _Float16* P = reinterpret_cast<_Float16*>(S + hc_max * seq * sp);
    _Float16* Vt = P + hc_max * seq * 2 * sp;
    const int64_t head_elems = (int64_t)seq * embed;
    const float scale = 1.0f / sqrtf((float)embed);
    for (int64_t h0 = 0; h0 < heads; h0 += hc_max) {
        const int hc = (int)(heads - h0 < hc_max ? heads - h0 : hc_max);
        // 1. S = scale * Q K^T (seq x seq, row stride sp)
        HgemmParams q{};
        q.A = Q + h0 * head_elems;
        q.B = K + h0 * head_elems;
        q.C = S;
        q.M = seq;
        q.N = seq;
        q.K = embed;
        q.n_store = sp;
        q.tiles_n = (seq + kHgBN - 1) / kHgBN;
        q.lda = embed;
        q.ldb = embed;
        q.ldc = sp;
        q.sa = head_elems;
        q.sb = head_elems;
        q.sc = (int64_t)seq * sp;
        q.alpha = scale;
        q.k_switch = -1;
        q.switch_mul = 1.0f;
        q.b_kwrap = 0;
        hipError_t e = launch_hgemm_direct<false>(q, hc, s);
        if (e != hipSuccess) return e;
        // 2. P' = split softmax rows
        const int64_t rows = (int64_t)hc * seq;
        const dim3 sm_grid((unsigned)((rows + 3) / 4));
        if (sp <= 512)
            hipLaunchKernelGGL((softmax_split_kernel<8>), sm_grid, dim3(256), 0, s, S, P, rows, seq, sp,
                               (int64_t)sp);
        else if (sp <= 1024)
            hipLaunchKernelGGL((softmax_split_kernel<16>), sm_grid, dim3(256), 0, s, S, P, rows, seq, sp,
                               (int64_t)sp);
        else
            hipLaunchKernelGGL((softmax_split_kernel<0>), sm_grid, dim3(256), 0, s, S, P, rows, seq, sp,
                               (int64_t)sp);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // 3. Vt = V^T
        hipLaunchKernelGGL(transpose_kernel,
                           dim3((unsigned)((embed + 63) / 64), (unsigned)((sp + 63) / 64), (unsigned)hc),
                           dim3(256), 0, s, V + h0 * head_elems, Vt, seq, embed, sp);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // 4. O = P' . [Vt | Vt]^T (seq x E, fp16): B wraps around Vt's sp columns
        HgemmParams o{};
        o.A = P;
        o.B = Vt;
        o.C = O + h0 * head_elems;
        o.M = seq;
        o.N = embed;
        o.K = 2 * sp;
        o.n_store = embed;
        o.tiles_n = (embed + kHgBN - 1) / kHgBN;
        o.lda = 2 * sp;
        o.ldb = sp;
        o.b_kwrap = sp;
        o.ldc = embed;
        o.sa = (int64_t)seq * 2 * sp;
        o.sb = (int64_t)embed * sp;
        o.sc = head_elems;
        o.k_switch = sp / kHgBK;       // first slice of the L half
        o.switch_mul = 2048.0f;        // 2^11: H.V -> 2^11 H.V, then + L.V
        o.alpha = 1.0f / (16384.0f * 2048.0f);  // 2^-25
        if ((e = launch_hgemm_direct<true>(o, hc, s)) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace mi
