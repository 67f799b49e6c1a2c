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
//   3. O = 2^-14 (H.V + 2^-11 L.V)       fp16 MFMA over [H | L] . [V ; V]
//                                        (the B operand's key index wraps),
//                                        V read in place with LDS transpose
//                                        loads, fp32 accumulation, fp16 out
// For seq <= 512 steps 1 and 2 are one kernel (qk_softmax_kernel): a tile of
// 128 queries holds whole score rows, so S never leaves the accumulators.
// Step 3 is one contraction of depth 2*Sp whose accumulator is multiplied by
// 2^11 where the H half ends, so the attention weights keep ~22 bits
// (fp32-like) although the MFMA takes fp16.  The 2^14 and 2^11 scalings keep
// H and L in binary16's normal range: the MFMA treats subnormal fp16 inputs
// as zero, which unscaled would drop most of L and every weight below 2^-14.
// Products of fp16 values are exact in fp32, so every step except the final
// rounding to fp16 carries fp32-level error, as the reference's fp32 math does.
// QK is "NT" (both operands contiguous along the reduction): one ds_read_b128
// feeds one MFMA operand (8 halves per lane); in PV the key-major V operand
// takes two ds_read_b64_tr_b16 per MFMA operand.
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
// fp16 contraction: C[b] (M x N) = alpha * A[b] (M x K) . B[b]^T, with A
// row-major (lda) and B stored N x K row-major (ldb), or key-major K x N;
// K % 64 == 0 and 16-byte aligned rows (lda, ldb multiples of 8).  Output
// fp32 (OUT_HALF = false) or fp16.
// ---------------------------------------------------------------------------
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
    int b_rows;           // key-major B (hgemm_direct_kernel<*, true>): valid key rows
    int64_t lda, ldb, ldc;
    int64_t sa, sb, sc;   // batch strides (elements)
    float alpha;
};

// ---------------------------------------------------------------------------
// Key-major fp16 operand (V of the PV contraction: keys x E, E contiguous),
// staged directly and read with the gfx950 LDS transpose load.  A slice is
// 64 key rows of 256 columns; wave instruction m (1 KiB) holds keys m (lanes
// 0-31) and m + 32 (lanes 32-63) in an LDS slot of 1088 bytes, so key k sits
// at slot k % 32, half k / 32.  ds_read_b64_tr_b16 works on groups of 16
// lanes: if lane j of a group points at the 4 halves x[j][0..3], lane i
// receives x[4 e + i / 4][i % 4] for e = 0..3 (measured on MI355X with an
// in-bounds probe).  So when lane j points at key kb + j / 4, column n0 +
// 4 (j % 4), lane i gets keys kb..kb+3 of column n0 + i -- a quarter of the
// MFMA operand the key-contiguous layout gives with one 16-byte read; two
// such reads make the 8 halves k = 16 ks + 8 (lane / 32) .. + 7 of column
// c0 + lane % 32.  The four key rows of one read sit in consecutive slots,
// 1088 = 4 * 256 + 64 bytes apart, i.e. in four different 64-byte windows
// of the 256-byte bank space: conflict-free.
// ---------------------------------------------------------------------------
typedef short s4v __attribute__((ext_vector_type(4)));

struct KeyLoader {
    static constexpr int ROWS = 256, BKH = 64, NW = 8;
    static constexpr int SLOT = 272;  // floats per instruction slot (1088 bytes)
    static constexpr int INSTR = BKH / 2, PER_WAVE = INSTR / NW;
    static constexpr int ELEMS = INSTR * SLOT;

    __device__ __forceinline__ static constexpr int byte_of(int key, int col) {
        return (key % 32) * (SLOT * 4) + (key / 32) * 512 + col * 2;
    }
    // Byte offsets (from the slice origin) of this wave's loads for the tile
    // at column n0; keys at or past krows (a slice that runs past the last
    // key) read key krows - 1 instead, whose weights are zero.
    __device__ __forceinline__ static void offsets(int64_t ld, int n0, int n_ext, int wave, int lane,
                                                   uint32_t (&vo)[PER_WAVE], int krows = BKH) {
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
            const int ins = wave * PER_WAVE + i;
            int key = ins + 32 * (lane >> 5);
            key = key < krows ? key : krows - 1;
            // (n_ext - n0 is a positive multiple of 8: E % 64 == 0)
            const int c0 = (lane & 31) * 8;
            const int c = n0 + c0 + 7 < n_ext ? c0 : n_ext - 8 - n0;
            vo[i] = ((uint32_t)key * (uint32_t)ld + (uint32_t)c) * 2u;
        }
    }
    __device__ __forceinline__ static void load(const _Float16* base, int64_t ld, int n0, int k0,
                                                const uint32_t (&vo)[PER_WAVE], float* lds,
                                                int wave) {
        const __amdgpu_buffer_rsrc_t rsrc =
            raw_rsrc(reinterpret_cast<const float*>(base + (int64_t)k0 * ld + n0));
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
            const int ins = wave * PER_WAVE + i;
            load_lds16(rsrc, vo[i], lds + ins * SLOT);
        }
    }
    // MFMA operand of k-step ks for the 32 columns at c0
    __device__ __forceinline__ static h8 frag(const float* lds, int c0, int ks, int lane) {
        const int g = lane >> 4, i = lane & 15;
        const char* base = reinterpret_cast<const char*>(lds);
        h8 out;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int key = 16 * ks + 8 * (g >> 1) + 4 * hh + (i >> 2);
            const int col = c0 + 16 * (g & 1) + 4 * (i & 3);
            const s4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s4v*)(base + byte_of(key, col)));
            const h4 hv = __builtin_bit_cast(h4, v);
#pragma unroll
            for (int e = 0; e < 4; ++e) out[4 * hh + e] = hv[e];
        }
        return out;
    }
};

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
// (An earlier 128 x 128 tile with 64 x 64 wave tiles needed 2 KiB of fragment
// reads per MFMA; the LDS read rate set its pace, ~20 % of the MFMA peak.)
// ---------------------------------------------------------------------------
template <bool OUT_HALF, bool B_KEYS>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
    hgemm_direct_kernel(const HgemmParams p, int batch) {
    constexpr int BM = 256, BN = 256, WM = 128, WN = 64, TM = 4, TN = 2, BKH = 64;
    using L = DirectLoader<true, 8>;
    // B_KEYS: B is key-major (K x N, N contiguous; ldb per key row), staged by
    // KeyLoader and read with transpose loads
    using LB = std::conditional_t<B_KEYS, KeyLoader, L>;
    __shared__ __attribute__((aligned(16))) float sA0[L::ELEMS];
    __shared__ __attribute__((aligned(16))) float sA1[L::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB0[LB::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB1[LB::ELEMS];

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

    uint32_t voA[L::PER_WAVE], voB[LB::PER_WAVE];
    auto set_offsets = [&](const Work& w) __attribute__((always_inline)) {
        L::offsets(lda, w.tm * BM, p.M, wave, lane, voA);
        if constexpr (B_KEYS)
            KeyLoader::offsets(p.ldb, w.tn * BN, p.N, wave, lane, voB);
        else
            L::offsets(ldb, w.tn * BN, p.N, wave, lane, voB);
    };
    auto issue = [&](const Work& w, int it, float* dA, float* dB) __attribute__((always_inline)) {
        const int k0 = it * BKH;
        const int kb = (p.b_kwrap > 0 && k0 >= p.b_kwrap) ? k0 - p.b_kwrap : k0;
        const float* A = reinterpret_cast<const float*>(p.A + (int64_t)w.b * p.sa);
        L::load(A, lda, w.tm * BM, k0 / 2, voA, dA, wave);
        if constexpr (B_KEYS) {
            const _Float16* B = p.B + (int64_t)w.b * p.sb;
            if (kb + BKH > p.b_rows) {  // slice runs past the last key: clamped offsets
                uint32_t tB[KeyLoader::PER_WAVE];
                KeyLoader::offsets(p.ldb, w.tn * BN, p.N, wave, lane, tB, p.b_rows - kb);
                KeyLoader::load(B, p.ldb, w.tn * BN, kb, tB, dB, wave);
            } else {
                KeyLoader::load(B, p.ldb, w.tn * BN, kb, voB, dB, wave);
            }
        } else {
            const float* B = reinterpret_cast<const float*>(p.B + (int64_t)w.b * p.sb);
            L::load(B, ldb, w.tn * BN, kb / 2, voB, dB, wave);
        }
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
            if constexpr (B_KEYS) {
                fb[ks & 1][j] = KeyLoader::frag(Bs, wn * WN + j * 32, ks, lane);
            } else {
                float t[4];
                L::frag(Bs, wn * WN + j * 32, ks, lane, t);
                fb[ks & 1][j] = __builtin_bit_cast(h8, f4{t[0], t[1], t[2], t[3]});
            }
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
// QK with the row softmax fused in, for sp <= 512: one tile is 128 queries x
// all 512 (padded) keys, so every score row is complete in the accumulators.
// 8 waves (2 x 4) of 64 x 128 (2 x 4 blocks); Q and K staged directly in
// 64-half slices (two stages of 16 + 64 KiB).  The epilogue computes the row
// max and the sum of exp over keys < n (lane, lane ^ 32, then the four key
// waves through LDS -- the stage just consumed is free by then) and writes the
// P' row [H | L] (2 * sp halves) with 2^14 p = H + 2^-11 L, as
// softmax_split_kernel does, without the fp32 score round trip.
// ---------------------------------------------------------------------------
struct QkSoftmaxParams {
    const _Float16* Q;
    const _Float16* K;
    _Float16* P;
    int n, sp, E;
    int64_t head_elems;  // Q / K elements per head (n * E)
    float scale;         // 1 / sqrt(E)
};

__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
    qk_softmax_kernel(const QkSoftmaxParams p, int heads) {
    // a 128-query x 512-key tile (BN = 512 keys: the loader shape below)
    constexpr int BM = 128, WM = 64, WN = 128, TM = 2, TN = 4, BKH = 64;
    using LA = DirectLoader<true, 8, BM, 32>;
    using LB = DirectLoader<true, 8, 512, 32>;
    __shared__ __attribute__((aligned(16))) float sA0[LA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sA1[LA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB0[LB::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB1[LB::ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const int per_b = (p.n + BM - 1) / BM;
    const int total = per_b * heads;
    const int nk = p.E / BKH;
    const int64_t ld = p.E / 2;  // floats

    struct Work {
        int b, tm;
    };
    auto decode = [&](int t) {
        const int id = xcd_remap(t, total);
        return Work{id / per_b, id % per_b};
    };
    uint32_t voA[LA::PER_WAVE], voB[LB::PER_WAVE];
    auto set_offsets = [&](const Work& w) __attribute__((always_inline)) {
        LA::offsets(ld, w.tm * BM, p.n, wave, lane, voA);
        LB::offsets(ld, 0, p.n, wave, lane, voB);  // key rows past n read row n - 1
    };
    auto issue = [&](const Work& w, int it, float* dA, float* dB) __attribute__((always_inline)) {
        const int k0 = it * BKH;
        const float* A = reinterpret_cast<const float*>(p.Q + (int64_t)w.b * p.head_elems);
        const float* B = reinterpret_cast<const float*>(p.K + (int64_t)w.b * p.head_elems);
        LA::load(A, ld, w.tm * BM, k0 / 2, voA, dA, wave);
        LB::load(B, ld, 0, k0 / 2, voB, dB, wave);
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
            LA::frag(As, wm * WM + i * 32, ks, lane, t);
            fa[ks & 1][i] = __builtin_bit_cast(h8, f4{t[0], t[1], t[2], t[3]});
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            float t[4];
            LB::frag(Bs, wn * WN + j * 32, ks, lane, t);
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
    // Epilogue.  Lane l holds, for query row 32 i + l % 32 of the wave, the
    // keys wn * 128 + 32 j + 8 g + 4 (l / 32) + e (register 4 g + e of block
    // j).  red: [2 wm][4 wn][64 rows] floats for the max, then for the sum.
    auto softmax_store = [&](const Work& w, float* red) __attribute__((always_inline)) {
        const int h = lane >> 5, l32 = lane & 31;
        float sm[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float m = -INFINITY;
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = wn * WN + 32 * j + 8 * (r >> 2) + 4 * h + (r & 3);
                    const float v = key < p.n ? acc[i][j][r] * p.scale : -INFINITY;
                    acc[i][j][r] = v;
                    m = fmaxf(m, v);
                }
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            if (h == 0) red[(wm * 4 + wn) * 64 + 32 * i + l32] = m;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float m = -INFINITY;
#pragma unroll
            for (int q = 0; q < 4; ++q) m = fmaxf(m, red[(wm * 4 + q) * 64 + 32 * i + l32]);
            float ssum = 0.f;
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e = expf(acc[i][j][r] - m);  // exp(-inf) = 0 past n
                    acc[i][j][r] = e;
                    ssum += e;
                }
            ssum += __shfl_xor(ssum, 32, 64);
            if (h == 0) red[512 + (wm * 4 + wn) * 64 + 32 * i + l32] = ssum;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float ssum = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) ssum += red[512 + (wm * 4 + q) * 64 + 32 * i + l32];
            sm[i] = 16384.0f / ssum;
        }
        __syncthreads();  // red is overwritten by the next slice's loads
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = w.tm * BM + wm * WM + 32 * i + l32;
            if (row >= p.n) continue;
            _Float16* out = p.P + ((int64_t)w.b * p.n + row) * (2 * (int64_t)p.sp);
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int key = wn * WN + 32 * j + 8 * g + 4 * h;
                    if (key >= p.sp) continue;
                    h4 hi, lo;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float pv = acc[i][j][4 * g + e] * sm[i];  // 2^14 p <= 2^14
                        // pv opaque: otherwise the compiler rounds the exact
                        // product to fp16 once (v_fma_mixlo) for L's H but
                        // stores H rounded via fp32, which differ at fp16 ties
                        asm volatile("" : "+v"(pv));
                        hi[e] = (_Float16)pv;
                        lo[e] = (_Float16)((pv - (float)hi[e]) * 2048.0f);
                    }
                    *reinterpret_cast<h4*>(out + key) = hi;
                    *reinterpret_cast<h4*>(out + p.sp + key) = lo;
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
        float* const red = CB == 0 ? sB0 : sB1;  // free once this slice is consumed
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
        compute(curA, curB, [&]() __attribute__((always_inline)) { issue(nw, nit, nxtA, nxtB); });
        __syncthreads();
        if (!last) {
            ++it;
            return false;
        }
        softmax_store(cur, red);
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
        float pv = e * scale;  // 2^14 p <= 2^14
        // H and the H inside L must be one rounding of one fp32 value: opaque
        // pv keeps the compiler from folding the product into either of them
        asm volatile("" : "+v"(pv));
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
// Host side: one chunk of heads at a time through the caller's workspace.
// ---------------------------------------------------------------------------
namespace {

int round_up(int x, int m) { return (x + m - 1) / m * m; }
// keys per half of a P' row: whole 64-deep slices, so the switch from
// the H half to the L half falls between slices
constexpr int kSdpaKeyPad = 64;

// The 256-tile direct kernel, persistent over (batch, tile): one workgroup per
// CU (its LDS holds two 64-deep slices of both operands).  Byte offsets within
// a slice fit 32 bits for lda, ldb < 2^22 halves; the C entry point's limits
// (seq <= 32768, embed <= 65536) keep every leading dimension far below.
template <bool OUT_HALF, bool B_KEYS = false>
hipError_t launch_hgemm_direct(HgemmParams p, int batch, hipStream_t s) {
    if (p.lda >= (INT64_C(1) << 22) || p.ldb >= (INT64_C(1) << 22)) return hipErrorInvalidValue;
    p.tiles_n = (p.N + 255) / 256;
    const int total = ((p.M + 255) / 256) * p.tiles_n * batch;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
    }
    const int grid = total < cus ? total : cus;
    hipLaunchKernelGGL((hgemm_direct_kernel<OUT_HALF, B_KEYS>), dim3((unsigned)grid), dim3(512), 0, s,
                       p, batch);
    return hipGetLastError();
}

hipError_t launch_qk_softmax(const QkSoftmaxParams& p, int heads, hipStream_t s) {
    const int total = ((p.n + 127) / 128) * heads;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
    }
    const int grid = total < cus ? total : cus;
    hipLaunchKernelGGL(qk_softmax_kernel, dim3((unsigned)grid), dim3(512), 0, s, p, heads);
    return hipGetLastError();
}

}  // namespace

int64_t sdpa_chunk_heads(int64_t heads) { return heads < kSdpaChunkHeads ? heads : kSdpaChunkHeads; }

// seq <= 512: the QK kernel writes P' straight from its accumulators, no S
bool sdpa_fused(int sp, int embed) { return sp <= 512 && embed < (1 << 22); }

size_t sdpa_workspace_bytes(int64_t heads, int seq, int embed) {
    if (heads <= 0 || seq <= 0 || embed <= 0) return 0;
    const int64_t hc = sdpa_chunk_heads(heads);
    const int64_t sp = round_up(seq, kSdpaKeyPad);
    // V is read in place
    const int64_t s_bytes = sdpa_fused((int)sp, embed) ? 0 : seq * sp * 4;  // S (fp32)
    return (size_t)hc * (s_bytes + seq * 2 * sp * 2);                      // + P' (fp16)
}

hipError_t launch_sdpa(const _Float16* Q, const _Float16* K, const _Float16* V, _Float16* O,
                       int64_t heads, int seq, int embed, void* ws, hipStream_t s) {
    const int sp = round_up(seq, kSdpaKeyPad);
    const int64_t hc_max = sdpa_chunk_heads(heads);
    const bool fused = sdpa_fused(sp, embed);
    float* S = static_cast<float*>(ws);
    _Float16* P = fused ? static_cast<_Float16*>(ws) : reinterpret_cast<_Float16*>(S + hc_max * seq * sp);
    const int64_t head_elems = (int64_t)seq * embed;
    const float scale = 1.0f / sqrtf((float)embed);
    for (int64_t h0 = 0; h0 < heads; h0 += hc_max) {
        const int hc = (int)(heads - h0 < hc_max ? heads - h0 : hc_max);
        hipError_t e;
        if (fused) {
            // 1+2. P' straight from the scores (one tile holds whole rows)
            QkSoftmaxParams f{};
            f.Q = Q + h0 * head_elems;
            f.K = K + h0 * head_elems;
            f.P = P;
            f.n = seq;
            f.sp = sp;
            f.E = embed;
            f.head_elems = head_elems;
            f.scale = scale;
            if ((e = launch_qk_softmax(f, hc, s)) != hipSuccess) return e;
        } else {
            // 1. S = scale * Q K^T (seq x seq, row stride sp)
            HgemmParams q{};
            q.A = Q + h0 * head_elems;
            q.B = K + h0 * head_elems;
            q.C = S;
            q.M = seq;
            q.N = seq;
            q.K = embed;
            q.n_store = sp;
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
            e = launch_hgemm_direct<false>(q, hc, s);
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
        }
        // 3. O = P' . [V ; V] (seq x E, fp16): the B operand's key index wraps
        // at sp (keys sp .. 2 sp - 1 read keys 0 .. sp - 1 again); keys past
        // seq carry zero weights
        HgemmParams o{};
        o.A = P;
        o.C = O + h0 * head_elems;
        o.M = seq;
        o.N = embed;
        o.K = 2 * sp;
        o.n_store = embed;
        o.lda = 2 * sp;
        o.b_kwrap = sp;
        o.ldc = embed;
        o.sa = (int64_t)seq * 2 * sp;
        o.sc = head_elems;
        o.B = V + h0 * head_elems;  // key-major V itself
        o.ldb = embed;
        o.sb = head_elems;
        o.b_rows = seq;
        o.k_switch = sp / 64;          // first 64-deep slice of the L half
        o.switch_mul = 2048.0f;        // 2^11: H.V -> 2^11 H.V, then + L.V
        o.alpha = 1.0f / (16384.0f * 2048.0f);  // 2^-25
        if ((e = launch_hgemm_direct<true, true>(o, hc, s)) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace mi
