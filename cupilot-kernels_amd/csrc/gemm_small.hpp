// gemm_small.hpp -- 64 x 64 output tiles for problems with few tiles
// (config kCfg64W): 1024^3 has 256 of them, one per CU, so the 128 and 256
// tiles can only fill the machine through split-K, whose partials cost a
// store burst and a reduction pass (two launches).  Here every workgroup
// reduces its tile's whole K range itself.
//
// Structure of one workgroup (8 waves, one workgroup per CU):
//   * K is walked in 64-deep slices staged straight into LDS (buffer_load
//     ... lds, DirectLoader's 64-row layouts) through a ring of four stage
//     buffers (A's slice, then B's, in each): the loads of slice i + 3 are
//     issued while slice i is computed, so each slice's loads have three slice
//     times (~2.5 us) to arrive from HBM -- every slice is new data for the
//     whole chip, since all workgroups walk K in step;
//   * wave w takes k-block w (k 8w .. 8w + 7) of every slice and the whole
//     64 x 64 tile (2 x 2 MFMA blocks, 16 v_mfma_f32_32x32x2_f32 per slice):
//     four independent accumulators per wave, one 16-byte fragment read per
//     MFMA;
//   * one barrier per slice: each wave first waits (vmcnt) for its own loads
//     of that slice only -- the two later slices stay in flight -- so after
//     the barrier the whole slice is in LDS;
//   * at the end the eight partial tiles go through LDS (two per stage
//     buffer, 16-byte chunks XOR-swizzled by row, conflict-free both ways) and are
//     added in wave order 0 .. 7, a fixed order, so results are deterministic.
// Persistent: workgroup b walks tiles b, b + grid, ... (XCD-aware raster),
// or its stream-K items.
#pragma once

#include "gemm_direct.hpp"

namespace mi {

// s_waitcnt that waits only for vmcnt <= N (gfx9 encoding: vmcnt in bits 3:0
// and 15:14; expcnt 6:4 and lgkmcnt 11:8 at their maxima, i.e. no wait).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt has 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// SK: the stream-K schedule (sk_item): workgroup b runs its items 0, 1, ...
// -- whole tiles, then its stream-K segments -- and stores a segment that
// does not start at k = 0 into that segment's workspace slot (64 x 64,
// tile-local) for sk_fixup to add in.
template <bool AT, bool BT, bool BIAS, bool SK = false>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
    gemm_f32_ksplit_kernel(const GemmParams p) {
    static_assert(!SK || !BIAS, "stream-K: no bias");
    constexpr int BM = 64, BK = 64, NW = 8;
    constexpr bool A_KC = !AT;  // A row-major (M x K) is contiguous along K
    constexpr bool B_KC = BT;   // B stored N x K is contiguous along K
    using LA = DirectLoader<A_KC, NW, BM, BK, 16>;
    using LB = DirectLoader<B_KC, NW, BM, BK, 16>;
    // per wave and slice: its loads of both operands (the vmcnt steps)
    constexpr int PER = LA::PER_WAVE + LB::PER_WAVE;
    // One object per stage, A's slice then B's: the compiler's wait
    // insertion tells the loads into one object from reads of another (it
    // tracks a handful of such objects; eight, one per operand and stage,
    // were too many: it waited for every load before reading stage 0).
    constexpr int SE = LA::ELEMS + LB::ELEMS;
    static_assert(SE >= 2 * BM * BM, "each stage buffer holds two waves' partial tiles");
    __shared__ __attribute__((aligned(16))) float st0[SE];
    __shared__ __attribute__((aligned(16))) float st1[SE];
    __shared__ __attribute__((aligned(16))) float st2[SE];
    __shared__ __attribute__((aligned(16))) float st3[SE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int l32 = lane & 31, half = lane >> 5;
    // wave-uniform, made scalar so LDS destinations (M0) need no readfirstlane
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int batch = blockIdx.z;
    const float* __restrict__ A = p.A + (int64_t)batch * p.sa;
    const float* __restrict__ B = p.B + (int64_t)batch * p.sb;
    float* C;
    int64_t ldc;
    if (p.split_k > 1) {
        C = p.ws + (int64_t)blockIdx.y * p.ws_split_stride + (int64_t)batch * p.ws_batch_stride;
        ldc = p.N;
    } else {
        C = p.C + (int64_t)batch * p.sc;
        ldc = p.ldc;
    }
    const bool c_vec = (ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(C) & 15u) == 0);

    // this wave's partial-tile buffer for the reduction, and the element
    // offset of 16-byte chunk c of tile row r in any of them
    float* const red = (wave < 4 ? (wave < 2 ? st0 : st1) : (wave < 6 ? st2 : st3)) + (wave & 1) * BM * BM;
    auto red_at = [](int r, int c) __attribute__((always_inline)) {
        return r * BM + ((c ^ (r & 15)) << 2);
    };

    uint32_t voA[LA::PER_WAVE], voB[LB::PER_WAVE];
    // stream-K: the current segment's workspace slot
    float* sk_slot = nullptr;
    for (int t = SK ? 0 : blockIdx.x;; t += SK ? 1 : gridDim.x) {
        int tm, tn, k_begin, k_end;
        bool to_slot = false;
        if constexpr (SK) {
            int lt, s0, s1;
            int64_t slot;
            if (!sk_item(blockIdx.x, t, gridDim.x, p.sk_dp, p.sk_tiles, p.sk_ipt, p.sk_ph, p.sk_nph,
                         lt, s0, s1, slot))
                break;
            raster(lt, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
            k_begin = s0 * BK;
            k_end = s1 * BK;
            to_slot = slot >= 0;
            if (to_slot) sk_slot = p.ws + slot * (BM * BM);
        } else {
            if (t >= p.num_tiles) break;
            tile_of<BM, BM, kDense>(p, t, p.num_tiles, blockIdx.y, tm, tn, k_begin, k_end);
        }
        // (the planner takes this config only with K and the split chunk
        // multiples of 64: every slice is full)
        const int ns = (k_end - k_begin) / BK;
        LA::offsets(p.lda, tm * BM, p.M, wave, lane, voA);
        LB::offsets(p.ldb, tn * BM, p.N, wave, lane, voB);
        auto issue = [&](int i, float* dA, float* dB) __attribute__((always_inline)) {
            const int k0 = k_begin + i * BK;
            LA::load(A, p.lda, tm * BM, k0, voA, dA, wave);
            LB::load(B, p.ldb, tn * BM, k0, voB, dB, wave);
        };

        f16v acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

        // Step j issues slice j into stage S = j % 4 (a compile-time buffer
        // name) and computes slice i = j - 3 from stage (S + 1) % 4.  Every
        // step issues the same loads on every path -- past the last slice it
        // loads the last slice again, into a stage no wave reads any more --
        // and every step from j = 3 on waits and meets at the barrier: the
        // compiler's own wait for a stage's loads is then vmcnt(12), already
        // met, where any path with fewer loads made it wait for all of them.
        // (Groups of four steps with no exit inside: an exit from the group
        // made the compiler move the accumulators between register sets.)
        auto step = [&](auto stage_tag, int j) __attribute__((always_inline)) {
            constexpr int S = decltype(stage_tag)::value;
            float* const dA = S == 0 ? st0 : S == 1 ? st1 : S == 2 ? st2 : st3;
            const float* const As = S == 0 ? st1 : S == 1 ? st2 : S == 2 ? st3 : st0;
            const float* const Bs = As + LA::ELEMS;
            const int i = j - 3;
            __builtin_amdgcn_sched_barrier(0);
            if (i >= 0) {
                // this wave's loads of slice i have landed (the two later
                // groups may not); then every wave's have, and every wave is
                // done with slice i - 1, whose stage the next loads overwrite
                wait_vmcnt<2 * PER>();
                __builtin_amdgcn_s_barrier();
            }
            __builtin_amdgcn_sched_barrier(0);
            issue(j < ns ? j : ns - 1, dA, dA + LA::ELEMS);
            __builtin_amdgcn_sched_barrier(0);
            if (i >= 0 && i < ns) {
                float fa[2][4], fb[2][4];
                if constexpr (A_KC) {
#pragma unroll
                    for (int m = 0; m < 2; ++m) LA::frag(As, 32 * m, wave, lane, fa[m]);
                } else {
                    LA::frag_pair(As, 0, wave, lane, fa);
                }
                if constexpr (B_KC) {
#pragma unroll
                    for (int n = 0; n < 2; ++n) LB::frag(Bs, 32 * n, wave, lane, fb[n]);
                } else {
                    LB::frag_pair(Bs, 0, wave, lane, fb);
                }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int m = 0; m < 2; ++m)
#pragma unroll
                        for (int n = 0; n < 2; ++n)
                            acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[n][s], fa[m][s],
                                                                             acc[m][n], 0, 0, 0);
            }
        };
        if (ns > 0) {
            for (int j = 0; j < ns + 3; j += 4) {
                step(std::integral_constant<int, 0>{}, j);
                step(std::integral_constant<int, 1>{}, j + 1);
                step(std::integral_constant<int, 2>{}, j + 2);
                step(std::integral_constant<int, 3>{}, j + 3);
            }
        }

        // Reduction.  Every wave is past its last fragment read (and its
        // loads: the barrier below waits for vmcnt 0) before any buffer is
        // reused.  Accumulator block (m, n) holds C^T: lane l is tile row
        // 32 m + l % 32 (A MN-contiguous, read in interleaved pairs: row
        // 2 (l % 32) + m); register 4 q + e is column 32 n + 8 q + 4 (l / 32)
        // + e (B MN-contiguous, pairs: columns 16 q + 8 (l / 32) + 2 e + n).
        __syncthreads();
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int row = A_KC ? 32 * m + l32 : 2 * l32 + m;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if constexpr (B_KC) {
#pragma unroll
                    for (int n = 0; n < 2; ++n) {
                        f4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = acc[m][n][4 * q + e];
                        *reinterpret_cast<f4*>(red + red_at(row, 8 * n + 2 * q + half)) = v;
                    }
                } else {
                    f4 lo, hi;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        lo[2 * e] = acc[m][0][4 * q + e];
                        lo[2 * e + 1] = acc[m][1][4 * q + e];
                        hi[2 * e] = acc[m][0][4 * q + 2 + e];
                        hi[2 * e + 1] = acc[m][1][4 * q + 2 + e];
                    }
                    *reinterpret_cast<f4*>(red + red_at(row, 4 * q + 2 * half)) = lo;
                    *reinterpret_cast<f4*>(red + red_at(row, 4 * q + 2 * half + 1)) = hi;
                }
            }
        }
        __syncthreads();
        // thread t: tile row t / 8, chunks 2 (t % 8) and + 1 (8 columns)
        {
            const int r = tid >> 3;
            const int row = tm * BM + r;
            const bool add_bias = BIAS && p.split_k == 1;
            const float bv = add_bias && row < p.M ? p.bias[row] : 0.f;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int c = 2 * (tid & 7) + h;
                const int o = red_at(r, c);
                constexpr int W1 = BM * BM;  // the second wave's buffer in a stage object
                f4 v = *reinterpret_cast<const f4*>(st0 + o);
                v += *reinterpret_cast<const f4*>(st0 + W1 + o);
                v += *reinterpret_cast<const f4*>(st1 + o);
                v += *reinterpret_cast<const f4*>(st1 + W1 + o);
                v += *reinterpret_cast<const f4*>(st2 + o);
                v += *reinterpret_cast<const f4*>(st2 + W1 + o);
                v += *reinterpret_cast<const f4*>(st3 + o);
                v += *reinterpret_cast<const f4*>(st3 + W1 + o);
                if (add_bias) v += bv;
                const int col = tn * BM + 4 * c;
                if (row < p.M) {
                    // (a stream-K segment that does not start at k = 0: its
                    // slot, tile-local, row stride BM, 16-byte aligned)
                    float* const dst = to_slot ? sk_slot + r * BM + 4 * c : C + (int64_t)row * ldc + col;
                    if ((to_slot || c_vec) && col + 3 < p.N) {
                        *reinterpret_cast<f4*>(dst) = v;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (col + e < p.N) dst[e] = v[e];
                    }
                }
            }
        }
        __syncthreads();  // the buffers are read before the next tile's loads refill them
    }
}

template <bool AT, bool BT>
inline hipError_t launch_ksplit(const GemmLaunch& g, hipStream_t s) {
    const GemmParams p = make_params(g);
    if (g.sk_tiles > 0) {  // stream-K (the scheduler plans it for batch 1, split 1, no bias)
        hipLaunchKernelGGL((gemm_f32_ksplit_kernel<AT, BT, false, true>), dim3((unsigned)g.grid_x),
                           dim3(512), 0, s, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_sk_fixup(g, s);
    }
    dim3 grid((unsigned)g.grid_x, (unsigned)g.split_k, (unsigned)g.batch);
    if constexpr (!AT && !BT) {  // the row bias exists for N/N only
        if (g.bias != nullptr && g.split_k == 1) {
            hipLaunchKernelGGL((gemm_f32_ksplit_kernel<false, false, true>), grid, dim3(512), 0, s, p);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemm_f32_ksplit_kernel<AT, BT, false>), grid, dim3(512), 0, s, p);
    return hipGetLastError();
}

}  // namespace mi
