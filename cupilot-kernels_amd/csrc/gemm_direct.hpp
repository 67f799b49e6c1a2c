// gemm_direct.hpp -- the 256 x 256 N/N contraction with global -> LDS direct
// loads (gfx950 global_load_lds_dwordx4), for dense problems whose slices are
// all full (K a multiple of 32, 16-byte aligned operands) and long (K >= 1024).
//
// Same tile, waves, MFMA order and epilogue as gemm_f32_kernel<Tile256>; what
// changes is the staging.  Each lane's 16-byte global load lands in LDS at
// (wave's LDS base + 16 * lane) without passing through VGPRs, so
//   * no VGPRs hold the next slice (32 per lane in the register-staged kernel),
//   * no ds_write instructions, and no wait for the loads before the MFMAs
//     of the current slice end: the single barrier per slice (which waits for
//     the wave's own loads first) publishes the whole next slice.
// A wave's 64 lanes fill 1 KiB of contiguous LDS, which fixes the layouts:
//   K-contiguous operand: [mn][32] with the 16-byte chunks of row mn stored
//     at chunk (q ^ (mn % 8)); a lane chooses which global chunk it loads so
//     that its fixed LDS slot holds the right one.  The fragment read of 32
//     consecutive rows at one chunk then touches 8 different bank groups per
//     8 lanes (no conflicts) without padding.
//   MN-contiguous operand: [32][256 + 4], one k-row per wave instruction
//     (the +4 padding sits between rows, where each instruction's base is free).
// Rows / columns past the matrix edge are loaded from the last valid row /
// column instead (they only feed outputs that are never stored); K has no
// tail here, so every loaded k is real.
#pragma once

#include <type_traits>

#include "gemm_kernel.hpp"

namespace mi {

typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(1))) void* global_void_ptr;

__device__ __forceinline__ void load_lds16(const float* g, float* lds) {
    __builtin_amdgcn_global_load_lds((global_void_ptr)(g), (lds_void_ptr)(lds), 16, 0, 0);
}

// One operand of a 256 x 32 slice, staged directly into LDS by NW waves.
template <bool KCONTIG, int NW>
struct DirectLoader {
    static constexpr int ROWS = 256, BK = 32;
    static constexpr int LD = KCONTIG ? BK : ROWS + 4;
    static constexpr int ELEMS = KCONTIG ? ROWS * BK : BK * LD;
    // wave instructions per slice: 8 rows of 128 B (K-contiguous) or one
    // k-row of 1 KiB (MN-contiguous) each
    static constexpr int INSTR = KCONTIG ? ROWS / 8 : BK;
    static_assert(INSTR % NW == 0, "instructions must split evenly over the waves");
    static constexpr int PER_WAVE = INSTR / NW;

    // Issue this wave's loads of the slice at (mn0, k0) into `lds`.
    __device__ __forceinline__ static void load(const float* __restrict__ base, int64_t ld, int mn0,
                                                int mn_ext, int k0, float* lds, int wave, int lane) {
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
            const int ins = wave * PER_WAVE + i;
            if (KCONTIG) {
                const int r = ins * 8 + (lane >> 3);          // tile row this lane fills
                const int q = (lane & 7) ^ (r & 7);           // global chunk for its slot
                int gr = mn0 + r;
                gr = gr < mn_ext ? gr : mn_ext - 1;
                load_lds16(base + (int64_t)gr * ld + k0 + q * 4, lds + ins * 8 * BK);
            } else {
                const int k = ins;
                int c = mn0 + lane * 4;
                c = c + 3 < mn_ext ? c : mn_ext - 4;
                load_lds16(base + (int64_t)(k0 + k) * ld + c, lds + k * LD);
            }
        }
    }

    // Operand values for the 4 MFMA steps of k-block kb, 32-row group at r0
    // (same k permutation as TileLoader::frag: k = 8 kb + 4 h + s).
    __device__ __forceinline__ static void frag(const float* lds, int r0, int kb, int lane,
                                                float out[4]) {
        const int half = lane >> 5;
        const int l32 = lane & 31;
        if (KCONTIG) {
            const int row = r0 + l32;
            const int q = (2 * kb + half) ^ (l32 & 7);  // r0 % 8 == 0, so row % 8 == l32 % 8
            const f4 t = *reinterpret_cast<const f4*>(lds + row * BK + q * 4);
            out[0] = t[0];
            out[1] = t[1];
            out[2] = t[2];
            out[3] = t[3];
        } else {
            const float* p = lds + (kb * 8 + half * 4) * LD + r0 + l32;
#pragma unroll
            for (int s = 0; s < 4; ++s) out[s] = p[s * LD];
        }
    }
};

// Persistent like gemm_f32_kernel; per slice: issue the next slice's direct
// loads (same tile, the next tile's first slice, or -- after the workgroup's
// last slice -- this slice again, never used) into the other buffer, run this
// slice's MFMAs, barrier (which first waits for this wave's loads), and after
// a tile's last slice issue its stores.  The two LDS buffers of each operand
// are separate __shared__ objects and the slice loop is unrolled by two, so
// each access names its buffer at compile time.
//
// Measured against the register-staged kernel at 8192^3 (same process,
// interleaved): N/N 136.7-136.9 vs 135.0-135.3 TFLOP/s; large-K and batched
// also gain ~1-2 %, but 4-D (K = 256) loses 5 % and the other layouts lose
// 2-7 %, so only N/N with K >= 1024 takes this path.
template <class T, bool BIAS>
__global__ void __launch_bounds__(T::NT)
    __attribute__((amdgpu_waves_per_eu(T::WAVES_PER_SIMD, T::WAVES_PER_SIMD)))
    gemm_f32_direct_kernel(const GemmParams p) {
    static_assert(T::BM == 256 && T::BN == 256 && T::BK == 32, "direct staging is built for Tile256");
    using LA = DirectLoader<true, T::NW>;   // A row-major: K-contiguous
    using LB = DirectLoader<false, T::NW>;  // B row-major: N-contiguous
    __shared__ __attribute__((aligned(16))) float sA0[LA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sA1[LA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB0[LB::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB1[LB::ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / T::WAVES_N;
    const int wn = wave % T::WAVES_N;
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

    f16v acc[T::TM][T::TN];
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
        for (int j = 0; j < T::TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    auto issue = [&](const TileWork& w, int it, float* dA, float* dB) __attribute__((always_inline)) {
        const int k0 = w.k_begin + it * T::BK;
        LA::load(A, p.lda, w.tm * T::BM, p.M, k0, dA, wave, lane);
        LB::load(B, p.ldb, w.tn * T::BN, p.N, k0, dB, wave, lane);
    };
    // fragments of one k-block, kept at kernel scope (two sets, by k-block parity)
    float fa[2][T::TM][4], fb[2][T::TN][4];
    // (every lambda here is force-inlined: a call would pass the accumulators
    // through scratch memory)
    auto compute = [&](const float* As, const float* Bs) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < T::BK / 8; ++kb) {
            const int set = kb & 1;
#pragma unroll
            for (int i = 0; i < T::TM; ++i) LA::frag(As, wm * T::WM + i * 32, kb, lane, fa[set][i]);
#pragma unroll
            for (int j = 0; j < T::TN; ++j) LB::frag(Bs, wn * T::WN + j * 32, kb, lane, fb[set][j]);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < T::TM; ++i)
#pragma unroll
                    for (int j = 0; j < T::TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[set][j][s], fa[set][i][s],
                                                                         acc[i][j], 0, 0, 0);
        }
    };

    int t = blockIdx.x;
    if (t >= p.num_tiles) return;
    TileWork cur = decode_tile<T, kDense>(p, t);
    int it = 0;
    issue(cur, 0, sA0, sB0);
    __syncthreads();

    // One slice from buffer CB; returns true after the workgroup's last tile.
    auto slice = [&](auto cb_tag) __attribute__((always_inline)) -> bool {
        constexpr int CB = decltype(cb_tag)::value;
        const float* const curA = CB == 0 ? sA0 : sA1;
        const float* const curB = CB == 0 ? sB0 : sB1;
        float* const nxtA = CB == 0 ? sA1 : sA0;
        float* const nxtB = CB == 0 ? sB1 : sB0;
        const bool last = it + 1 >= cur.nk;
        int nt = t;
        bool has_next = true;
        TileWork nw = cur;
        int nit = it + 1;
        if (last) {
            nt = t + gridDim.x;
            has_next = nt < p.num_tiles;
            nit = has_next ? 0 : it;
            if (has_next) nw = decode_tile<T, kDense>(p, nt);
        }
        issue(nw, nit, nxtA, nxtB);
        compute(curA, curB);
        __syncthreads();
        if (!last) {
            ++it;
            return false;
        }
        store_tile<T, kDense, BIAS>(p, C, ldc, c_vec, cur, acc, false, wm, wn, lane);
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
#pragma unroll
            for (int j = 0; j < T::TN; ++j)
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

// N/N launches of the 256 tile on dense problems with every slice full,
// 16-byte aligned operands and K >= 1024 take direct staging.
inline bool direct_ok(const GemmLaunch& g) {
    return g.cfg == kCfg256 && g.structure == kDense && g.vec == 4 && g.K % 32 == 0 &&
           g.k_chunk % 32 == 0 && g.k_chunk >= 1024 && g.op_a == 0 && g.op_b == 0;
}

inline hipError_t launch_direct_nn(const GemmLaunch& g, hipStream_t s) {
    const GemmParams p = make_params(g);
    dim3 grid((unsigned)g.grid_x, (unsigned)g.split_k, (unsigned)g.batch);
    if (g.bias != nullptr && g.split_k == 1)
        hipLaunchKernelGGL((gemm_f32_direct_kernel<Tile256, true>), grid, dim3(Tile256::NT), 0, s, p);
    else
        hipLaunchKernelGGL((gemm_f32_direct_kernel<Tile256, false>), grid, dim3(Tile256::NT), 0, s, p);
    return hipGetLastError();
}

}  // namespace mi
