// gemm_kernel.hpp -- fp32 MFMA contraction engine for gfx950 (CDNA4).
//
// One kernel template covers the whole dense family of the reference
// (kernels/1,2,3,6,7,8,9,10,11,13,16,17,18) and the triangular pair
// (kernels/14,15): C[b] = op_a(A[b]) . op_b(B[b]) in true fp32 on
// v_mfma_f32_32x32x2_f32 (the reference quantises to fp16/bf16/tf32 first).
//
// Structure of one workgroup:
//   * a BM x BN output tile; waves arranged WAVES_M x WAVES_N, each owning a
//     WM x WN sub-tile held as (WM/32) x (WN/32) MFMA accumulators (16 VGPR each);
//   * K is walked in BK-deep slices (16 or 32; the small-K configs take the
//     whole K in one slice) through two LDS buffers (one barrier per slice:
//     the next slice's global loads are issued before the MFMAs of the current
//     one and written to the other buffer after them);
//   * each operand is kept in LDS in the orientation it has in HBM, so every
//     global load is a coalesced 16-byte load and every LDS store a
//     ds_write_b128 with no transpose:
//       K-contiguous operand (A row-major, B stored N x K): [mn][BK + 4],
//         fragments read with one ds_read_b128 per 4 MFMA steps;
//       MN-contiguous operand (A stored K x M, B row-major): [BK][MN + 4],
//         fragments read with ds_read_b32 (32 consecutive floats per half wave).
//     Within a k-block of 8, lane half h = lane / 32 and MFMA step s use
//     k = 8*kb + 4*h + s for both operands, which is what lets the
//     K-contiguous side use 16-byte reads.
//   * the B fragment is the MFMA's row operand, so each accumulator block is
//     the block of C^T: lane l holds output row l % 32 and, in register group
//     g, the 4 consecutive columns 8g + 4h .. +3 -> one 16-byte store per
//     group, masked at the matrix edge and, for the triangular modes, on the
//     diagonal (+0.0 on the wrong side);
//   * persistent over tiles and software-pipelined across them (see
//     gemm_f32_kernel), with an XCD-aware grouped raster.
// Split-K (used for K >> M, N) writes fp32 partial tiles to a workspace that
// a second kernel sums in fixed split order, so results are deterministic.
#pragma once

#include "mi_device.hpp"
#include "mi_internal.hpp"

namespace mi {

template <int BM_, int BN_, int WM_, int WN_, int BK_, int WAVES_PER_SIMD_, int STAGES_ = 2>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    // LDS buffers per operand: 2 = double-buffered K loop; 1 = the whole K of
    // a tile fits one slice (small-K configs), halving the LDS footprint.
    static constexpr int STAGES = STAGES_;
    // occupancy the build is held to, so the persistent grid (the scheduler's
    // resident workgroups per CU) matches what the hardware can hold
    static constexpr int WAVES_PER_SIMD = WAVES_PER_SIMD_;
    static constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
    static constexpr int NW = WAVES_M * WAVES_N, NT = NW * 64;
    static constexpr int TM = WM / 32, TN = WN / 32;
};

using Tile64 = Tile<64, 64, 32, 32, 16, 8>;      // 8 workgroups of 4 waves per CU
using Tile128 = Tile<128, 128, 64, 64, 16, 3>;   // 3 workgroups of 4 waves per CU
using Tile256 = Tile<256, 256, 128, 64, 32, 2>;  // 1 workgroup of 8 waves per CU
using Tile128K32 = Tile<128, 128, 64, 64, 32, 3, 1>;  // K <= 32 in one slice, 3 WGs per CU
using Tile128K64 = Tile<128, 128, 64, 64, 64, 2, 1>;  // K <= 64 in one slice, 2 WGs per CU
using Tile128B32 = Tile<128, 128, 64, 64, 32, 2>;     // 32-deep slices, direct-staged, 2 WGs per CU
using Tile128W8 = Tile<128, 128, 32, 64, 32, 4>;      // the same, 8 waves of 32 x 64, 2 WGs per CU

enum { kDense = 0, kLower = 1, kUpper = 2 };

// One operand tile of ROWS (m or n) x BK (k) floats, staged through registers.
template <int ROWS, int BK, int NT, bool KCONTIG, int VEC>
struct TileLoader {
    static constexpr int PAD = 4;
    static constexpr int LD = KCONTIG ? (BK + PAD) : (ROWS + PAD);
    static constexpr int ELEMS = KCONTIG ? ROWS * LD : BK * LD;
    static constexpr int SLOTS = ROWS * BK / 4;  // 16-byte slots per tile
    static_assert(SLOTS % NT == 0, "tile must split evenly over the workgroup");
    static constexpr int NS = SLOTS / NT;

    f4 v[NS];

    // First element (mn, k) of slot idx; its 4 elements run along k when the
    // operand is K-contiguous, along mn otherwise.
    __device__ __forceinline__ static void slot_pos(int idx, int& mn, int& k) {
        if (KCONTIG) {
            mn = idx / (BK / 4);
            k = (idx % (BK / 4)) * 4;
        } else {
            k = idx / (ROWS / 4);
            mn = (idx % (ROWS / 4)) * 4;
        }
    }

    // Load the tile at (mn0, k0).  Elements with mn >= mn_ext or k >= k_end
    // read as zero.  VEC == 4 requires the contiguous extent and ld to be
    // multiples of 4 and a 16-byte aligned base (checked by the host).
    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int mn0,
                                         int mn_ext, int k0, int k_end, int tid) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            int mn, k;
            slot_pos(tid + s * NT, mn, k);
            const int gmn = mn0 + mn, gk = k0 + k;
            if (VEC == 4) {
                const bool ok = gmn < mn_ext && gk < k_end;
                const int64_t off = KCONTIG ? (int64_t)gmn * ld + gk : (int64_t)gk * ld + gmn;
                if (ok) {
                    v[s] = *reinterpret_cast<const f4*>(base + off);
                } else {
                    v[s] = f4{0.f, 0.f, 0.f, 0.f};
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int emn = KCONTIG ? gmn : gmn + e;
                    const int ek = KCONTIG ? gk + e : gk;
                    const bool ok = emn < mn_ext && ek < k_end;
                    const int64_t off = KCONTIG ? (int64_t)emn * ld + ek : (int64_t)ek * ld + emn;
                    v[s][e] = ok ? base[off] : 0.f;
                }
            }
        }
    }

    // Triangular input masks: IS_A selects the row operand (mn = i) else the
    // column operand (mn = j).  LOWER keeps A[i][k] for k <= i and B[k][j] for
    // k >= j; UPPER the mirror image.
    template <int MODE, bool IS_A>
    __device__ __forceinline__ void mask(int mn0, int k0, int tid) {
        if (MODE == kDense) return;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            int mn, k;
            slot_pos(tid + s * NT, mn, k);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int emn = mn0 + (KCONTIG ? mn : mn + e);
                const int ek = k0 + (KCONTIG ? k + e : k);
                bool keep;
                if (MODE == kLower) keep = IS_A ? (ek <= emn) : (ek >= emn);
                else keep = IS_A ? (ek >= emn) : (ek <= emn);
                if (!keep) v[s][e] = 0.f;
            }
        }
    }

    __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            int mn, k;
            slot_pos(tid + s * NT, mn, k);
            float* dst = KCONTIG ? lds + mn * LD + k : lds + k * LD + mn;
            *reinterpret_cast<f4*>(dst) = v[s];
        }
    }

    // Operand values for the 4 MFMA steps of k-block kb, 32-row group at r0.
    __device__ __forceinline__ static void frag(const float* lds, int r0, int kb, int lane,
                                                float out[4]) {
        const int half = lane >> 5;
        if (KCONTIG) {
            const f4 t = *reinterpret_cast<const f4*>(lds + (r0 + (lane & 31)) * LD + kb * 8 + half * 4);
            out[0] = t[0];
            out[1] = t[1];
            out[2] = t[2];
            out[3] = t[3];
        } else {
            const float* p = lds + (kb * 8 + half * 4) * LD + r0 + (lane & 31);
#pragma unroll
            for (int s = 0; s < 4; ++s) out[s] = p[s * LD];
        }
    }
};

// Which output tile workgroup `bid` (of `nblocks`) owns and which K range
// [k_begin, k_end) it reduces for split `split`.  Returns false for a
// triangular off-structure tile (written with zeros).  Shared by the kernel
// and the host introspection entry point mi_gemm_tile_of.
template <int BM, int BN, int MODE>
__host__ __device__ __forceinline__ bool tile_of(const GemmParams& p, int bid, int nblocks, int split,
                                                 int& tm, int& tn, int& k_begin, int& k_end) {
    if (MODE == kDense) {
        const int pid = xcd_remap(bid, nblocks);
        raster(pid, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
        k_begin = split * p.k_chunk;
        k_end = p.K < k_begin + p.k_chunk ? p.K : k_begin + p.k_chunk;
        return true;
    }
    // Triangular tiles differ in length, so they keep the hardware's
    // round-robin XCD order: every XCD then draws from the whole longest-first
    // list instead of one XCD receiving all the longest tiles.
    const bool lower = MODE == kLower;
    if (!tri_tile(bid, p.tiles_m, lower, tm, tn)) {
        k_begin = k_end = 0;
        return false;
    }
    const int hi = lower ? (tm + 1) * BM : (tn + 1) * BN;
    k_begin = lower ? tn * BN : tm * BM;
    k_end = p.K < hi ? p.K : hi;
    return true;
}

// One output tile's assignment, uniform across the workgroup.
struct TileWork {
    int tm, tn, k_begin, k_end, nk;
    // 0 or 1 (ints, so that the struct has no padding bytes: copies of a
    // padded struct keep the padding in memory -- here, in LDS)
    int compute;
    int mirror;  // chunked triangular list: partial sum goes to tile (tn, tm);
                 // stream-K: the segment goes to workspace slot `slot`
    int slot;
};

template <class T, int MODE>
__device__ __forceinline__ TileWork decode_tile(const GemmParams& p, int tile) {
    TileWork w;
    w.compute = tile_of<T::BM, T::BN, MODE>(p, tile, p.num_tiles, blockIdx.y, w.tm, w.tn,
                                            w.k_begin, w.k_end);
    w.nk = w.compute && w.k_end > w.k_begin ? (w.k_end - w.k_begin + T::BK - 1) / T::BK : 0;
    w.mirror = 0;
    w.slot = 0;
    return w;
}

// Store one finished tile from its accumulators (zeros for a tile with no K
// work).  Block (i, j) holds C^T: lane l owns row l%32 of the 32x32 block and
// accumulator registers 4g..4g+3 its columns 8g + 4*(l/32) .. +3, so every
// register group is one 16-byte store.  Triangular modes write +0.0 on the
// wrong side of the diagonal.  A per-row bias (dense only) is added here when
// the tile holds the full sum; split-K partials get it in the reduction.
template <class T, int MODE, bool BIAS>
__device__ __forceinline__ void store_tile(const GemmParams& p, float* C, int64_t ldc, bool c_vec,
                                           const TileWork& w, const f16v (&acc)[T::TM][T::TN],
                                           bool zero, int wm, int wn, int lane) {
    const int m0 = w.tm * T::BM, n0 = w.tn * T::BN;
    const int half = lane >> 5;
    // (a separate instantiation, so the plain epilogue carries no bias code)
    const bool add_bias = BIAS && MODE == kDense && p.split_k == 1;
#pragma unroll
    for (int i = 0; i < T::TM; ++i) {
        const int brow = m0 + wm * T::WM + i * 32 + (lane & 31);
        const float bv = add_bias && brow < p.M ? p.bias[brow] : 0.f;
#pragma unroll
        for (int j = 0; j < T::TN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int row = brow;
                const int col = n0 + wn * T::WN + j * 32 + g * 8 + half * 4;
                if (row >= p.M) continue;
                f4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = zero ? 0.f : acc[i][j][4 * g + e];
                    if (add_bias) x += bv;
                    if (MODE == kLower && col + e > row) x = 0.f;
                    if (MODE == kUpper && col + e < row) x = 0.f;
                    v[e] = x;
                }
                float* dst = C + (int64_t)row * ldc + col;
                if (c_vec && col + 3 < p.N) {
                    *reinterpret_cast<f4*>(dst) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < p.N) dst[e] = v[e];
                }
            }
    }
}

// Persistent over tiles (workgroup b owns tiles b, b + gridDim.x, ...) and
// software-pipelined over the sequence of (tile, K slice): while the MFMAs of
// one slice run, the global loads of the next slice -- of the same tile, or
// the first slice of the next tile -- are in flight; they are written to the
// other LDS buffer, and only then are a finished tile's stores issued.  vmcnt
// counts in issue order and the stores sit behind data-dependent branches, so
// any wait for a prefetch also waits for every store issued before it; with
// this order those are the previous tile's stores, which have had at least a
// slice of MFMAs to drain.
template <class T, bool AT, bool BT, int VEC, int MODE, bool BIAS>
__global__ void __launch_bounds__(T::NT)
    __attribute__((amdgpu_waves_per_eu(T::WAVES_PER_SIMD, T::WAVES_PER_SIMD)))
    gemm_f32_kernel(const GemmParams p) {
    constexpr bool A_KC = !AT;  // A row-major (M x K) is contiguous along K
    constexpr bool B_KC = BT;   // B stored N x K is contiguous along K
    using LA = TileLoader<T::BM, T::BK, T::NT, A_KC, VEC>;
    using LB = TileLoader<T::BN, T::BK, T::NT, B_KC, VEC>;
    __shared__ __attribute__((aligned(16))) float sA[T::STAGES][LA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB[T::STAGES][LB::ELEMS];

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
    // 16-byte output stores need every row start 16-byte aligned
    const bool c_vec = (ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(C) & 15u) == 0);

    f16v acc[T::TM][T::TN];
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
        for (int j = 0; j < T::TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Next tile at or after t (stride gridDim.x) that has K work; tiles
    // without any (triangular off-structure tiles) are written with zeros on
    // the way.  Uniform across the workgroup.
    auto next_work = [&](int& t, TileWork& w) -> bool {
        while (t < p.num_tiles) {
            w = decode_tile<T, MODE>(p, t);
            if (w.nk > 0) return true;
            store_tile<T, MODE, BIAS>(p, C, ldc, c_vec, w, acc, true, wm, wn, lane);
            t += gridDim.x;
        }
        return false;
    };
    auto load_slice = [&](LA& la, LB& lb, const TileWork& w, int it) {
        const int k0 = w.k_begin + it * T::BK;
        la.load(A, p.lda, w.tm * T::BM, p.M, k0, w.k_end, tid);
        lb.load(B, p.ldb, w.tn * T::BN, p.N, k0, w.k_end, tid);
        la.template mask<MODE, true>(w.tm * T::BM, k0, tid);
        lb.template mask<MODE, false>(w.tn * T::BN, k0, tid);
    };

    // MFMAs of the slice in LDS buffer cb into acc
    auto compute = [&](int cb) {
        const float* As = sA[cb];
        const float* Bs = sB[cb];
#pragma unroll
        for (int kb = 0; kb < T::BK / 8; ++kb) {
            float a[T::TM][4], b[T::TN][4];
#pragma unroll
            for (int i = 0; i < T::TM; ++i) LA::frag(As, wm * T::WM + i * 32, kb, lane, a[i]);
#pragma unroll
            for (int j = 0; j < T::TN; ++j) LB::frag(Bs, wn * T::WN + j * 32, kb, lane, b[j]);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < T::TM; ++i)
#pragma unroll
                    for (int j = 0; j < T::TN; ++j)
                        // B fragment as the row operand: the 32x32 result is
                        // the block of C^T (see store_tile)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[j][s], a[i][s],
                                                                         acc[i][j], 0, 0, 0);
        }
    };

    int t = blockIdx.x;
    TileWork cur;
    if (!next_work(t, cur)) return;

    LA la;
    LB lb;
    load_slice(la, lb, cur, 0);
    la.store(sA[0], tid);
    lb.store(sB[0], tid);
    __syncthreads();

    int cb = 0;
    for (;;) {
        // Inner slices of the tile: the next slice is always this tile's, so
        // the prefetch and its LDS write are unconditional and every load is
        // awaited in the iteration that issued it.
        for (int it = 0; it + 1 < cur.nk; ++it) {
            load_slice(la, lb, cur, it + 1);
            compute(cb);
            if (T::STAGES == 1) __syncthreads();  // the one buffer is free only now
            const int nb = T::STAGES == 2 ? (cb ^ 1) : 0;
            la.store(sA[nb], tid);
            lb.store(sB[nb], tid);
            __syncthreads();
            cb = nb;
        }

        // Last slice: prefetch the first slice of the next tile (or, after the
        // last tile, re-read the current slice, never used), write it to LDS,
        // and only then issue this tile's stores -- vmcnt counts in issue
        // order, so a wait for the prefetch never covers fresh stores.
        int nt = t + gridDim.x;
        TileWork nw;
        const bool has_next = next_work(nt, nw);
        if (has_next) load_slice(la, lb, nw, 0);
        else load_slice(la, lb, cur, cur.nk - 1);
        compute(cb);
        if (T::STAGES == 1) __syncthreads();
        const int nb = T::STAGES == 2 ? (cb ^ 1) : 0;
        la.store(sA[nb], tid);
        lb.store(sB[nb], tid);
        store_tile<T, MODE, BIAS>(p, C, ldc, c_vec, cur, acc, false, wm, wn, lane);
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
#pragma unroll
            for (int j = 0; j < T::TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
        __syncthreads();
        if (!has_next) break;
        t = nt;
        cur = nw;
        cb = nb;
    }
}

inline GemmParams make_params(const GemmLaunch& g) {
    GemmParams p;
    p.A = g.A;
    p.B = g.B;
    p.C = g.C;
    p.ws = g.ws;
    p.bias = g.bias;
    p.M = g.M;
    p.N = g.N;
    p.K = g.K;
    p.tiles_m = g.tiles_m;
    p.tiles_n = g.tiles_n;
    p.group_m = g.group_m;
    p.k_chunk = g.k_chunk;
    p.split_k = g.split_k;
    p.lda = g.lda;
    p.ldb = g.ldb;
    p.ldc = g.ldc;
    p.sa = g.sa;
    p.sb = g.sb;
    p.sc = g.sc;
    p.num_tiles = g.num_tiles;
    p.col_splits = g.col_splits;
    p.tri_cap = g.tri_cap;
    p.sk_dp = g.sk_dp;
    p.sk_tiles = g.sk_tiles;
    p.sk_ipt = g.sk_ipt;
    p.sk_nph = g.sk_nph;
    for (int q = 0; q < kSkMaxPhases; ++q) p.sk_ph[q] = g.sk_ph[q];
    p.ws_batch_stride = (int64_t)g.M * g.N;
    p.ws_split_stride = p.ws_batch_stride * g.batch;
    return p;
}

template <class T, bool AT, bool BT, int VEC, int MODE, bool BIAS = false>
hipError_t launch_one(const GemmLaunch& g, hipStream_t s) {
    const GemmParams p = make_params(g);
    dim3 grid((unsigned)g.grid_x, (unsigned)g.split_k, (unsigned)g.batch);
    // grid_x <= num_tiles workgroups walk the tile list (persistent)
    hipLaunchKernelGGL((gemm_f32_kernel<T, AT, BT, VEC, MODE, BIAS>), grid, dim3(T::NT), 0, s, p);
    return hipGetLastError();
}

template <class T, bool AT, bool BT>
hipError_t launch_cfg(const GemmLaunch& g, hipStream_t s) {
    // the per-row bias epilogue exists for the N/N layout only (the scheduler
    // rejects bias with any other)
    if constexpr (!AT && !BT) {
        if (g.structure == kDense && g.bias != nullptr && g.split_k == 1)
            return g.vec == 4 ? launch_one<T, AT, BT, 4, kDense, true>(g, s)
                              : launch_one<T, AT, BT, 1, kDense, true>(g, s);
    }
    if (g.structure == kDense) {
        return g.vec == 4 ? launch_one<T, AT, BT, 4, kDense>(g, s)
                          : launch_one<T, AT, BT, 1, kDense>(g, s);
    }
    if constexpr (!AT && !BT) {
        if (g.structure == kLower)
            return g.vec == 4 ? launch_one<T, AT, BT, 4, kLower>(g, s)
                              : launch_one<T, AT, BT, 1, kLower>(g, s);
        return g.vec == 4 ? launch_one<T, AT, BT, 4, kUpper>(g, s)
                          : launch_one<T, AT, BT, 1, kUpper>(g, s);
    }
    return hipErrorInvalidValue;
}

template <bool AT, bool BT>
hipError_t launch_layout(const GemmLaunch& g, hipStream_t s) {
    switch (g.cfg) {
        case kCfg64: return launch_cfg<Tile64, AT, BT>(g, s);
        case kCfg128: return launch_cfg<Tile128, AT, BT>(g, s);
        case kCfg256: return launch_cfg<Tile256, AT, BT>(g, s);
        case kCfg128K32: return launch_cfg<Tile128K32, AT, BT>(g, s);
        case kCfg128K64: return launch_cfg<Tile128K64, AT, BT>(g, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mi
