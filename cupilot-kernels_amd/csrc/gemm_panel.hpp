// gemm_panel.hpp -- fp32 MFMA contraction for small K (K <= KMAX = 32 or 64):
// the store-bound shapes of the family (kernels/7_... small K, kernels/9_...
// tall-skinny), where C is 32x-64x larger than A and B.
//
// With the whole K in one slice, the general engine re-reads an A tile and a B
// tile for every output tile; at K = 64 and 128 x 128 tiles that is as many
// bytes loaded (from L2/MALL) as stored, and the loads, not the MFMAs or the
// stores, set the pace.  Here a workgroup instead owns one BM-row panel of A,
// kept in LDS for its whole life, and walks a run of BN-wide column tiles:
// per step it loads only the K x BN tile of B (double-buffered in LDS),
// computes the BM x BN tile and stores it.  The next B tile's global loads run
// under the current tile's MFMAs and are written to LDS before the current
// tile's stores are issued: vmcnt counts in issue order, so the wait for those
// loads covers only the previous tile's stores, which have drained behind a
// whole tile of MFMAs.  Load traffic falls to ~K/BM of the output (1/4 at K = 64).
#pragma once

#include "gemm_kernel.hpp"

namespace mi {

template <int BM_, int BN_, int KMAX_, int WM_ = 64, int WN_ = 64, bool PANEL_B_ = false>
struct PanelTile {
    static constexpr int BM = BM_, BN = BN_, KMAX = KMAX_;
    static constexpr int WM = WM_, WN = WN_;  // wave tile
    static constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
    static constexpr int NW = WAVES_M * WAVES_N, NT = NW * 64;
    static constexpr int TM = WM / 32, TN = WN / 32;
    // false: the resident panel is A's BM rows and the walk streams B's
    // BN-column tiles; true: the resident panel is B's BN columns and the walk
    // streams A's BM-row tiles (work items: column panels x row runs)
    static constexpr bool PANEL_B = PANEL_B_;
};

using Panel32 = PanelTile<256, 128, 32>;
using Panel64 = PanelTile<256, 128, 64>;
// 128-row panels (M = 128 .. 2047 not a multiple of 256: a 256-row panel
// would spend MFMAs on padding rows), 8 waves of 64 x 32
using Panel128x64 = PanelTile<128, 128, 64, 64, 32>;
// B-resident 256-column panels streaming 128-row A tiles (K <= 64), for
// large M: the workgroups of one XCD walk the same A tiles in step, so each
// A tile comes from HBM once per XCD and is shared in its L2, while their
// stores go to the same rows in different column panels, i.e. to contiguous
// addresses spread over every channel.  (With the A panel resident, a
// lockstep walk shares the B tiles the same way but stores every
// workgroup's tile to the same columns of different rows: measured 16 %
// slower on 65536^2 x 64 than the rotated walk, whose B tiles, read by
// every workgroup at its own time, miss L2: 4.3 GB fetched per call.)
// Measured on 65536^2 x 64: 4.98-5.09 vs 5.25-5.27 ms (N/N; T/N, N/T, T/T
// 7-10 % faster), 0.15 GB fetched per call; results bitwise equal to the
// A-resident panel's.  (Holding the accumulators as C instead of C^T, for
// 4-byte stores each covering two whole 128-byte row segments, measured
// 6 % slower.)
using Panel64B = PanelTile<128, 256, 64, 64, 64, true>;

template <class T, bool AT, bool BT, int VEC, bool BIAS>
__global__ void __launch_bounds__(T::NT) gemm_f32_panel_kernel(const GemmParams p) {
    constexpr bool A_KC = !AT;
    constexpr bool B_KC = BT;
    constexpr bool PB = T::PANEL_B;
    static_assert(!(PB && BIAS), "the B-resident panel carries no per-row bias");
    using LA = TileLoader<T::BM, T::KMAX, T::NT, A_KC, VEC>;
    using LB = TileLoader<T::BN, T::KMAX, T::NT, B_KC, VEC>;
    // the resident operand has one LDS buffer, the streamed one two
    constexpr int NBA = PB ? 2 : 1, NBB = PB ? 1 : 2;
    __shared__ __attribute__((aligned(16))) float sA[NBA][LA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB[NBB][LB::ELEMS];
    // Where LDS has room (the 32-deep and the 128-row panels, not the 64-deep
    // 256-row or 256-column ones), each wave turns its finished 32 x 32 blocks
    // into whole-row stores through a [32][32] staging block whose 16-byte
    // chunks are XOR-swizzled per row (chunk ^ (row % 8)), so the writes (one
    // chunk of each of 32 rows) and the reads (whole rows) spread over the
    // banks.  Measured on the 32-deep panel (16384^2 x 32): 0 bank-conflict
    // cycles (SQ_LDS_BANK_CONFLICT) against 17 % of the LDS cycles with
    // rows padded to 36 floats, and twice that with chunk ^ ((row / 2) % 8);
    // the same speed.
    constexpr bool STAGE_C =
        (NBA * LA::ELEMS + NBB * LB::ELEMS + T::NW * 32 * 32) * 4 <= 160 * 1024;
    constexpr int SCLD = 32;
    __shared__ __attribute__((aligned(16))) float sC[STAGE_C ? T::NW * 32 * SCLD : 4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / T::WAVES_N;
    const int wn = wave % T::WAVES_N;
    const int half = lane >> 5;
    const int batch = blockIdx.z;
    const int nkb = (p.K + 7) / 8;  // 8-deep k-blocks that hold data (the rest is zero fill)

    const float* __restrict__ A = p.A + (int64_t)batch * p.sa;
    const float* __restrict__ B = p.B + (int64_t)batch * p.sb;
    float* C = p.C + (int64_t)batch * p.sc;
    const bool c_vec = (p.ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15u) == 0) &&
                       (p.sc % 4 == 0);

    // panels along the resident operand, each cut into col_splits runs of
    // streamed tiles
    const int tiles_p = PB ? p.tiles_n : p.tiles_m;
    const int tiles_s = PB ? p.tiles_m : p.tiles_n;
    const int items = tiles_p * p.col_splits;
    // bias (the panel kernel never splits K) is a separate instantiation, so
    // the plain store path carries no bias code
    constexpr bool add_bias = BIAS;
    LA la;
    LB lb;
    for (int w = blockIdx.x; w < items; w += gridDim.x) {
        const int tp = w / p.col_splits;
        const int cs = w - tp * p.col_splits;
        const int ts_begin = (int)((int64_t)cs * tiles_s / p.col_splits);
        const int ts_end = (int)((int64_t)(cs + 1) * tiles_s / p.col_splits);
        // the panel's first row (A panel) or column (B panel)
        const int p0 = tp * (PB ? T::BN : T::BM);
        // per-row bias of this lane's TM output rows, read once per item
        float bias_r[T::TM];
#pragma unroll
        for (int i = 0; i < T::TM; ++i) {
            const int row = p0 + wm * T::WM + i * 32 + (lane & 31);
            bias_r[i] = 0.f;
            if (add_bias && row < p.M) bias_r[i] = p.bias[row];
        }

        // Order of the walk.  A panel: each item starts at its own rotation,
        // so the workgroups running together store to different columns (in
        // lockstep from the same start they would hit addresses that differ
        // only in the row, i.e. the same few HBM channels).  B panel: the
        // items of one XCD (consecutive workgroups are dealt round-robin over
        // the 8 XCDs) start at the same row tile and walk in step, sharing
        // each A tile in their L2; the XCDs start 1/8 of the run apart.
        const int run = ts_end - ts_begin;
        const int rot = run <= 0 ? 0
                        : PB   ? (int)((int64_t)(blockIdx.x % kNumXcd) * run / kNumXcd)
                               : w % run;
        auto s_tile = [&](int step) {
            const int q = step + rot;
            return ts_begin + (q >= run ? q - run : q);
        };
        // output tile origin of streamed tile ts
        auto tile_m0 = [&](int ts) { return PB ? ts * T::BM : p0; };
        auto tile_n0 = [&](int ts) { return PB ? p0 : ts * T::BN; };
        // streamed-tile load into registers / into LDS buffer `buf`
        auto s_load = [&](int ts, int t) {
            if constexpr (PB)
                la.load(A, p.lda, ts * T::BM, p.M, 0, p.K, t);
            else
                lb.load(B, p.ldb, ts * T::BN, p.N, 0, p.K, t);
        };
        auto s_store = [&](int buf, int t) {
            if constexpr (PB)
                la.store(sA[buf], t);
            else
                lb.store(sB[buf], t);
        };

        // every wave is past the previous item's last barrier: LDS is free.
        // (the leading dimension and the thread index are made opaque per
        // item: otherwise the panel load's per-slot rows and addresses,
        // invariant across items, are hoisted out of the item loop and kept
        // live through it -- with A stored K x M more than the 64-deep
        // 256-row panel's 256 VGPRs hold.)
        int64_t ld_item = PB ? p.ldb : p.lda;
        int tid_p = tid;
        asm volatile("" : "+s"(ld_item), "+v"(tid_p));
        if constexpr (PB) {
            lb.load(B, ld_item, p0, p.N, 0, p.K, tid_p);
            lb.store(sB[0], tid_p);
        } else {
            la.load(A, ld_item, p0, p.M, 0, p.K, tid_p);
            la.store(sA[0], tid_p);
        }
        if (run > 0) {
            s_load(s_tile(0), tid);
            s_store(0, tid);
        }
        __syncthreads();

        // Fast path: the item's tiles are all interior and rows are 16-byte
        // aligned, so every store is unconditional; K may leave trailing
        // k-blocks of a 32-deep panel empty.  Two
        // accumulator sets: while tile s is computed, tile s-1 is stored, a
        // few 16-byte stores after each k-block of MFMAs, so stores and MFMAs
        // overlap inside each wave instead of alternating.
        // (the 64-deep 256-row panel takes it only when K fills all its
        // k-blocks: there a per-k-block skip test cost 6 % on the MFMA-bound
        // tall-skinny shape)
        constexpr bool SKIP_KB = T::KMAX == 32 || T::BM == 128;
        const bool interior = PB ? (p0 + T::BN <= p.N && (int64_t)ts_end * T::BM <= p.M)
                                 : (p0 + T::BM <= p.M && (int64_t)ts_end * T::BN <= p.N);
        const bool fast = c_vec && interior && run >= 2 && (SKIP_KB || nkb == T::KMAX / 8);
        if (fast) {
            constexpr int KBLK = T::KMAX / 8;
            // store units per wave per tile: 16-byte stores, or whole blocks
            // when staged through LDS
            constexpr int NST = STAGE_C ? T::TM * T::TN : T::TM * T::TN * 4;
            constexpr int SPK = (NST + KBLK - 1) / KBLK;
            f16v acc0[T::TM][T::TN], acc1[T::TM][T::TN];

            auto store_one = [&](const f16v (&acc)[T::TM][T::TN], int q, int ts) {
                const int m0 = tile_m0(ts), n0 = tile_n0(ts);
                if constexpr (STAGE_C) {
                    // block (i, j): write it in its C^T register layout (lane l:
                    // row l % 32, columns 8 g + 4 h .. +3), read it back as rows
                    // (lane L: row 8 r + L / 8, columns 4 (L % 8) .. +3), so each
                    // 16-byte store has 8 lanes covering one whole 128-byte row
                    // segment.  One wave's LDS operations run in order, so the
                    // reads see the writes and the next block's writes follow them.
                    const int i = q / T::TN, j = q % T::TN;
                    float* const buf = sC + wave * (32 * SCLD);
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        f4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                acc[i][j][4 * g + 3]};
                        if (add_bias) v += bias_r[i];
                        const int row = lane & 31, chunk = (2 * g + half) ^ (row & 7);
                        *reinterpret_cast<f4*>(buf + row * SCLD + chunk * 4) = v;
                    }
                    const int r0 = m0 + wm * T::WM + i * 32;
                    const int c0 = n0 + wn * T::WN + j * 32 + (lane & 7) * 4;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int rr = r * 8 + (lane >> 3);
                        const int chunk = (lane & 7) ^ (rr & 7);
                        const f4 v = *reinterpret_cast<const f4*>(buf + rr * SCLD + chunk * 4);
                        f4* const dst = reinterpret_cast<f4*>(C + (int64_t)(r0 + rr) * p.ldc + c0);
                        // non-temporal for the 128-row panel: measured 190 vs 208 us on
                        // the 1x1 convolution shape; equal or slower (up to 4 %) for
                        // the 256-row panels
                        if constexpr (T::BM == 128)
                            __builtin_nontemporal_store(v, dst);
                        else
                            *dst = v;
                    }
                } else {
                    const int i = q / (T::TN * 4), j = (q / 4) % T::TN, g = q % 4;
                    const int row = m0 + wm * T::WM + i * 32 + (lane & 31);
                    const int col = n0 + wn * T::WN + j * 32 + g * 8 + half * 4;
                    f4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                            acc[i][j][4 * g + 3]};
                    if (add_bias) v += bias_r[i];
                    *reinterpret_cast<f4*>(C + (int64_t)row * p.ldc + col) = v;
                }
            };
            // MFMAs of one tile from LDS buffers As / Bs into acc_c; with
            // STORE, the previous tile's stores ride along, SPK per k-block.
            auto tile_step = [&](f16v (&acc_c)[T::TM][T::TN], const float* As, const float* Bs,
                                 const f16v (&acc_s)[T::TM][T::TN], int ts_s, bool store) {
#pragma unroll
                for (int i = 0; i < T::TM; ++i)
#pragma unroll
                    for (int j = 0; j < T::TN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc_c[i][j][r] = 0.f;
#pragma unroll
                for (int kb = 0; kb < KBLK; ++kb) {
                    // k-blocks past K hold only zero fill: their MFMAs are
                    // skipped, the stores riding along with them are not
                    if (!SKIP_KB || kb < nkb) {
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
                                    acc_c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[j][s], a[i][s],
                                                                                       acc_c[i][j], 0, 0, 0);
                    }
                    if (store) {
#pragma unroll
                        for (int qq = 0; qq < SPK; ++qq)
                            if (kb * SPK + qq < NST) store_one(acc_s, kb * SPK + qq, ts_s);
                        // keep these stores among this k-block's MFMAs: only
                        // MFMAs (0x8) and LDS reads (0x100) may move across
                        __builtin_amdgcn_sched_barrier(0x108);
                    }
                }
            };
            // one step: prefetch the next streamed tile, compute (and store
            // the previous tile), then put the prefetched tile in the other buffer
            // The 64-deep 256-row panel with A stored K x M runs at the 256-VGPR
            // limit: there the streamed loader's addresses are recomputed each
            // step from an opaque copy of the thread index instead of being kept
            // live (and spilled) across the walk.
            constexpr bool TIGHT = AT && T::KMAX == 64 && T::BM == 256;
            auto step_fn = [&](int step, f16v (&acc_c)[T::TM][T::TN],
                               const f16v (&acc_s)[T::TM][T::TN], bool store) {
                const int buf = step & 1;
                const int ts_next = s_tile(step + 1 < run ? step + 1 : step);
                int tid_s = tid;
                if constexpr (TIGHT) asm volatile("" : "+v"(tid_s));
                s_load(ts_next, tid_s);
                tile_step(acc_c, sA[PB ? buf : 0], sB[PB ? 0 : buf], acc_s,
                          store ? s_tile(step - 1) : 0, store);
                if constexpr (TIGHT) asm volatile("" : "+v"(tid_s));
                s_store(buf ^ 1, tid_s);
                __syncthreads();
            };

            step_fn(0, acc0, acc1, false);
            int step = 1;
            for (; step + 1 < run; step += 2) {
                step_fn(step, acc1, acc0, true);
                step_fn(step + 1, acc0, acc1, true);
            }
            if (step < run) {
                step_fn(step, acc1, acc0, true);
#pragma unroll
                for (int q = 0; q < NST; ++q) store_one(acc1, q, s_tile(step));
            } else {
#pragma unroll
                for (int q = 0; q < NST; ++q) store_one(acc0, q, s_tile(run - 1));
            }
            continue;
        }

        for (int step = 0; step < run; ++step) {
            const int buf = step & 1;
            const int ts = s_tile(step);
            // unconditional prefetch (the last step re-reads its own tile, never
            // used) so each load is awaited in the step that issued it
            s_load(s_tile(step + 1 < run ? step + 1 : step), tid);
            const float* const As = sA[PB ? buf : 0];
            const float* const Bs = sB[PB ? 0 : buf];

            f16v acc[T::TM][T::TN];
#pragma unroll
            for (int i = 0; i < T::TM; ++i)
#pragma unroll
                for (int j = 0; j < T::TN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
#pragma unroll
            for (int kb = 0; kb < T::KMAX / 8; ++kb) {
                if (kb < nkb) {
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
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[j][s], a[i][s],
                                                                                 acc[i][j], 0, 0, 0);
                }
            }

            // the next streamed tile goes to LDS before this tile's stores are
            // issued (see the file comment: waits then never cover fresh stores)
            s_store(buf ^ 1, tid);

            // block (i, j) holds C^T: lane l owns row l%32, registers 4g..4g+3
            // its columns 8g + 4*half .. +3
            const int m0 = tile_m0(ts), n0 = tile_n0(ts);
#pragma unroll
            for (int i = 0; i < T::TM; ++i)
#pragma unroll
                for (int j = 0; j < T::TN; ++j)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int row = m0 + wm * T::WM + i * 32 + (lane & 31);
                        const int col = n0 + wn * T::WN + j * 32 + g * 8 + half * 4;
                        if (row >= p.M) continue;
                        f4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                acc[i][j][4 * g + 3]};
                        if (add_bias) v += bias_r[i];
                        float* dst = C + (int64_t)row * p.ldc + col;
                        if (c_vec && col + 3 < p.N) {
                            *reinterpret_cast<f4*>(dst) = v;
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (col + e < p.N) dst[e] = v[e];
                        }
                    }

            __syncthreads();
        }
    }
}

template <class T, bool AT, bool BT, int VEC, bool BIAS = false>
hipError_t launch_panel_one(const GemmLaunch& g, hipStream_t s) {
    const GemmParams p = make_params(g);
    dim3 grid((unsigned)g.grid_x, 1u, (unsigned)g.batch);
    hipLaunchKernelGGL((gemm_f32_panel_kernel<T, AT, BT, VEC, BIAS>), grid, dim3(T::NT), 0, s, p);
    return hipGetLastError();
}

template <bool AT, bool BT>
hipError_t launch_panel(const GemmLaunch& g, hipStream_t s) {
    if constexpr (!AT && !BT) {
        if (g.bias != nullptr) {
            if (g.cfg == kCfgPanel32)
                return g.vec == 4 ? launch_panel_one<Panel32, AT, BT, 4, true>(g, s)
                                  : launch_panel_one<Panel32, AT, BT, 1, true>(g, s);
            if (g.cfg == kCfgPanel128x64)
                return g.vec == 4 ? launch_panel_one<Panel128x64, AT, BT, 4, true>(g, s)
                                  : launch_panel_one<Panel128x64, AT, BT, 1, true>(g, s);
            return g.vec == 4 ? launch_panel_one<Panel64, AT, BT, 4, true>(g, s)
                              : launch_panel_one<Panel64, AT, BT, 1, true>(g, s);
        }
    }
    if (g.cfg == kCfgPanel32)
        return g.vec == 4 ? launch_panel_one<Panel32, AT, BT, 4>(g, s)
                          : launch_panel_one<Panel32, AT, BT, 1>(g, s);
    if (g.cfg == kCfgPanel64B)
        return g.vec == 4 ? launch_panel_one<Panel64B, AT, BT, 4>(g, s)
                          : launch_panel_one<Panel64B, AT, BT, 1>(g, s);
    if (g.cfg == kCfgPanel128x64)
        return g.vec == 4 ? launch_panel_one<Panel128x64, AT, BT, 4>(g, s)
                          : launch_panel_one<Panel128x64, AT, BT, 1>(g, s);
    return g.vec == 4 ? launch_panel_one<Panel64, AT, BT, 4>(g, s)
                      : launch_panel_one<Panel64, AT, BT, 1>(g, s);
}

}  // namespace mi
