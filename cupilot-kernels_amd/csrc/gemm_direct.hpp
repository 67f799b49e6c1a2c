// gemm_direct.hpp -- the 256 x 256 and 128 x 128 contractions (all four
// operand layouts) with global -> LDS direct loads (gfx950
// buffer_load_dwordx4 ... lds), for dense problems whose slices are all full
// (K a multiple of the slice depth, 16-byte aligned operands) and deep enough
// (direct_ok).
//
// Same tiles, waves and MFMA order as gemm_f32_kernel<Tile256> /
// <Tile128> (so the same results, bit for bit); what changes is the staging
// and, with it, the order of rows / columns within a wave's MN-contiguous
// blocks.  The layouts below are given for the 256 tile's 32-deep slices; the
// 128 tile's 16-deep ones follow the same rules (4 chunks per K-contiguous
// row, swizzled by (mn / 4) % 4; two 128-float k-rows per MN-contiguous
// instruction).  Each lane's
// 16-byte global load lands in LDS at (wave's LDS base + 16 * lane) without
// passing through VGPRs, so
//   * no VGPRs hold the next slice (32 per lane in the register-staged kernel),
//   * no ds_write instructions, and no wait for the loads before the MFMAs
//     of the current slice end: the single barrier per slice (which waits for
//     the wave's own loads first) publishes the whole next slice.
// A wave's 64 lanes fill 1 KiB of contiguous LDS, which fixes the layouts:
//   K-contiguous operand: [mn][32] with the 16-byte chunks of row mn stored
//     at chunk (q ^ ((mn / 2) % 8)); a lane chooses which global chunk it
//     loads so that its fixed LDS slot holds the right one.  A fragment read
//     (32 consecutive rows at one chunk) then puts any 16 consecutive rows --
//     2 rows per 256 bytes of banks -- in 16 different 16-byte bank groups:
//     no conflicts, no padding.  (Swizzling by mn % 8 instead left rows r and
//     r + 8 in one bank group: rocprof counted LDS bank-conflict stalls on
//     40-50 % of the LDS-active cycles of the N/N and N/T kernels.)
//   MN-contiguous operand: [32][256 + 4], one k-row per wave instruction
//     (the +4 padding sits between rows, where each instruction's base is
//     free).  k-row k = 4 g + s sits at LDS row 8 s + g.
// MN-contiguous fragments are read as pairs of adjacent rows / columns: two
// 32-wide MFMA blocks are interleaved (block t holds c0 + 2 i + t, i < 32),
// so one 8-byte read per k gives a lane its value in both blocks.  With the
// row order above, the reads of one pair are >= 2080 bytes apart, more than
// a ds_read2_b64 offset reaches, so the compiler cannot merge them (merged
// reads of this kind were given a full vmcnt(0) wait -- the wait inserter no
// longer told the buffer being read from the one the next slice's direct
// loads are writing).
// Rows / columns past the matrix edge are loaded from the last valid row /
// column instead (they only feed outputs that are never stored); K has no
// tail here, so every loaded k is real.
#pragma once

#include <type_traits>

#include "gemm_kernel.hpp"

namespace mi {

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// Raw buffer descriptor at `base` (dword 3 of the gfx9 format: untyped
// dwords).  The range check is off (num_records = 2^32 - 1): every offset a
// caller passes stays inside its operand by construction.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, -1, 0x00020000);
}

// One wave instruction, 4 bytes per lane: lane l's float at byte offset voff
// lands in LDS at lds + 4 l.
__device__ __forceinline__ void load_lds4(__amdgpu_buffer_rsrc_t r, uint32_t voff, float* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_ptr)(lds), 4, (int)voff, 0, 0, 0);
}

// One wave instruction: lane l's 16 bytes at byte offset voff from the
// descriptor's base land in LDS at lds + 16 l.  (The buffer form, not
// global_load_lds: a pending FLAT-encoded LDS load forces every LDS-read wait
// behind it down to lgkmcnt(0).)
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, float* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_ptr)(lds), 16, (int)voff, 0, 0, 0);
}

// One operand of a ROWS x BK slice (256 x 32 or 128 x 16), staged directly
// into LDS by NW waves, VB bytes per lane and instruction: 16 (16-byte
// aligned operands whose slices are all full) or 4 (any operand; the last
// slice of a K range may be partial).  The LDS layout is the same for both,
// so the fragment reads are too.
template <bool KCONTIG, int NW, int ROWS = 256, int BK = 32, int VB = 16>
struct DirectLoader {
    static_assert((ROWS == 256 && BK == 32) || (ROWS == 128 && BK == 16) ||
                      (ROWS == 128 && BK == 32 && VB == 16) ||
                      (ROWS == 64 && BK == 64 && VB == 16) ||
                      (ROWS == 512 && BK == 32 && KCONTIG && VB == 16),
                  "slice shapes built");
    static_assert(VB == 16 || VB == 4, "dwordx4 or dword loads");
    // K-contiguous: a row is CH 16-byte chunks, swizzled; RPW rows share one
    // 256-byte window of the 64 banks.
    static constexpr int CH = BK / 4, RPW = 64 / BK;
    // MN-contiguous: LDS rows of ROWS floats, KPI rows (1 KiB) followed by 4
    // floats of padding (MN-contiguous slices have at most 256 rows; the
    // 512-row K-contiguous shape never uses KPI).
    static constexpr int KPI = ROWS <= 256 ? 256 / ROWS : 1, IPITCH = KPI * ROWS + 4;
    // floats one wave instruction writes (64 lanes x VB bytes)
    static constexpr int IFL = 16 * VB;
    static constexpr int INSTR = KCONTIG ? ROWS * BK / IFL : BK * (VB == 16 ? 1 : ROWS / 64) / (VB == 16 ? KPI : 1);
    static constexpr int ELEMS = KCONTIG ? ROWS * BK : (BK / KPI) * IPITCH;
    static_assert(INSTR % NW == 0, "instructions must split evenly over the waves");
    static constexpr int PER_WAVE = INSTR / NW;

    // MN-contiguous layout: LDS row rho holds k-row k_of(rho), where k =
    // 4 g + s sits at rho = (BK / 4) s + g, so the four reads of one fragment
    // (s = 0..3) are >= 2080 bytes apart.
    __device__ __forceinline__ static constexpr int k_of(int rho) {
        return 4 * (rho % (BK / 4)) + rho / (BK / 4);
    }
    __device__ __forceinline__ static constexpr int row_base(int rho) {
        return (rho / KPI) * IPITCH + (rho % KPI) * ROWS;
    }
    // LDS float offset written by wave instruction ins (lane l adds VB/4 l)
    __device__ __forceinline__ static constexpr int dest(int ins) {
        if (KCONTIG) return ins * IFL;
        if (VB == 16) return ins * IPITCH;
        return row_base(ins / (ROWS / 64)) + (ins % (ROWS / 64)) * 64;
    }

    // Byte offsets, from a slice's origin, of this wave's loads for the tile
    // at mn0 (the same for every full slice of the tile, so computed once per
    // tile).  klim < BK (a partial last slice, VB == 4 only): k-rows / columns
    // at or past klim are read from klim - 1 instead, so every address stays
    // inside the operand (the fragments of those k are zeroed).  They fit 32
    // bits: direct_ok bounds ld.
    __device__ __forceinline__ static void offsets(int64_t ld, int mn0, int mn_ext, int wave,
                                                   int lane, uint32_t (&vo)[PER_WAVE],
                                                   int klim = BK) {
        const uint32_t ld4 = (uint32_t)ld * 4u;
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
            const int ins = wave * PER_WAVE + i;
            if (KCONTIG) {
                int r, k;
                if (VB == 16) {
                    r = ins * (64 / CH) + lane / CH;            // tile row this lane fills
                    k = 4 * ((lane % CH) ^ ((r / RPW) % CH));  // global chunk for its slot
                } else {
                    r = ins * (64 / BK) + lane / BK;
                    const int e = lane % BK;  // float within the row's LDS slots
                    k = 4 * ((e / 4) ^ ((r / RPW) % CH)) + (e & 3);
                    k = k < klim ? k : klim - 1;
                }
                const int rr = mn0 + r < mn_ext ? r : mn_ext - 1 - mn0;
                vo[i] = (uint32_t)rr * ld4 + (uint32_t)k * 4u;
            } else {
                int k, c;
                if (VB == 16) {
                    constexpr int LPR = ROWS / 4;  // lanes per k-row
                    k = k_of(ins * KPI + lane / LPR);
                    // (mn_ext - mn0 is a positive multiple of 4: vec4 operands)
                    const int c0 = (lane % LPR) * 4;
                    c = mn0 + c0 + 3 < mn_ext ? c0 : mn_ext - 4 - mn0;
                } else {
                    k = k_of(ins / (ROWS / 64));
                    k = k < klim ? k : klim - 1;
                    const int c0 = (ins % (ROWS / 64)) * 64 + lane;
                    c = mn0 + c0 < mn_ext ? c0 : mn_ext - 1 - mn0;
                }
                vo[i] = (uint32_t)k * ld4 + (uint32_t)c * 4u;
            }
        }
    }

    // Issue this wave's loads of the slice at (mn0, k0) into `lds`; per
    // slice only the (scalar) descriptor base moves.
    __device__ __forceinline__ static void load(const float* __restrict__ base, int64_t ld, int mn0,
                                                int k0, const uint32_t (&vo)[PER_WAVE], float* lds,
                                                int wave) {
        const __amdgpu_buffer_rsrc_t rsrc =
            raw_rsrc(KCONTIG ? base + (int64_t)mn0 * ld + k0 : base + (int64_t)k0 * ld + mn0);
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
            const int ins = wave * PER_WAVE + i;
            if (VB == 16)
                load_lds16(rsrc, vo[i], lds + dest(ins));
            else
                load_lds4(rsrc, vo[i], lds + dest(ins));
        }
    }

    // The buffer descriptor of the slice at (mn0, k0), and load i (< PER_WAVE)
    // of this wave's share of it: for callers that spread a slice's loads
    // between other instructions.
    __device__ __forceinline__ static __amdgpu_buffer_rsrc_t slice_rsrc(const float* __restrict__ base,
                                                                        int64_t ld, int mn0, int k0) {
        return raw_rsrc(KCONTIG ? base + (int64_t)mn0 * ld + k0 : base + (int64_t)k0 * ld + mn0);
    }
    __device__ __forceinline__ static void load_one(__amdgpu_buffer_rsrc_t rsrc, const uint32_t (&vo)[PER_WAVE],
                                                    float* lds, int wave, int i) {
        const int ins = wave * PER_WAVE + i;
        if (VB == 16)
            load_lds16(rsrc, vo[i], lds + dest(ins));
        else
            load_lds4(rsrc, vo[i], lds + dest(ins));
    }

    // K-contiguous operand: values for the 4 MFMA steps of k-block kb,
    // 32-row group at r0 (same k permutation as TileLoader::frag:
    // k = 8 kb + 4 h + s).
    __device__ __forceinline__ static void frag(const float* lds, int r0, int kb, int lane,
                                                float out[4]) {
        static_assert(KCONTIG, "MN-contiguous fragments are read in pairs");
        const int half = lane >> 5;
        const int l32 = lane & 31;
        const int row = r0 + l32;
        // r0 % 16 == 0, so (row / RPW) % CH = (l32 / RPW) % CH
        const int q = (2 * kb + half) ^ ((l32 / RPW) % CH);
        const f4 t = *reinterpret_cast<const f4*>(lds + row * BK + q * 4);
        out[0] = t[0];
        out[1] = t[1];
        out[2] = t[2];
        out[3] = t[3];
    }

    // MN-contiguous operand, four blocks at once: values for the 4 MFMA steps
    // of k-block kb in the four interleaved blocks of the 128 columns at c0
    // (block t, lane i: column c0 + 4 i + t), one 16-byte read per step.
    __device__ __forceinline__ static void frag_quad(const float* lds, int c0, int kb, int lane,
                                                     float out[4][4]) {
        static_assert(!KCONTIG, "K-contiguous fragments are read one block at a time");
        const int g = 2 * kb + (lane >> 5);  // k = 4 g + s
        const int col = c0 + 4 * (lane & 31);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const f4 t = *reinterpret_cast<const f4*>(lds + row_base(s * (BK / 4) + g) + col);
#pragma unroll
            for (int b = 0; b < 4; ++b) out[b][s] = t[b];
        }
    }

    // MN-contiguous operand: values for the 4 MFMA steps of k-block kb in the
    // two interleaved blocks of the 64 columns at c0 (block t, lane i: column
    // c0 + 2 i + t).
    __device__ __forceinline__ static void frag_pair(const float* lds, int c0, int kb, int lane,
                                                     float out[2][4]) {
        static_assert(!KCONTIG, "K-contiguous fragments are read one block at a time");
        const int g = 2 * kb + (lane >> 5);  // k = 4 g + s
        const int col = c0 + 2 * (lane & 31);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const f2 t = *reinterpret_cast<const f2*>(lds + row_base(s * (BK / 4) + g) + col);
            out[0][s] = t[0];
            out[1][s] = t[1];
        }
    }
};

// Epilogue.  An MN-contiguous operand's 32-wide blocks are interleaved in
// pairs (frag_pair), which moves its rows / columns:
//   A (rows):    block i = 2 u + t, lane l -> row 64 u + 2 (l % 32) + t;
//                with four row blocks per wave (frag_quad) block i = 4 u + t,
//                lane l -> row 128 u + 4 (l % 32) + t;
//                K-contiguous A: block i, lane l -> row 32 i + l % 32.
//   B (columns): register r of the swapped-operand MFMA is block column
//                i' = 8 (r / 4) + 4 (l / 32) + r % 4; interleaved B puts it at
//                column 2 i' + t of block t, so for each r / 4 a lane holds 8
//                consecutive columns (two 16-byte stores); K-contiguous B puts
//                it at 32 j + i' (4 consecutive columns per r / 4).
//
// Triangular modes write +0.0 on the wrong side of the diagonal, except for a
// chunk whose partial sum goes to the mirror tile: it is stored unmasked at
// (tn, tm) -- the same offsets within the tile -- for tri_finish to add in.
// LOCAL: C points at a BM x BN workspace tile (row stride ldc) that receives
// the tile's elements at their offsets within the tile (a stream-K partial);
// rows and columns past M / N are still skipped.
template <class T, bool A_IL, bool B_IL, bool BIAS, int MODE, bool LOCAL = false>
__device__ __forceinline__ void store_tile_direct(const GemmParams& p, float* C, int64_t ldc,
                                                  bool c_vec, const TileWork& w,
                                                  const f16v (&acc)[T::TM][T::TN], int wm, int wn,
                                                  int lane) {
    static_assert(!B_IL || T::TN % 2 == 0, "column blocks interleave in pairs");
    static_assert(!A_IL || T::TM % 2 == 0, "row blocks pair up");
    constexpr bool A_QUAD = A_IL && T::TM % 4 == 0;  // frag_quad's interleave
    const bool to_mirror = MODE != kDense && w.mirror;
    const bool tri_mask = MODE != kDense && !w.mirror;
    const int r0 = (to_mirror ? w.tn : w.tm) * T::BM;
    const int c0 = (to_mirror ? w.tm : w.tn) * T::BN;
    const int l32 = lane & 31;
    const int cw = c0 + wn * T::WN + (lane >> 5) * 4;
    const bool add_bias = BIAS && p.split_k == 1;
#pragma unroll
    for (int i = 0; i < T::TM; ++i) {
        const int row = r0 + wm * T::WM +
                        (A_QUAD ? 128 * (i / 4) + 4 * l32 + (i & 3)
                                : A_IL ? 64 * (i / 2) + 2 * l32 + (i & 1) : 32 * i + l32);
        if (row >= p.M) continue;
        const float bv = add_bias ? p.bias[row] : 0.f;
        float* const crow = LOCAL ? C + (int64_t)(row - r0) * ldc : C + (int64_t)row * ldc;
        // one 16-byte group: columns col .. col + 3 get v
        auto put = [&](int col, f4 v) __attribute__((always_inline)) {
            if (add_bias) v += bv;
            if (tri_mask) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (MODE == kLower ? col + e > row : col + e < row) v[e] = 0.f;
            }
            float* const dst = LOCAL ? crow + (col - c0) : crow + col;
            if (c_vec && col + 3 < p.N) {
                *reinterpret_cast<f4*>(dst) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < p.N) dst[e] = v[e];
            }
        };
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (B_IL) {
#pragma unroll
                for (int u = 0; u < T::TN / 2; ++u) {  // block pair u: columns 64 u ..
                    f4 lo, hi;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        lo[2 * e] = acc[i][2 * u][4 * q + e];
                        lo[2 * e + 1] = acc[i][2 * u + 1][4 * q + e];
                        hi[2 * e] = acc[i][2 * u][4 * q + 2 + e];
                        hi[2 * e + 1] = acc[i][2 * u + 1][4 * q + 2 + e];
                    }
                    const int col = cw + 64 * u + 16 * q + (lane >> 5) * 4;  // 16 q + 8 h
                    put(col, lo);
                    put(col + 4, hi);
                }
            } else {
#pragma unroll
                for (int j = 0; j < T::TN; ++j) {
                    f4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
                    put(cw + 32 * j + 8 * q, v);
                }
            }
        }
    }
}

// Persistent like gemm_f32_kernel; per slice: issue the next slice's direct
// loads (same tile, the next tile's first slice, or -- after the workgroup's
// last slice -- this slice again, never used) into the other buffer, run this
// slice's MFMAs, barrier (which first waits for this wave's loads), and after
// a tile's last slice issue its stores.  The two LDS buffers of each operand
// are separate __shared__ objects and the slice loop is unrolled by two, so
// each access names its buffer at compile time.
//
// MODE kLower / kUpper: the chunked triangular work list (tri_item), one item
// per workgroup (grid = items, dispatched longest first).  Operand entries on
// the wrong side of the diagonal are zeroed in the fragments of the diagonal
// K unit (tril(A) tril(B) / triu(A) triu(B) for any input).
//
// SK: the stream-K schedule (sk_item): workgroup b runs its items 0, 1, ...
// -- whole tiles, then its stream-K segments -- and stores a segment that
// does not start at k = 0 into that segment's workspace slot, tile-local,
// for sk_fixup to add in.  With 4-byte
// staging (128 tile) a tile's last slice may be partial: the segment that
// holds it ends at K.
template <class T, bool AT, bool BT, bool BIAS, int MODE = kDense, int VB = 16, bool SK = false>
__global__ void __launch_bounds__(T::NT)
    __attribute__((amdgpu_waves_per_eu(T::WAVES_PER_SIMD, T::WAVES_PER_SIMD)))
    gemm_f32_direct_kernel(const GemmParams p) {
    static_assert(T::STAGES == 2 && T::BM == T::BN, "double-buffered square tiles");
    static_assert(MODE == kDense || (!AT && !BT && T::BM == 256 && VB == 16),
                  "triangular products are N/N on the 256 tile");
    static_assert(!SK || (MODE == kDense && !BIAS && (VB == 16 || T::BM == 128)),
                  "stream-K: dense, no bias; 4-byte staging on the 128 tile only");
    constexpr bool A_KC = !AT;  // A row-major (M x K) is contiguous along K
    constexpr bool B_KC = BT;   // B stored N x K is contiguous along K
    using LA = DirectLoader<A_KC, T::NW, T::BM, T::BK, VB>;
    using LB = DirectLoader<B_KC, T::NW, T::BN, T::BK, VB>;
    __shared__ __attribute__((aligned(16))) float sA0[LA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sA1[LA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB0[LB::ELEMS];
    __shared__ __attribute__((aligned(16))) float sB1[LB::ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform, made scalar so LDS destinations (M0) need no readfirstlane
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Triangular modes: the two waves on a SIMD (waves w and w + 4) own
    // different column blocks, so when the diagonal masks leave whole waves
    // without work (idle) both halves of the machine shed work together.
    const int wm = wave / T::WAVES_N;
    const int wn = MODE == kDense ? wave % T::WAVES_N : (wave + 2 * wm) % T::WAVES_N;
    // Batched grids (no split): the hardware deals consecutive workgroups --
    // here the gridDim.x workgroups of one batch entry -- round-robin over the
    // 8 XCDs, so a batch entry's workgroups, which walk the tile rows of the
    // same column panels in step, would share nothing in L2.  xcd_remap of the
    // linear index puts each batch entry's workgroups on one XCD.  Measured on
    // 128 x (512 x 1024 . 1024 x 768), 2 workgroups per entry, interleaved
    // over 3 rounds: 0.755-0.759 vs 0.761-0.768 ms.
    int bx = blockIdx.x, batch = blockIdx.z;
    if (!SK && MODE == kDense && gridDim.z > 1 && gridDim.y == 1) {
        const int lin = blockIdx.x + gridDim.x * blockIdx.z;
        const int L = xcd_remap(lin, gridDim.x * gridDim.z);
        bx = L % gridDim.x;
        batch = L / gridDim.x;
    }

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

    // load offsets of the tile whose slices are being issued
    uint32_t voA[LA::PER_WAVE], voB[LB::PER_WAVE];
    auto set_offsets = [&](const TileWork& w) __attribute__((always_inline)) {
        LA::offsets(p.lda, w.tm * T::BM, p.M, wave, lane, voA);
        LB::offsets(p.ldb, w.tn * T::BN, p.N, wave, lane, voB);
    };
    auto issue = [&](const TileWork& w, int it, float* dA, float* dB) __attribute__((always_inline)) {
        const int k0 = w.k_begin + it * T::BK;
        if constexpr (VB == 4) {
            if (k0 + T::BK > w.k_end) {  // partial last slice: offsets clamped to the K range
                uint32_t tA[LA::PER_WAVE], tB[LB::PER_WAVE];
                LA::offsets(p.lda, w.tm * T::BM, p.M, wave, lane, tA, w.k_end - k0);
                LB::offsets(p.ldb, w.tn * T::BN, p.N, wave, lane, tB, w.k_end - k0);
                LA::load(A, p.lda, w.tm * T::BM, k0, tA, dA, wave);
                LB::load(B, p.ldb, w.tn * T::BN, k0, tB, dB, wave);
                return;
            }
        }
        LA::load(A, p.lda, w.tm * T::BM, k0, voA, dA, wave);
        LB::load(B, p.ldb, w.tn * T::BN, k0, voB, dB, wave);
    };
    auto decode = [&](int item) __attribute__((always_inline)) -> TileWork {
        if constexpr (SK) {
            // compute = 0: past the workgroup's last item
            TileWork w;
            int lt, s0, s1;
            int64_t slot;
            w.compute = sk_item(blockIdx.x, item, gridDim.x, p.sk_dp, p.sk_tiles, p.sk_ipt,
                                p.sk_ph, p.sk_nph, lt, s0, s1, slot)
                            ? 1
                            : 0;
            if (!w.compute) {
                lt = s0 = s1 = 0;
                slot = -1;
            }
            raster(lt, p.tiles_m, p.tiles_n, p.group_m, w.tm, w.tn);
            w.k_begin = s0 * T::BK;
            // (4-byte staging: the tile's last slice may end past K)
            w.k_end = s1 * T::BK < p.K ? s1 * T::BK : p.K;
            w.nk = s1 - s0;
            w.mirror = slot >= 0;
            w.slot = slot >= 0 ? (int)slot : 0;
            return w;
        } else if constexpr (MODE == kDense) {
            return decode_tile<T, kDense>(p, item);
        } else {
            TileWork w;
            int u0, u1;
            tri_item(item, p.tiles_m, p.tri_cap, MODE == kLower, w.tm, w.tn, u0, u1, w.mirror);
            // (the work list is planned only for N a multiple of 256)
            w.k_begin = u0 * T::BM;
            w.k_end = u1 * T::BM;
            w.nk = (w.k_end - w.k_begin) / T::BK;
            w.compute = 1;
            return w;
        }
    };
    // fragments of one k-block, kept at kernel scope (two sets, by k-block parity)
    float fa[2][T::TM][4], fb[2][T::TN][4];
    // Triangular modes: the slice lies in one K unit; in the unit of A's row
    // tile (mask_a) / B's column tile (mask_b) entries past the diagonal are
    // set to +0.0 in LDS (zero_masked) before any fragment of the slice is
    // read.  kl0 = the slice's first k within that unit.
    int mask_a = 0, mask_b = 0, kl0 = 0;
    // the wave's fragments of the slice are all zero (masked): its MFMAs are
    // skipped (they would add exact zeros)
    int idle = 0;
    // VB == 4: k of the slice being computed that are in range (< BK only in
    // a partial last slice, whose fragments past it are zeroed)
    int kv = T::BK;
    // (every lambda here is force-inlined: a call would pass the accumulators
    // through scratch memory)
    auto frags = [&](const float* As, const float* Bs, int kb) __attribute__((always_inline)) {
        if constexpr (A_KC) {
#pragma unroll
            for (int i = 0; i < T::TM; ++i) LA::frag(As, wm * T::WM + i * 32, kb, lane, fa[kb & 1][i]);
        } else if constexpr (T::TM % 4 == 0) {  // four row blocks per 16-byte read
#pragma unroll
            for (int u = 0; u < T::TM / 4; ++u)
                LA::frag_quad(As, wm * T::WM + u * 128, kb, lane, fa[kb & 1] + 4 * u);
        } else {
#pragma unroll
            for (int u = 0; u < T::TM / 2; ++u)
                LA::frag_pair(As, wm * T::WM + u * 64, kb, lane, fa[kb & 1] + 2 * u);
        }
        if constexpr (B_KC) {
#pragma unroll
            for (int j = 0; j < T::TN; ++j) LB::frag(Bs, wn * T::WN + j * 32, kb, lane, fb[kb & 1][j]);
        } else {
#pragma unroll
            for (int u = 0; u < T::TN / 2; ++u)
                LB::frag_pair(Bs, wn * T::WN + u * 64, kb, lane, fb[kb & 1] + 2 * u);
        }
        if constexpr (VB == 4) {
            if (kv < T::BK) {
                const int klb = 8 * kb + 4 * (lane >> 5);  // + s
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    if (klb + s >= kv) {
#pragma unroll
                        for (int i = 0; i < T::TM; ++i) fa[kb & 1][i][s] = 0.f;
#pragma unroll
                        for (int j = 0; j < T::TN; ++j) fb[kb & 1][j][s] = 0.f;
                    }
                }
            }
        }
    };
    // Triangular modes, a slice in a masked unit, once its loads have landed
    // (after the barrier) and before any of its fragments are read: +0.0 over
    // the entries past the diagonal, so the fragment reads and MFMAs are the
    // dense kernel's.  (Zeroing the fragments in registers instead put compare
    // and select code after every k-block's fragment reads, masked unit or
    // not: full units ran ~5 % slower than the dense kernel's.)  The slice is
    // N/N: A K-contiguous (row r: 32 floats, 16-byte chunk g at slot
    // g ^ (r / 2) % 8), B MN-contiguous (k-row k at LDS row 8 (k % 4) + k / 4,
    // rows of 256 floats + 4 padding).  A(m, k): lower keeps k <= m, upper
    // k >= m; B(k, n): lower keeps n <= k, upper n >= k.
    auto zero_masked = [&](float* As, float* Bs) __attribute__((always_inline)) {
        if constexpr (MODE != kDense) {
            static_assert(A_KC && !B_KC && T::BM == 256 && T::BK == 32, "N/N 256 x 32 slices");
            if (mask_a) {
#pragma unroll
                for (int q = 0; q < 256 * 8 / T::NT; ++q) {
                    const int c = tid + q * T::NT;
                    const int r = c >> 3, g = c & 7;
                    const int k0 = kl0 + 4 * g;  // unit-local k of the chunk's first entry
                    float* const ptr = As + r * 32 + ((g ^ ((r >> 1) & 7)) << 2);
                    if (MODE == kLower ? k0 > r : k0 + 3 < r) {
                        *reinterpret_cast<f4*>(ptr) = f4{0.f, 0.f, 0.f, 0.f};
                    } else if (MODE == kLower ? k0 + 3 > r : k0 < r) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (MODE == kLower ? k0 + e > r : k0 + e < r) ptr[e] = 0.f;
                    }
                }
            }
            if (mask_b) {
#pragma unroll
                for (int q = 0; q < 32 * 64 / T::NT; ++q) {
                    const int c = tid + q * T::NT;
                    const int kr = c >> 6, n0 = (c & 63) * 4;
                    const int k = kl0 + kr;  // unit-local k of this k-row
                    float* const ptr = Bs + (8 * (kr & 3) + (kr >> 2)) * LB::IPITCH + n0;
                    if (MODE == kLower ? n0 > k : n0 + 3 < k) {
                        *reinterpret_cast<f4*>(ptr) = f4{0.f, 0.f, 0.f, 0.f};
                    } else if (MODE == kLower ? n0 + 3 > k : n0 < k) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (MODE == kLower ? n0 + e > k : n0 + e < k) ptr[e] = 0.f;
                    }
                }
            }
        }
    };
    // Per slice: the next slice's loads, then for each k-block the next
    // k-block's fragment reads ahead of this k-block's MFMAs (scheduling
    // barriers keep that order).  With full 16-byte slices the loads are
    // spread: part(s) after MFMA step s of the first k-block, so a wave does
    // not stall on the address unit with all of them at once while its
    // SIMD's MFMA pipe drains (8192^3 N/N +0.5 %, N/T +1.2 %, T/N and T/T
    // +0.3 % once MN-contiguous A takes frag_quad; before that, spreading
    // A's loads cost those two layouts 0.5 %).  The last k-block's s = 2, 3 MFMAs are held
    // back until after the slice barrier (tail), where they cover the latency
    // of the next slice's first fragment reads, issued right after the
    // barrier; so the slice's first k-block fragments are already in
    // registers (set 0) when compute starts.
    constexpr int NKB = T::BK / 8;
    constexpr bool SPREAD = VB == 16 && NKB >= 2;
    // wave priority across the slice barrier (see there): the 256 tile; with
    // a row-major B the 8-wave 128 tile and the 32-deep 128 tile's stream-K
    // kernel; the 128 tile's stream-K kernels and its 4-byte staging
    constexpr bool PRIO = T::BM == 256 || (std::is_same<T, Tile128W8>::value && !B_KC) ||
                          (std::is_same<T, Tile128B32>::value && !B_KC && SK) ||
                          (std::is_same<T, Tile128>::value && (SK || VB == 4));
    auto compute = [&](const float* As, const float* Bs, auto&& loads, auto&& part) __attribute__((always_inline)) {
        if constexpr (!SPREAD) loads();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const int set = kb & 1;
            if (kb + 1 < NKB) frags(As, Bs, kb + 1);
            __builtin_amdgcn_sched_barrier(0);
            if (MODE == kDense || !idle) {
#pragma unroll
                for (int s = 0; s < (kb + 1 < NKB ? 4 : 2); ++s) {
#pragma unroll
                    for (int i = 0; i < T::TM; ++i)
#pragma unroll
                        for (int j = 0; j < T::TN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                fb[set][j][s], fa[set][i][s], acc[i][j], 0, 0, 0);
                    if (SPREAD && kb == 0) {
                        __builtin_amdgcn_sched_barrier(0);
                        part(s);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            } else if (SPREAD && kb == 0) {  // an idle wave still issues its loads
#pragma unroll
                for (int s = 0; s < 4; ++s) part(s);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto tail = [&](int skip) __attribute__((always_inline)) {
        constexpr int set = (NKB - 1) & 1;
        if (MODE != kDense && skip) return;
#pragma unroll
        for (int s = 2; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < T::TM; ++i)
#pragma unroll
                for (int j = 0; j < T::TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[set][j][s], fa[set][i][s],
                                                                     acc[i][j], 0, 0, 0);
    };

    // per-slice fragment masks of slice i of tile w (read by frags)
    auto slice_state = [&](const TileWork& w, int i) __attribute__((always_inline)) {
        if constexpr (VB == 4) {
            const int left = w.k_end - (w.k_begin + i * T::BK);
            kv = left < T::BK ? left : T::BK;
        }
        if constexpr (MODE != kDense) {
            const int k0 = w.k_begin + i * T::BK;
            const int unit = k0 / T::BM;
            mask_a = unit == w.tm;
            mask_b = unit == w.tn;
            kl0 = k0 - unit * T::BM;
            // slice k range [kl0, kl0 + BK) against the wave's rows (A masked:
            // lower keeps k <= m, upper k >= m) and columns (B masked: lower
            // keeps n <= k, upper n >= k)
            const int r0 = wm * T::WM, c0 = wn * T::WN;
            const bool a_idle = MODE == kLower ? kl0 > r0 + T::WM - 1 : kl0 + T::BK - 1 < r0;
            const bool b_idle = MODE == kLower ? c0 > kl0 + T::BK - 1 : c0 + T::WN - 1 < kl0;
            idle = (mask_a && a_idle) || (mask_b && b_idle);
        }
    };

    // Triangular work list, dynamic order: persistent workgroups take the
    // next item of the longest-first list from a counter as they finish one,
    // so XCDs that run faster take more items.  The counter is the first word
    // of zero-triangle tile (0, 1) (lower; (1, 0) upper): with cap >= 2 it is
    // never a mirror tile, the launcher zeroes the word first and the
    // finishing pass zeroes the tile.  One thread claims the next item at the
    // current item's second-to-last slice (as late as the one-slice load
    // lookahead allows: a claim made earlier would reserve the item for a
    // workgroup still busy), through LDS: written after every wave has read
    // the previous value (items have >= 8 slices), read at the last slice.
    const bool dyn = MODE != kDense && p.tri_cap >= 2;
    __shared__ int s_item;
    int* const ctr = MODE == kLower ? reinterpret_cast<int*>(p.C + 256)
                                    : reinterpret_cast<int*>(p.C + 256 * p.ldc);
    // Past the compute items the counter hands out the zero-triangle tiles
    // of tri_zero_tile (tiles with no parked partial): a workgroup writes
    // +0.0 over each it claims, so the tail of the list, when CUs run out of
    // compute items, does the stores the finishing pass would do after the
    // kernel.
    auto zero_items = [&](int z) __attribute__((always_inline)) {
        if constexpr (MODE != kDense) {
            const int total = p.num_tiles + tri_zero_items(p.tiles_m, p.tri_cap);
            while (z < total) {
                int zm, zn;
                tri_zero_tile(z - p.num_tiles, p.tiles_m, MODE == kLower, zm, zn);
                float* const z0 = C + (int64_t)zm * T::BM * ldc + (int64_t)zn * T::BN;
#pragma unroll 4
                for (int e = tid; e < T::BM * (T::BN / 4); e += T::NT) {
                    float* const d = z0 + (int64_t)(e / (T::BN / 4)) * ldc + (e % (T::BN / 4)) * 4;
                    if (c_vec) {
                        *reinterpret_cast<f4*>(d) = f4{0.f, 0.f, 0.f, 0.f};
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q) d[q] = 0.f;
                    }
                }
                __syncthreads();  // every wave has read s_item
                if (tid == 0) s_item = atomicAdd(ctr, 1);
                __syncthreads();
                z = s_item;
            }
        }
    };
    int t = SK ? 0 : bx;
    if (dyn) {
        if (tid == 0) s_item = atomicAdd(ctr, 1);
        __syncthreads();
        t = s_item;
        if (t >= p.num_tiles) {
            zero_items(t);
            return;
        }
    }
    if (!SK && t >= p.num_tiles) return;
    TileWork cur = decode(t);
    if (SK && !cur.compute) return;
    int it = 0;
    set_offsets(cur);
    issue(cur, 0, sA0, sB0);
    __syncthreads();
    slice_state(cur, 0);
    if (MODE != kDense && (mask_a || mask_b)) {
        zero_masked(sA0, sB0);
        __syncthreads();
    }
    frags(sA0, sB0, 0);

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
        if constexpr (MODE != kDense) {
            if (dyn && it == cur.nk - 2 && tid == 0) s_item = atomicAdd(ctr, 1);
        }
        if (last) {
            if constexpr (SK) {
                nt = t + 1;
                const TileWork cand = decode(nt);
                has_next = cand.compute != 0;
                if (has_next) nw = cand;
            } else {
                nt = dyn ? s_item : t + gridDim.x;
                has_next = nt < p.num_tiles;
                if (dyn && !has_next) t = nt;  // handed on to zero_items
                if (has_next) nw = decode(nt);
            }
            nit = has_next ? 0 : it;
            if (has_next) set_offsets(nw);
        }
        // (the scheduling barriers keep the loads ahead of the MFMAs: the
        // scheduler would sink them to the barrier, exposing their latency)
        const int k0n = nw.k_begin + nit * T::BK;
        const __amdgpu_buffer_rsrc_t ra = LA::slice_rsrc(A, p.lda, nw.tm * T::BM, k0n);
        const __amdgpu_buffer_rsrc_t rb = LB::slice_rsrc(B, p.ldb, nw.tn * T::BN, k0n);
        static_assert(!SPREAD || (LA::PER_WAVE <= 4 && LB::PER_WAVE <= 4), "parts 0..3 cover every load");
        compute(curA, curB, [&]() __attribute__((always_inline)) { issue(nw, nit, nxtA, nxtB); },
                [&](int q) __attribute__((always_inline)) {
                    if (q >= 0 && q < LA::PER_WAVE) LA::load_one(ra, voA, nxtA, wave, q);
                    if (q >= 0 && q < LB::PER_WAVE) LB::load_one(rb, voB, nxtB, wave, q);
                });
        __syncthreads();
        // The 256 tile (one workgroup of 8 waves per CU) raises the waves'
        // issue priority from the barrier through the held-back MFMAs: each
        // wave, right after the barrier, gets its fragment reads and MFMAs
        // issued ahead of a SIMD-mate's lower-priority instructions, which
        // shortens the slice-boundary bubble.  Measured in one process,
        // 8192^3: N/N 151.7 vs 149.9, T/N 151.9 vs 149.2, N/T 152.3 vs 149.8,
        // T/T 151.4 vs 150.4 TFLOP/s.  (The 128 tile, three workgroups per CU
        // at different phases, lost 2.5 % that way on 65536 x 512 x 256.)
        // The 8-wave 128 tile (two workgroups per CU) gains 0.2-0.8 % with a
        // row-major B (2048 x 4096 x 8192 0.920 vs 0.926 ms, 4096 x 2048 x
        // 4096 0.465 vs 0.468, 16384 x 768 x 2048 0.355 vs 0.356) and loses
        // 0.2 % with B stored N x K, so only the former raises it.  So does
        // the 32-deep 128 tile's stream-K kernel (N/N 0.5-1.1 %, T/N 1.4-2.2 %
        // faster; N/T and T/T 0.2-0.5 % slower, and its data-parallel plans up
        // to 1.2 % slower); the 128 tile's stream-K kernels gain in every
        // layout (16-byte staging: 3072^3 N/N 0.432 vs 0.438 ms, 4608^3 1.383
        // vs 1.414; 4-byte: 4097 x 4099 x 4095 1.202 vs 1.234, 1.4-2.9 % on
        // eight unaligned shapes, N/T within noise), and so does its 4-byte
        // data-parallel kernel (1.2-2.6 % on six unaligned shapes: 3652 x 8764
        // x 1435 0.690 vs 0.700 ms); its 16-byte data-parallel kernel is the
        // one the 65536 x 512 x 256 figure above is for.
        // Measured in one process each, alternating, medians of 3.
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
        // the next slice's first k-block (fragment set 0; the held-back MFMAs
        // use set (NKB - 1) & 1 = 1), with that slice's masks
        const int tail_idle = idle;  // (slice_state below moves on to the next slice)
        if (has_next) {
            slice_state(nw, nit);
            if (MODE != kDense && (mask_a || mask_b)) {
                zero_masked(nxtA, nxtB);
                __syncthreads();
            }
            frags(nxtA, nxtB, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        tail(tail_idle);
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        if (!last) {
            ++it;
            return false;
        }
        if (SK && cur.mirror)  // stream-K: the segment's workspace slot (tile-local, BM x BN)
            store_tile_direct<T, !A_KC, !B_KC, BIAS, MODE, true>(
                p, p.ws + (int64_t)cur.slot * (T::BM * T::BN), T::BN, true, cur, acc, wm, wn, lane);
        else
            store_tile_direct<T, !A_KC, !B_KC, BIAS, MODE>(p, C, ldc, c_vec, cur, acc, wm, wn, lane);
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
    if (dyn) zero_items(t);  // t: the claim that ended the compute items
}

// Triangular N/N products on the chunked work list (the scheduler plans it
// when N is a multiple of 256 and the direct path's operand conditions hold),
// then the pass that folds the mirror partials in and zeroes the rest of the
// zero triangle.
inline hipError_t launch_direct_tri(const GemmLaunch& g, hipStream_t s) {
    const GemmParams p = make_params(g);
    if (g.tri_cap >= 2) {  // dynamic order (see the kernel): the item counter starts at 0
        float* const ctr = g.structure == kLower ? g.C + 256 : g.C + 256 * g.ldc;
        hipError_t e = launch_zero_word(ctr, s);
        if (e != hipSuccess) return e;
    }
    // the planner's grid: one persistent workgroup per CU for the dynamic
    // order, one per item otherwise
    dim3 grid((unsigned)g.grid_x, 1, 1);
    if (g.structure == kLower)
        hipLaunchKernelGGL((gemm_f32_direct_kernel<Tile256, false, false, false, kLower>), grid,
                           dim3(Tile256::NT), 0, s, p);
    else
        hipLaunchKernelGGL((gemm_f32_direct_kernel<Tile256, false, false, false, kUpper>), grid,
                           dim3(Tile256::NT), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_tri_finish(g.C, g.ldc, g.tiles_m, g.tri_cap, g.structure == kLower, g.tri_cap >= 2, s);
}

template <class T, bool AT, bool BT, int VB>
inline hipError_t launch_direct_tile(const GemmLaunch& g, hipStream_t s) {
    const GemmParams p = make_params(g);
    dim3 grid((unsigned)g.grid_x, (unsigned)g.split_k, (unsigned)g.batch);
    if constexpr (VB == 16 || T::BM == 128) {
        if (g.sk_tiles > 0) {  // stream-K (the scheduler plans it for batch 1, split 1, no bias)
            hipLaunchKernelGGL((gemm_f32_direct_kernel<T, AT, BT, false, kDense, VB, true>),
                               dim3((unsigned)g.grid_x), dim3(T::NT), 0, s, p);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            return launch_sk_fixup(g, s);
        }
    }
    if constexpr (!AT && !BT) {  // the row bias exists for N/N only
        if (g.bias != nullptr && g.split_k == 1) {
            hipLaunchKernelGGL((gemm_f32_direct_kernel<T, false, false, true, kDense, VB>), grid,
                               dim3(T::NT), 0, s, p);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemm_f32_direct_kernel<T, AT, BT, false, kDense, VB>), grid, dim3(T::NT),
                       0, s, p);
    return hipGetLastError();
}

// 16-byte direct staging (direct_ok), else 4-byte (direct4_ok); the caller
// has checked one of them.
template <bool AT, bool BT>
inline hipError_t launch_direct(const GemmLaunch& g, hipStream_t s) {
    if (!direct_ok(g)) return launch_direct_tile<Tile128, AT, BT, 4>(g, s);
    if (g.cfg == kCfg128B32) return launch_direct_tile<Tile128B32, AT, BT, 16>(g, s);
    if constexpr (!AT) {
        if (g.cfg == kCfg128W8) return launch_direct_tile<Tile128W8, AT, BT, 16>(g, s);
    }
    return g.cfg == kCfg128 ? launch_direct_tile<Tile128, AT, BT, 16>(g, s)
                            : launch_direct_tile<Tile256, AT, BT, 16>(g, s);
}

}  // namespace mi
