// mi_internal.hpp -- interface between the ABI/scheduler (host C++) and the
// kernel translation units.  Not installed; the public boundary is
// include/mi355_gemm.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mi_device.hpp"

namespace mi {

// Tile configurations of the fp32 MFMA contraction engine (v_mfma_f32_32x32x2_f32).
//   id  block (BM x BN)  waves  wave tile   LDS (double-buffered)
//   1   64 x 64          4      32 x 32     ~20 KiB
//   2   128 x 128        4      64 x 64     ~40 KiB
//   3   256 x 256        8      128 x 64    ~140 KiB (32-deep K slices)
//   4   128 x 128        4      64 x 64     ~35 KiB, one 32-deep slice (K <= 32)
//   5   128 x 128        4      64 x 64     ~68 KiB, one 64-deep slice (K <= 64)
//   6   256 x 128 panel  8      64 x 64     A panel resident, K <= 32 (~71 KiB, 1 WG/CU)
//   7   256 x 128 panel  8      64 x 64     A panel resident, K <= 64 (~137 KiB)
//   8   128 x 128 panel  8      64 x 32     A panel resident, K <= 64
//   9   128 x 128        4      64 x 64     32-deep slices, direct-staged only (~65 KiB, 2 WGs/CU)
//   10  64 x 64          8      64 x 64     each wave one 8-deep k-block of every 64-deep
//                                           slice, 4-stage direct ring (~130 KiB, 1 WG/CU)
//   11  128 x 128        8      32 x 64     32-deep slices, direct-staged, A K-contiguous
//   12  128 x 256 panel  8      64 x 64     B panel resident, A row tiles streamed,
//                                           K <= 64 (~136 KiB, 1 WG/CU), no row bias
enum TileCfgId {
    kCfg64 = 1, kCfg128 = 2, kCfg256 = 3, kCfg128K32 = 4, kCfg128K64 = 5,
    kCfgPanel32 = 6, kCfgPanel64 = 7, kCfgPanel128x64 = 8, kCfg128B32 = 9, kCfg64W = 10,
    kCfg128W8 = 11, kCfgPanel64B = 12, kNumCfg = 13
};
inline bool is_panel_cfg(int id) {
    return id == kCfgPanel32 || id == kCfgPanel64 || id == kCfgPanel128x64 || id == kCfgPanel64B;
}
// panel configs whose resident panel is B (work items: column panels)
inline bool is_panel_b_cfg(int id) { return id == kCfgPanel64B; }

struct CfgInfo {
    int bm, bn, bk, threads;
};
inline CfgInfo cfg_info(int id) {
    switch (id) {
        case kCfg64: return {64, 64, 16, 256};
        case kCfg128: return {128, 128, 16, 256};
        case kCfg256: return {256, 256, 32, 512};
        case kCfg128K32: return {128, 128, 32, 256};
        case kCfg128K64: return {128, 128, 64, 256};
        case kCfgPanel32: return {256, 128, 32, 512};
        case kCfgPanel64: return {256, 128, 64, 512};
        case kCfgPanel128x64: return {128, 128, 64, 512};
        case kCfg128B32: return {128, 128, 32, 256};
        case kCfg64W: return {64, 64, 64, 512};
        case kCfg128W8: return {128, 128, 32, 512};
        case kCfgPanel64B: return {128, 256, 64, 512};
        default: return {0, 0, 0, 0};
    }
}

// Fully resolved contraction launch (all validation done by the caller).
struct GemmLaunch {
    const float* A;
    const float* B;
    float* C;
    float* ws;            // split-K partials: split_k x batch x M x N (ld = N)
    const float* bias;    // NULL or M per-row values added after the full sum
    int M, N, K, batch;
    int64_t lda, ldb, ldc;
    int64_t sa, sb, sc;
    int op_a, op_b;       // 0 = N, 1 = T
    int structure;        // 0 dense, 1 lower, 2 upper
    int cfg;              // TileCfgId
    int vec;              // 4: 16-byte operand loads; 1: element loads
    int split_k;
    int k_chunk;
    int tiles_m, tiles_n;
    int group_m;
    int num_tiles;        // output tiles per (split, batch): tiles_m*tiles_n, or tiles_m^2 (triangular)
    int grid_x;           // workgroups per (split, batch), <= num_tiles; each walks its tiles
    int col_splits;       // panel configs: runs of streamed tiles per resident panel
    int tri_cap;          // > 0: chunked triangular work list (tri_item) of the direct kernel
    // stream-K (sk_tiles > 0; direct-staged 128 / 256 tiles, batch 1, split 1):
    // the first sk_dp tiles data-parallel, the last sk_tiles dealt out as
    // K-slices (sk_ipt per tile) over the grid_x workgroups (sk_item: the
    // phase table sk_ph[0 .. sk_nph) when sk_nph > 0, else contiguous
    // ranges); the workspace holds up to grid_x partial tiles, added in by
    // sk_fixup
    int sk_dp, sk_tiles, sk_ipt;
    int sk_nph;
    SkPhase sk_ph[kSkMaxPhases];
};

// Direct global -> LDS staging (gemm_direct.hpp) takes launches of the 256
// tile on dense problems with every slice full (K and the split chunk
// multiples of 32) and 16-byte operands when each split is deep enough.
// Measured against the register-staged kernel (same process, interleaved,
// MI355X): direct wins on every layout from K = 512 per split (8192^3:
// +3-6 %; 8192^2 x 512: +2-5 %); at K = 256 N/N still wins (65536 x 512 x 256:
// +3 %, 8192^2 x 256: +5 %) but the other layouts lose up to 6 %
// (65536 x 512 x 256 T/T).  The 128 tile (16-deep slices) takes it at any
// depth with K and the chunk multiples of 16 (it won on every shape
// measured, K = 96 ... 3072).
inline bool direct_ok(const GemmLaunch& g) {
    if (g.structure != 0 || g.vec != 4) return false;
    if (g.cfg == kCfg256) {
        // byte offsets within a slice (256 rows of a K-contiguous operand, 32
        // rows of an MN-contiguous one) fit 32 bits
        const int64_t lim_a = g.op_a == 0 ? (INT64_C(1) << 21) : (INT64_C(1) << 24);
        const int64_t lim_b = g.op_b != 0 ? (INT64_C(1) << 21) : (INT64_C(1) << 24);
        const int64_t min_chunk = (g.op_a == 0 && g.op_b == 0) ? 256 : 512;
        return g.K % 32 == 0 && g.k_chunk % 32 == 0 && g.k_chunk >= min_chunk &&
               g.lda <= lim_a && g.ldb <= lim_b;
    }
    if (g.cfg == kCfg128) {
        // 128 rows of a K-contiguous operand, 16 rows of an MN-contiguous one
        const int64_t lim_a = g.op_a == 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 25);
        const int64_t lim_b = g.op_b != 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 25);
        return g.K % 16 == 0 && g.k_chunk % 16 == 0 && g.lda <= lim_a && g.ldb <= lim_b;
    }
    if (g.cfg == kCfg128W8) {
        // the 8-wave 32-deep 128 tile: A K-contiguous only (its waves hold one
        // 32-row block, and MN-contiguous A is read in row-block pairs)
        const int64_t lim_a = INT64_C(1) << 22;
        const int64_t lim_b = g.op_b != 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 24);
        return g.op_a == 0 && g.K % 32 == 0 && g.k_chunk % 32 == 0 && g.lda <= lim_a && g.ldb <= lim_b;
    }
    if (g.cfg == kCfg128B32) {
        // 128 rows of a K-contiguous operand, 32 rows of an MN-contiguous one
        const int64_t lim_a = g.op_a == 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 24);
        const int64_t lim_b = g.op_b != 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 24);
        return g.K % 32 == 0 && g.k_chunk % 32 == 0 && g.lda <= lim_a && g.ldb <= lim_b;
    }
    return false;
}

// The 64 x 64 k-split tile (gemm_small.hpp) stages 16-byte slices only:
// dense, K and the split chunk multiples of 64, and the byte offsets within a
// slice (64 rows of either operand layout) below 2^31.
inline bool ksplit_ok(int structure, int vec, int64_t K, int64_t k_chunk, int64_t lda, int64_t ldb) {
    return structure == 0 && vec == 4 && K % 64 == 0 && k_chunk % 64 == 0 &&
           lda <= (INT64_C(1) << 23) && ldb <= (INT64_C(1) << 23);
}

// Dense 128-tile launches the 16-byte path cannot take (operands not 16-byte
// aligned, or K not a multiple of 16) stage with 4-byte direct loads; only
// the last slice of each K range may be partial (the split chunk is a
// multiple of 16).  (The 256 tile with 4-byte loads needs 16 offset VGPRs
// per operand and spilled.)
inline bool direct4_ok(const GemmLaunch& g) {
    const int64_t lim_a = g.op_a == 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 25);
    const int64_t lim_b = g.op_b != 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 25);
    return g.cfg == kCfg128 && g.structure == 0 && !direct_ok(g) && g.K > 0 &&
           g.k_chunk % 16 == 0 && g.lda <= lim_a && g.ldb <= lim_b;
}

// Kernel-side parameter block (passed by value).
struct GemmParams {
    const float* A;
    const float* B;
    float* C;
    float* ws;
    const float* bias;        // NULL or M values; added by the kernel only when split_k == 1
    int M, N, K;
    int tiles_m, tiles_n, group_m;
    int num_tiles;
    int col_splits;
    int tri_cap;
    int sk_dp, sk_tiles, sk_ipt;  // stream-K schedule (GemmLaunch)
    int sk_nph;
    SkPhase sk_ph[kSkMaxPhases];
    int k_chunk, split_k;
    int64_t lda, ldb, ldc;
    int64_t sa, sb, sc;
    int64_t ws_split_stride;  // elements between consecutive split slices
    int64_t ws_batch_stride;
};

hipError_t launch_gemm_nn(const GemmLaunch& g, hipStream_t s);
hipError_t launch_gemm_tn(const GemmLaunch& g, hipStream_t s);
hipError_t launch_gemm_nt(const GemmLaunch& g, hipStream_t s);
hipError_t launch_gemm_tt(const GemmLaunch& g, hipStream_t s);

// After a stream-K launch: adds each split tile's workspace partials into C
// in slot order (sk_tile_slots).
hipError_t launch_sk_fixup(const GemmLaunch& g, hipStream_t s);
hipError_t launch_splitk_reduce(const float* ws, float* C, int M, int N, int batch, int split_k,
                                int64_t ldc, int64_t sc, const float* bias, hipStream_t s);
// After the chunked triangular direct kernel: for every tile of the zero
// triangle, add it into its mirror compute tile when that tile was cut in two
// (it holds the second chunk's partial sum), then write it with +0.0.  C is
// nt*256 square.
// zeroed: the dynamic-order kernel already wrote the zero tiles that hold no
// partial (tri_zero_tile), so only the mirrors and the counter's tile remain.
hipError_t launch_tri_finish(float* C, int64_t ldc, int nt, int cap, bool lower, bool zeroed,
                             hipStream_t s);
// Packs R rows of an operand K-contiguous into dst (row stride kp, a multiple
// of 32; 16-byte aligned): dst[r][k] = src(r, k) for k < K, 0 up to kp.
// k_contig: src(r, k) = src[r*ld + k]; else src[k*ld + r] (transposed).
hipError_t launch_pack_rows(const float* src, int64_t ld, bool k_contig, int64_t R, int64_t K, float* dst,
                            int64_t kp, hipStream_t s);
// Writes integer 0 to one 4-byte word (a kernel, so it can be graph-captured).
hipError_t launch_zero_word(void* w, hipStream_t s);
// C[b][r][c] = bias ? bias[r] : 0 (a contraction with K = 0)
hipError_t launch_fill_zero_2d(float* C, int64_t rows, int64_t cols, int64_t ld, int64_t batch,
                               int64_t batch_stride, hipStream_t s, const float* bias = nullptr);
hipError_t launch_fill_uniform(float* out, int64_t n, uint64_t seed, int64_t offset, hipStream_t s);
hipError_t launch_diag(const float* a, const float* B, float* out, int64_t N, int64_t M,
                       hipStream_t s);
hipError_t launch_scale(const float* A, float* C, int64_t n, float s, hipStream_t st);

// scaled dot-product attention (attention.hip): heads per workspace chunk
constexpr int64_t kSdpaChunkHeads = 128;
int64_t sdpa_chunk_heads(int64_t heads);
size_t sdpa_workspace_bytes(int64_t heads, int seq, int embed);
hipError_t launch_sdpa(const _Float16* Q, const _Float16* K, const _Float16* V, _Float16* O,
                       int64_t heads, int seq, int embed, void* ws, hipStream_t s);

struct GemvPlan {
    int split_k;
    int k_chunk;
    int rows_per_wg;
    int vec;
    size_t ws_bytes;
};
GemvPlan gemv_plan(int64_t M, int64_t K, bool aligned);
hipError_t launch_gemv(const GemvPlan& p, const float* A, const float* x, float* y, float* ws,
                       int M, int K, int64_t lda, hipStream_t s);

}  // namespace mi
