// scheduler.cpp -- host tile scheduler for the fp32 MFMA engine.
//
// A pure function of (M, N, K, batch, layout, structure, CU count, workspace
// available): no device access, no state, so it is tested on the CPU.  It
// replaces the reference's per-kernel compile-time tilings and shape-specific
// literals (e.g. kernels/2_...:16-18 and :129-132 hard-code 2048x8192x4096 and a
// 4x108 persistent grid; kernels/6_...:147-188 splits K over 8 host streams)
// with one cost model:
//   rounds(c, s) = ceil(tiles(c) * s / (CUs * resident(c)))
//   time(c, s)   = rounds * BM*BN*(K/s) * resident(c) / efficiency(c)
//                  + split-K reduction traffic (s * batch * M * N * 4 B * 2 / HBM)
// and picks the cheapest (tile config c, split s).  Triangular problems use a
// square tiling with the compute tiles ordered longest-K first.
#include <algorithm>
#include <cstdint>

#include "../../include/mi355_gemm.h"
#include "mi_internal.hpp"

namespace mi {

namespace {

struct CfgModel {
    int id;
    double efficiency;  // sustained fraction of the CU's MFMA peak
    int resident;       // workgroups resident per CU
};

// efficiency / residency per tile config (gfx950: 4 SIMDs, 512 VGPRs/lane,
// 160 KiB LDS per CU).  Efficiency ranks larger tiles higher because each
// LDS fragment feeds more MFMAs and each HBM byte more flops.
constexpr CfgModel kModels[] = {
    {kCfg256, 1.00, 1},
    {kCfg128, 0.85, 2},
    {kCfg64, 0.55, 4},
};

constexpr double kPeakFlopsPerCuNs = 256.0 * 2.4;  // fp32 MFMA flop per ns per CU
constexpr double kHbmBytesPerNs = 8000.0;

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// Operand-load width: 16-byte loads need the contiguous extent, the leading
// dimension and the batch stride to be multiples of 4 floats and 16-byte
// aligned bases (or a null pointer, as in a pure planning query).
int choose_vec(const mi_gemm_args& a) {
    const bool a_ok = (a.op_a == MI_OP_N ? a.K % 4 == 0 : a.M % 4 == 0) && a.lda % 4 == 0 &&
                      (a.batch <= 1 || a.stride_a % 4 == 0) && aligned16(a.A);
    const bool b_ok = (a.op_b == MI_OP_N ? a.N % 4 == 0 : a.K % 4 == 0) && a.ldb % 4 == 0 &&
                      (a.batch <= 1 || a.stride_b % 4 == 0) && aligned16(a.B);
    return (a_ok && b_ok) ? 4 : 1;
}

// Validation shared by the planner and the launcher.  Returns MI_OK or a
// negative mi_status.  Pointers are not checked here (a plan query may pass none).
int validate_shape(const mi_gemm_args& a) {
    if (a.M < 0 || a.N < 0 || a.K < 0 || a.batch < 0) return MI_ERR_BAD_SIZE;
    if (a.M > INT32_MAX - 256 || a.N > INT32_MAX - 256 || a.K > INT32_MAX - 256)
        return MI_ERR_BAD_SIZE;
    if (a.batch > 65535) return MI_ERR_BAD_SIZE;
    if (a.op_a != MI_OP_N && a.op_a != MI_OP_T) return MI_ERR_BAD_LAYOUT;
    if (a.op_b != MI_OP_N && a.op_b != MI_OP_T) return MI_ERR_BAD_LAYOUT;
    if (a.structure < MI_DENSE || a.structure > MI_UPPER) return MI_ERR_BAD_LAYOUT;
    if (a.structure != MI_DENSE) {
        if (a.M != a.N || a.N != a.K) return MI_ERR_NOT_SQUARE;
        if (a.op_a != MI_OP_N || a.op_b != MI_OP_N || a.batch > 1) return MI_ERR_BAD_LAYOUT;
    }
    const int64_t a_row = a.op_a == MI_OP_N ? a.K : a.M;
    const int64_t b_row = a.op_b == MI_OP_N ? a.N : a.K;
    if (a.M && a.K && a.lda < std::max<int64_t>(1, a_row)) return MI_ERR_BAD_LD;
    if (a.N && a.K && a.ldb < std::max<int64_t>(1, b_row)) return MI_ERR_BAD_LD;
    if (a.M && a.N && a.ldc < std::max<int64_t>(1, a.N)) return MI_ERR_BAD_LD;
    if (a.stride_a < 0 || a.stride_b < 0 || a.stride_c < 0) return MI_ERR_BAD_LD;
    return MI_OK;
}

int plan_gemm(const mi_gemm_args& a, int num_cus, mi_plan& out, GemmLaunch* launch) {
    int rc = validate_shape(a);
    if (rc != MI_OK) return rc;
    if (num_cus <= 0) num_cus = 256;

    int best_cfg = kCfg128, best_split = 1;
    const int override_cfg = a.plan_override & 0xF;
    const int override_split = (a.plan_override >> 8) & 0xFFFF;

    if (a.structure != MI_DENSE) {
        best_cfg = a.N > 2048 ? kCfg128 : kCfg64;
        if (override_cfg >= kCfg64 && override_cfg <= kCfg256) best_cfg = override_cfg;
    } else if (override_cfg >= kCfg64 && override_cfg <= kCfg256) {
        best_cfg = override_cfg;
        best_split = std::max(1, override_split);
    } else {
        double best_t = 1e300;
        const int64_t batch = std::max<int64_t>(1, a.batch);
        for (const CfgModel& m : kModels) {
            const CfgInfo ci = cfg_info(m.id);
            const int64_t tiles = cdiv(a.M, ci.bm) * cdiv(a.N, ci.bn) * batch;
            for (int s = 1; s <= 1024; s *= 2) {
                if (s > 1) {
                    // split only to fill the machine, with >= 1024 K per split
                    if (tiles * (s / 2) >= (int64_t)num_cus * m.resident) break;
                    if (a.K / s < 1024) break;
                    const size_t need = (size_t)s * batch * a.M * a.N * sizeof(float);
                    if (a.workspace_bytes < need) break;
                }
                const int64_t kc = cdiv(cdiv(a.K, s), ci.bk) * ci.bk;
                const double rounds = (double)cdiv(tiles * s, (int64_t)num_cus * m.resident);
                double t = rounds * (2.0 * ci.bm * ci.bn * (double)std::max<int64_t>(kc, ci.bk) *
                                     m.resident) /
                           (m.efficiency * kPeakFlopsPerCuNs);
                if (s > 1) t += 2.0 * s * batch * (double)a.M * a.N * 4.0 / kHbmBytesPerNs;
                if (t < best_t * 0.999) {
                    best_t = t;
                    best_cfg = m.id;
                    best_split = s;
                }
            }
        }
    }

    const CfgInfo ci = cfg_info(best_cfg);
    const int64_t tiles_m = cdiv(a.M, ci.bm), tiles_n = cdiv(a.N, ci.bn);
    int64_t k_chunk = cdiv(cdiv(std::max<int64_t>(a.K, 1), best_split), ci.bk) * ci.bk;
    if (a.structure != MI_DENSE) best_split = 1;
    // an override split larger than K allows collapses to what K can feed
    best_split = (int)std::min<int64_t>(best_split, cdiv(std::max<int64_t>(a.K, 1), k_chunk));
    if (best_split > 65535) return MI_ERR_BAD_SIZE;
    int64_t grid = a.structure != MI_DENSE ? tiles_m * tiles_m : tiles_m * tiles_n;
    if (grid > INT32_MAX) return MI_ERR_BAD_SIZE;

    out.plan_id = best_cfg;
    out.block_m = ci.bm;
    out.block_n = ci.bn;
    out.block_k = ci.bk;
    out.tiles_m = (int32_t)tiles_m;
    out.tiles_n = (int32_t)tiles_n;
    out.split_k = best_split;
    out.k_chunk = k_chunk;
    out.group_m = (int32_t)std::min<int64_t>(tiles_m, 8);
    if (out.group_m < 1) out.group_m = 1;
    out.grid = grid;
    out.workspace_bytes =
        best_split > 1 ? (size_t)best_split * std::max<int64_t>(1, a.batch) * a.M * a.N * sizeof(float) : 0;

    if (launch) {
        GemmLaunch& g = *launch;
        g.A = a.A;
        g.B = a.B;
        g.C = a.C;
        g.ws = static_cast<float*>(a.workspace);
        g.M = (int)a.M;
        g.N = (int)a.N;
        g.K = (int)a.K;
        g.batch = (int)std::max<int64_t>(1, a.batch);
        g.lda = a.lda;
        g.ldb = a.ldb;
        g.ldc = a.ldc;
        g.sa = a.stride_a;
        g.sb = a.stride_b;
        g.sc = a.stride_c;
        g.op_a = a.op_a;
        g.op_b = a.op_b;
        g.structure = a.structure;
        g.cfg = best_cfg;
        g.vec = choose_vec(a);
        g.split_k = best_split;
        g.k_chunk = (int)k_chunk;
        g.tiles_m = (int)tiles_m;
        g.tiles_n = (int)tiles_n;
        g.group_m = out.group_m;
        g.grid_x = (int)grid;
    }
    return MI_OK;
}

}  // namespace mi
