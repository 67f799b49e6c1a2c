// scheduler.cpp -- host tile scheduler for the fp32 MFMA engine.
//
// A pure function of (M, N, K, batch, layout, structure, CU count, workspace
// available): no device access, no state, so it is tested on the CPU.  It
// replaces the reference's per-kernel compile-time tilings and shape-specific
// literals (e.g. kernels/2_...:16-18 and :129-132 hard-code 2048x8192x4096 and a
// 4x108 persistent grid; kernels/6_...:147-188 splits K over 8 host streams)
// with one cost model over (tile config c, split s) and stream-K:
//   per_cu        = ceil(tiles(c) * batch * s / CUs) work items per CU
//   occ           = min(resident workgroups of c, per_cu)
//   time(c, s)    = 2*BM*BN*(K/s) / CU peak * (rounds of occ items / eff(c, occ)
//                     + the last round's leftover items / eff(c, leftover))
//                   + items per workgroup * fixed item cost(c)
//                   + exposed(c, occ) * output bytes * s / sustained write bandwidth
//                   + split-K reduction (read s partials, write C; one pass)
//   stream-K(c)   = the same MFMA work spread evenly over every resident
//                   workgroup, a partial tile per workgroup (the priced
//                   upper bound of either schedule's workspace slots), and the fixup
// and picks the cheapest.  The constants are fitted to MI355X timings (see
// kModels).  Triangular problems use a square tiling with the compute tiles
// ordered longest-K first.
#include <algorithm>
#include <cstdint>

#include "../../include/mi355_gemm.h"
#include "mi_device.hpp"
#include "mi_internal.hpp"

namespace mi {

namespace {

struct CfgModel {
    int id;
    double eff[3];         // sustained fraction of the CU's MFMA peak with 1, 2, >= 3
                           // workgroups of the config resident on the CU
    double item_ns;        // fixed cost per work item of a workgroup
    double store_exp[2];   // fraction of the output store time left exposed with
                           // 1 and >= 2 workgroups per CU
    double sk_eff;         // stream-K: efficiency relative to eff (each segment restarts
                           // the k-split tile's four-stage ring)
};

// Cost model of a dense plan, fitted to 4515 MI355X timings of candidate
// plans -- 64 / 128 / 32-deep 128 / 8-wave 128 / 256 tiles, the 64-tile
// k-split config, split-K 1 - 32, stream-K -- over 229 shapes from 256 x 512 x 4096 to
// 8192 x 3072 x 16384: 141 with 16-byte operand rows, N/N plus all four
// layouts of 12 of them, and 72 random ones in all four layouts whose rows or
// K are not multiples of 4 floats (or K of 16) (tests/data/plan_timings_mi355x.csv,
// fitted offline: a local search on the ranking from the previous
// constants).  The plan it picks is on average 0.7 % slower than the fastest
// one measured, 11 % at worst.  The single-slice configs (K <= 32 / 64) take the 128 tile's
// constants with half its exposed store time.
constexpr CfgModel kModels[] = {
    {kCfg256, {0.9547, 0.9547, 0.9547}, 1.372, {1.447, 1.447}, 1.0},
    {kCfg128, {0.8892, 0.91, 0.9178}, 2904, {1.5, 0.4952}, 1.0},
    {kCfg64, {0.4263, 0.654, 0.72}, 2961, {1.5, 0.4952}, 1.0},
    {kCfg128K32, {0.8892, 0.91, 0.9178}, 0.0, {0.75, 0.2476}, 1.0},
    {kCfg128K64, {0.8892, 0.91, 0.9178}, 0.0, {0.75, 0.2476}, 1.0},
    {kCfg128B32, {0.861, 0.9231, 0.9231}, 4510, {1.5, 0.4952}, 1.0},
    {kCfg64W, {0.850, 0.850, 0.850}, 2361.0, {0.733, 0.733}, 0.798},
    {kCfg128W8, {0.995, 0.9354, 0.9354}, 4815, {1.5, 0.4952}, 1.0},
};

constexpr double kPeakFlopsPerCuNs = 256.0 * 2.4;  // fp32 MFMA flop per ns per CU
constexpr double kW8OneRoundEff = 0.95;              // config 11, one round of <= 1 tile per CU
constexpr double kB32OneRoundEff = 0.90;             // config 9, likewise
constexpr double kWriteBytesPerNs = 5500.0;        // sustained write-only bandwidth (measured)
// split-K reduction and stream-K fixup passes: bytes per ns over what they
// read and write, plus a fixed cost per reduction pass
constexpr double kReduceBytesPerNs = 7592.0;
constexpr double kReduceNs = 5354.0;
// stream-K: the fixup workgroup of a tile adds its G / S partials one after
// another (G workgroups, S stream-K tiles)
constexpr double kSkSlotNs = 962.3;
// Operands the 16-byte loaders cannot stage: efficiency relative to eff of
// the 128 tile's 4-byte direct staging (data-parallel / split-K, and
// stream-K) with its extra cost per work item (each sets up its 4-byte load
// offsets), and of the 64 and 256 tiles, which then load through registers
// one float at a time.
constexpr double kFourByteEff = 0.8815;
constexpr double kFourByteItemNs = 1010.0;
constexpr double kFourByteSkEff = 1.121;
constexpr double kFourByteSkItemNs = 5552.0;
constexpr double kReg64Eff = 0.5706;
constexpr double kReg256Eff = 0.8389;
// C rows not 16-byte aligned: the output stores are element-wise (their time
// x kScalarStoreFactor), and so are the split-K reduction and the stream-K
// fixup (bandwidth x kScalarReduceEff).
constexpr double kScalarStoreFactor = 5.497;
constexpr double kScalarReduceEff = 0.2811;
// packing pass (plan_gemm): bytes per ns over what it reads and writes and
// a fixed cost per pack launch (measured: 8205 x 5921 x 2949 in the four
// layouts 58-87 us for 335 MB, 4095^3 63 us, 1021^3 15 us); the gain a
// packed plan must promise, and the smallest K it is offered for (30 random
// unaligned shapes with K 256-1535, M, N 768-9000, timed packed and unpacked:
// never packing them cost 5.3 % on average, up to 29 % (1471 x 1329 x 1188);
// the model's choice 0.6 %, up to 6.5 % (7494 x 2940 x 465))
constexpr double kPackBytesPerNs = 5000.0;
constexpr double kPackLaunchNs = 5000.0;
constexpr double kPackMargin = 0.97;
constexpr int64_t kPackMinK = 256;
// Against an unpacked stream-K plan on the 4-byte path the packed plan is
// taken unless it is modelled kPackMarginSk times slower: on 40 random
// unaligned shapes (M, N 768-9000, K 1536-10000, all four layouts) that
// plan's modelled time ran 10-30 % below its measured time while the packed
// plans' stayed within 3-8 %, and packing measured faster on 35 of them
// (mean regret of the choice 2.9 %, up to 12 %, with kPackMargin; 0.05 %,
// up to 0.9 %, with this margin).
constexpr double kPackMarginSk = 1.25;

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Smallest K per split the cost model may choose.
constexpr int64_t kMinSplitK = 128;

// Workgroups of each config held on one CU at once; the kernels are built to
// exactly this occupancy (amdgpu_waves_per_eu): 64-tile 8, 128-tile 3, 256-tile 1.
int resident_wgs(int cfg) {
    switch (cfg) {
        case kCfg256: return 1;
        case kCfg128: return 3;
        case kCfg128K32: return 3;
        case kCfg128K64: return 2;
        case kCfgPanel32: return 1;
        case kCfgPanel64: return 1;
        case kCfgPanel128x64: return 1;
        case kCfgPanel64B: return 1;
        case kCfg128B32: return 2;
        case kCfg128W8: return 2;
        case kCfg64W: return 1;
        default: return 8;
    }
}

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
    if (a.bias_m && (a.op_a != MI_OP_N || a.op_b != MI_OP_N)) return MI_ERR_BAD_LAYOUT;
    if (a.structure != MI_DENSE) {
        if (a.bias_m) return MI_ERR_BAD_LAYOUT;
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

namespace {

// Stream-K schedule of a dense product on config cfg (sk_item in
// mi_device.hpp: contiguous K-slice ranges, or the phase table), or
// sk.tiles = 0 where it does not apply: batch 1, no bias, the direct-staged
// 16-byte kernels (every K-slice full), a tile count that whole waves of the
// persistent grid do not cover exactly, at least two slices per workgroup,
// and a workspace of one partial tile per workgroup (either schedule's slots
// fit it).
struct SkChoice {
    int dp = 0, tiles = 0, ipt = 0, grid = 0;
    size_t ws = 0;
    int nph = 0;  // > 0: the phase table (sk_build_phases), else contiguous ranges
    SkPhase ph[kSkMaxPhases] = {};
};

SkChoice plan_stream_k(const mi_gemm_args& a, int cfg, int num_cus) {
    SkChoice sk;
    if (cfg != kCfg256 && cfg != kCfg128 && cfg != kCfg128B32 && cfg != kCfg64W) return sk;
    if (a.structure != MI_DENSE || a.batch > 1 || a.bias_m != nullptr) return sk;
    if (((uintptr_t)a.workspace & 15u) != 0) return sk;
    const CfgInfo ci = cfg_info(cfg);
    GemmLaunch g{};
    g.structure = 0;
    g.vec = choose_vec(a);
    g.cfg = cfg;
    g.K = (int)a.K;
    g.k_chunk = (int)a.K;
    g.op_a = a.op_a;
    g.op_b = a.op_b;
    g.lda = a.lda;
    g.ldb = a.ldb;
    bool staged = cfg == kCfg64W ? ksplit_ok(a.structure, g.vec, a.K, a.K, a.lda, a.ldb)
                                 : direct_ok(g);
    if (!staged && cfg == kCfg128 && a.K > 0) {
        // 4-byte direct staging: one K range per tile, of whole 16-deep
        // slices but its last, which may end at K
        g.k_chunk = (int)(cdiv(a.K, ci.bk) * ci.bk);
        staged = direct4_ok(g);
    }
    if (a.K <= 0 || !staged) return sk;
    const int64_t T = cdiv(a.M, ci.bm) * cdiv(a.N, ci.bn);
    const int64_t G = (int64_t)num_cus * resident_wgs(cfg);
    if (G % 8 != 0 || T % G == 0) return sk;
    // Every whole wave of tiles runs data-parallel and only the remainder is
    // dealt out in K-slices.  The data-parallel tiles of one XCD, neighbours
    // in the raster, run in step and share their A rows and B columns in L2;
    // stream-K segments start at different K offsets and share nothing.
    // Measured against keeping the last whole wave in the stream-K part
    // (one process, 11 shapes with 1-6 waves): equal or faster on all, by
    // 0.2-1.7 % (4608^3 1.360 vs 1.375 ms in every layout, fetching 1.09 vs
    // 3.06 GB from beyond L2; 10240^2 x 2048 2.94 vs 2.99 ms).
    const int64_t waves = T / G;
    const int64_t dp = waves * G;
    const int64_t S = T - dp;
    const int64_t ipt = cdiv(a.K, ci.bk);
    if (S * ipt < 2 * G || T > INT32_MAX) return sk;
    const size_t need = (size_t)G * ci.bm * ci.bn * sizeof(float);
    if (a.workspace_bytes < need) return sk;
    sk.dp = (int)dp;
    sk.tiles = (int)S;
    sk.ipt = (int)ipt;
    sk.grid = (int)G;
    sk.ws = need;
    return sk;
}

// The phased schedule (sk_build_phases) of a stream-K choice at the smallest
// budget it meets, where that is no more than the contiguous ranges' busiest
// workgroup (plan_override MI_PLAN_SK_RANGES: always the ranges).  Its slots
// must not outnumber the workgroups, so the workspace stays the same.  Only
// the chosen plan's schedule is built: the cost model prices stream-K the
// same under either.
void sk_choose_phases(const mi_gemm_args& a, SkChoice& sk) {
    sk.nph = 0;
    if (sk.tiles <= 0 || (a.plan_override & MI_PLAN_SK_RANGES) != 0) return;
    const int64_t S = sk.tiles, ipt = sk.ipt, G = sk.grid;
    const int64_t limit = sk_ranges_cost(S, ipt, G);
    for (int64_t B = cdiv(S * ipt, G) + kSkSegCost; B <= limit; ++B) {
        SkPhase ph[kSkMaxPhases];
        int nph = 0;
        int64_t slots = 0;
        const int most = sk_build_phases(S, ipt, G, B, ph, nph, slots);
        if (most > 0 && most <= kSkMaxSegments && slots <= G) {
            sk.nph = nph;
            for (int q = 0; q < nph; ++q) sk.ph[q] = ph[q];
            return;
        }
    }
}

// The planner proper (plan_gemm below adds the choice of packing the
// operands).  cost: the cost model's time of the chosen plan in ns, or -1
// when the plan does not come from the cost model (structured products,
// panel configs, overrides).
int plan_core(const mi_gemm_args& a, int num_cus, mi_plan& out, GemmLaunch* launch, double* cost) {
    int rc = validate_shape(a);
    if (rc != MI_OK) return rc;
    if (num_cus <= 0) num_cus = 256;
    double model_t = -1.0;

    int best_cfg = kCfg128, best_split = 1;
    SkChoice best_sk;
    // plan_override bit 4: take stream-K on the override config where it
    // applies; bit 5: never take stream-K
    const bool force_sk = (a.plan_override & 0x10) != 0;
    const bool no_sk = (a.plan_override & 0x20) != 0;
    const int override_cfg = a.plan_override & 0xF;
    const int override_split = (a.plan_override >> 8) & 0xFFF;
    const int override_group = (a.plan_override >> 20) & 0x3FF;

    // the 32-deep 128 tile exists only direct-staged (16-byte operands, K % 32 == 0)
    // (its row limits: the buffer offsets of 128 K-contiguous rows or 32
    // MN-contiguous rows stay below 2^31 bytes)
    const bool b32_ok = a.structure == MI_DENSE && choose_vec(a) == 4 && a.K % 32 == 0 &&
                        a.lda <= (a.op_a == 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 24)) &&
                        a.ldb <= (a.op_b != 0 ? (INT64_C(1) << 22) : (INT64_C(1) << 24));
    // the 64-tile k-split config: 16-byte operands, K a multiple of 64
    const bool w64_ok = ksplit_ok(a.structure, choose_vec(a), a.K, 64, a.lda, a.ldb) && a.K > 0;
    const bool override_ok =
        override_cfg >= kCfg64 && override_cfg < kNumCfg && (override_cfg != kCfg128B32 || b32_ok) &&
        (override_cfg != kCfg128W8 || (b32_ok && a.op_a == MI_OP_N)) &&
        (override_cfg != kCfg64W || w64_ok) &&
        !((override_cfg == kCfg128K32 || override_cfg == kCfg128K64 || is_panel_cfg(override_cfg)) &&
          a.K > cfg_info(override_cfg).bk) &&
        !(is_panel_cfg(override_cfg) && a.structure != MI_DENSE) &&
        !(is_panel_b_cfg(override_cfg) && a.bias_m != nullptr);
    // Triangular products with N a multiple of 256 and operands the direct
    // kernel can stage run on the 256-tile direct kernel over the chunked
    // longest-first work list (tri_item) when the structure has a tile for
    // every CU (or the 256 config is asked for).  Tiles longer than a CU's
    // share of the work are cut in two (cap = ceil(nt / 2) units), so the
    // longest item no longer sets the finishing time; an override split
    // (>= ceil(nt / 2)) sets the cap instead.
    int tri_cap = 0;
    if (a.structure != MI_DENSE && a.N % 256 == 0 && choose_vec(a) == 4 &&
        a.lda <= (INT64_C(1) << 21) && a.ldb <= (INT64_C(1) << 24)) {
        const int64_t nt = a.N / 256;
        const bool wanted =
            override_ok ? override_cfg == kCfg256 : nt * (nt + 1) / 2 >= (int64_t)num_cus;
        if (wanted) {
            const double units_per_cu = (double)nt * (nt + 1) * (nt + 2) / 6.0 / num_cus;
            tri_cap = (int)(units_per_cu < (double)nt ? (nt + 1) / 2 : nt);
            if (override_ok && override_split > 0)
                tri_cap = (int)std::min<int64_t>(nt, std::max<int64_t>((nt + 1) / 2, override_split));
        }
    }
    if (a.structure != MI_DENSE) {
        best_cfg = a.N > 2048 ? kCfg128 : kCfg64;
        if (override_ok) best_cfg = override_cfg;
        if (tri_cap > 0) best_cfg = kCfg256;
    } else if (override_ok) {
        best_cfg = override_cfg;
        best_split = is_panel_cfg(override_cfg) ? 1 : std::max(1, override_split);
        if (force_sk && !no_sk) {
            best_sk = plan_stream_k(a, override_cfg, num_cus);
            if (best_sk.tiles > 0) best_split = 1;
        }
    } else if (a.K <= 64 && a.M % 128 == 0 && a.M % 256 != 0 && a.M < 2048 &&
               cdiv(a.M, 128) * cdiv(a.N, 128) * std::max<int64_t>(1, a.batch) >=
                   2 * (int64_t)num_cus) {
        // The same for M an odd multiple of 128 (the 1x1 convolution's
        // output channels): 128-row panels, none of them padding.
        best_cfg = kCfgPanel128x64;
    } else if (a.K > 32 && a.K <= 64 && a.bias_m == nullptr && (a.N % 256 == 0 || a.N >= 2048) &&
               (a.M % 128 == 0 || a.M >= 1024) &&
               cdiv(a.M, 128) * cdiv(a.N, 256) * std::max<int64_t>(1, a.batch) >=
                   2 * (int64_t)num_cus) {
        // 33-64 deep with a large output and no row bias: the B-resident
        // panel, whose workgroups share A tiles in L2 and store to
        // contiguous rows (65536^2 x 64: 4.98-5.09 vs 5.25-5.49 ms for the
        // A-resident panel, all four layouts; 4096 x 2048 x 64: 19 vs 23 us).
        // Its panels are 256 columns and its streamed tiles 128 rows, each
        // filled to at least 7/8.
        best_cfg = kCfgPanel64B;
    } else if (a.K <= 64 && (a.M % 256 == 0 || a.M >= 2048) &&
               cdiv(a.M, 256) * cdiv(a.N, 128) * std::max<int64_t>(1, a.batch) >=
                   2 * (int64_t)num_cus) {
        // Small K and a large output: the A-panel kernel cuts operand reloads
        // to ~K/256 of the output bytes (tall-skinny: 4 GiB instead of 16 GiB).
        // Its panels are 256 rows: M must fill them (at most 1/8 padding), or
        // the padded rows cost MFMA time for nothing (M = 128: half).
        // The panel depth matching K takes the overlapped-store path
        // (16384^2 x 32: 0.29 ms with the 32-deep panel, 0.34 ms with the
        // 64-deep one).
        best_cfg = a.K <= 32 ? kCfgPanel32 : kCfgPanel64;
    } else {
        double best_t = 1e300;
        const int64_t batch = std::max<int64_t>(1, a.batch);
        const double out_bytes = 4.0 * (double)batch * a.M * a.N;
        // C rows not 16-byte aligned: element-wise stores, reduction and fixup
        const bool c_vec = a.N % 4 == 0 && a.ldc % 4 == 0 && (a.batch <= 1 || a.stride_c % 4 == 0) &&
                           (a.C == nullptr || aligned16(a.C));
        const double st_x = c_vec ? 1.0 : kScalarStoreFactor;
        const double red_x = c_vec ? 1.0 : 1.0 / kScalarReduceEff;
        // The 256 tile stages through LDS directly only with 16-byte operands
        // and K a multiple of 32; otherwise it loads through registers one
        // float at a time, while the 128 tile keeps direct (4-byte) staging:
        // measured 8191^3 111 vs 137, 2048 x 8190 x 4096 109 vs 137 TFLOP/s.
        const bool full16 = choose_vec(a) == 4 && a.K % 32 == 0;
        for (const CfgModel& m : kModels) {
            const CfgInfo ci = cfg_info(m.id);
            if ((m.id == kCfg128K32 || m.id == kCfg128K64) && a.K > ci.bk) continue;
            if (m.id == kCfg128B32 && !b32_ok) continue;
            // the 8-wave tile: its longer per-tile prologue and store pay off
            // from K = 1024 (4096^2 x 512: 131 vs 127 us for the 128 tile)
            if (m.id == kCfg128W8 && !(b32_ok && a.op_a == MI_OP_N && a.K >= 1024)) continue;
            if (m.id == kCfg64W && !w64_ok) continue;
            // the 64 tile stages through registers: with operands that are not
            // 16-byte aligned it loads one float at a time, where the 128 tile
            // keeps direct 4-byte staging (4248 x 2044 x 3769: 59 vs 96 TFLOP/s)
            // (the 128 tile's 4-byte direct staging: kFourByteEff for its
            // data-parallel and split-K plans, kFourByteSkEff for stream-K)
            const bool four_byte = m.id == kCfg128 && !(choose_vec(a) == 4 && a.K % 16 == 0);
            const double scale = m.id == kCfg256 && !full16           ? kReg256Eff
                                 : m.id == kCfg64 && choose_vec(a) != 4 ? kReg64Eff
                                 : four_byte                            ? kFourByteEff
                                                                        : 1.0;
            const int res = resident_wgs(m.id);
            const int64_t tiles = cdiv(a.M, ci.bm) * cdiv(a.N, ci.bn) * batch;
            const double tile_bytes = 4.0 * ci.bm * ci.bn;
            for (int s = 1; s <= 1024; s *= 2) {
                if (s > 1) {
                    // the 8-wave tile is for one tile per CU: with split-K it
                    // measured no faster than unsplit (1024 x 3072 x 16384:
                    // 0.95, 0.94, 0.94 ms at split 1, 2, 4)
                    if (m.id == kCfg128W8) break;
                    // split only to fill the machine, with >= kMinSplitK of K per
                    // split: while the previous split's items stay below four
                    // times the CUs (the k-split 64 tile, one workgroup per CU,
                    // measured fastest at 4.5 items per CU: 3620 x 296 x 6144)
                    if (tiles * (s / 2) >= 4 * (int64_t)num_cus) break;
                    if (a.K / s < kMinSplitK) break;
                    const size_t need = (size_t)s * batch * a.M * a.N * sizeof(float);
                    if (a.workspace_bytes < need) break;
                }
                // per CU: its share of the work items, run with as many of them
                // resident as the config allows; each workgroup walks its items
                const int64_t items = tiles * s;
                const int64_t kc = cdiv(cdiv(std::max<int64_t>(a.K, 1), s), ci.bk) * ci.bk;
                const int64_t per_cu = cdiv(items, (int64_t)num_cus);
                const int occ = (int)std::min<int64_t>(res, per_cu);
                const int64_t grid = std::min<int64_t>((int64_t)num_cus * res, items);
                // full rounds of occ resident items at that occupancy, then the
                // last round's leftover items at their own, lower occupancy
                const int64_t rounds = per_cu / occ, rem = per_cu % occ;
                // With at most one tile per CU (the whole problem in one
                // round) two tiles run at efficiencies of their own: the
                // 8-wave tile ~5 % below what its fit gives full rounds
                // (1792^2 x 2048 123.2 us, 1536 x 2304 x 4096 240.7 us, against
                // 115.5 / 225.7 us for the 32-deep 128 tile's stream-K, which
                // the model had priced higher), and the 32-deep 128 tile
                // above it, ~2.5 % faster than the 16-deep 128 tile in every
                // one-round case of the timing table, all layouts (2048^2 x
                // 4096 T/N 250.4 vs 267.6 us, T/T 252.0 vs 264.5)
                const double e_one = per_cu != 1              ? m.eff[0]
                                     : m.id == kCfg128W8   ? kW8OneRoundEff
                                     : m.id == kCfg128B32  ? kB32OneRoundEff
                                                           : m.eff[0];
                const double slots = (double)(rounds * occ) / (occ == 1 ? e_one : m.eff[std::min(occ, 3) - 1]) +
                                     (rem ? (double)rem / m.eff[std::min<int64_t>(rem, 3) - 1] : 0.0);
                double t = slots * 2.0 * ci.bm * ci.bn * (double)kc / (scale * kPeakFlopsPerCuNs);
                t += (double)cdiv(items, grid) * (m.item_ns + (four_byte ? kFourByteItemNs : 0.0));
                t += m.store_exp[occ > 1 ? 1 : 0] * st_x * out_bytes * s / kWriteBytesPerNs;
                if (s > 1) t += (s + 1) * out_bytes / kReduceBytesPerNs * red_x + kReduceNs;
                if (t < best_t * 0.999) {
                    best_t = t;
                    best_cfg = m.id;
                    best_split = s;
                    best_sk = SkChoice{};
                }
            }
            // Stream-K on this config: the MFMA work spread evenly over every
            // resident workgroup (no wave quantisation), plus one partial tile
            // stored per workgroup and the fixup pass (read the partials, read
            // and write the split tiles of C).
            const SkChoice sk = no_sk ? SkChoice{} : plan_stream_k(a, m.id, num_cus);
            // 4-byte staging: stream-K measured faster only with deep tiles,
            // enough of them (with fewer than G / 6 each tile splits into many
            // segments), and a data-parallel plan whose busiest CU has >= 12 %
            // more tiles than the mean (72 random unaligned shapes, all four
            // layouts); the cost model is not offered it otherwise
            // Below K = 1024 stream-K measured slower than the data-parallel
            // plan on all 25 shapes of the timing table; the 8-wave tile is
            // offered data-parallel only.
            // The k-split tile below one wave of tiles with K <= 2048 (at most
            // 32 slices per tile, about two segments each) measured faster
            // data-parallel or split in two on all 18 such shapes tried
            // (768^2 x 2048 36.7 vs 40.4 us, 1408 x 256 x 2048 24.9 vs 33.1,
            // 256 x 1280 x 1024 17.0 vs 18.8); with deeper K its stream-K
            // stayed ahead of the split-K plans (2688 x 256 x 4096 53.6 vs
            // 61.4 us, 1152 x 256 x 8192 51.5 vs 57.4).
            const bool sk_offered =
                a.K >= 1024 && m.id != kCfg128W8 &&
                !(m.id == kCfg64W && a.K <= 2048 && sk.dp == 0) &&
                (!four_byte || (a.K >= 1536 && 6 * tiles >= (int64_t)sk.grid &&
                                (double)cdiv(tiles, num_cus) * num_cus >= 1.12 * (double)tiles));
            if (sk.tiles > 0 && sk_offered) {
                const double eff = (four_byte ? kFourByteSkEff : scale) * m.sk_eff *
                                   m.eff[std::min(res, 3) - 1];
                double t = (double)tiles * 2.0 * ci.bm * ci.bn * (double)a.K / num_cus /
                           (eff * kPeakFlopsPerCuNs);
                t += (double)(sk.dp / sk.grid + 2) * (m.item_ns + (four_byte ? kFourByteSkItemNs : 0.0));
                t += m.store_exp[res > 1 ? 1 : 0] * (st_x * out_bytes + sk.grid * tile_bytes) /
                     kWriteBytesPerNs;
                t += 3.0 * sk.grid * tile_bytes / kReduceBytesPerNs * red_x +
                     kSkSlotNs * (double)sk.grid / sk.tiles;
                if (t < best_t * 0.999) {
                    best_t = t;
                    best_cfg = m.id;
                    best_split = 1;
                    best_sk = sk;
                }
            }
        }
        model_t = best_t;
    }

    const CfgInfo ci = cfg_info(best_cfg);
    const int64_t tiles_m = cdiv(a.M, ci.bm), tiles_n = cdiv(a.N, ci.bn);
    int64_t k_chunk = cdiv(cdiv(std::max<int64_t>(a.K, 1), best_split), ci.bk) * ci.bk;
    if (a.structure != MI_DENSE) best_split = 1;
    // an override split larger than K allows collapses to what K can feed
    best_split = (int)std::min<int64_t>(best_split, cdiv(std::max<int64_t>(a.K, 1), k_chunk));
    if (best_split > 65535) return MI_ERR_BAD_SIZE;
    const int64_t num_tiles = tri_cap > 0              ? tri_items((int)tiles_m, tri_cap)
                              : a.structure != MI_DENSE ? tiles_m * tiles_m
                                                        : tiles_m * tiles_n;
    if (num_tiles > INT32_MAX) return MI_ERR_BAD_SIZE;
    // Persistent grid: as many workgroups as the CUs hold at once (a multiple
    // of the 8 XCDs so every workgroup keeps to one XCD), each walking the
    // tile list with stride grid.
    const int64_t batch = std::max<int64_t>(1, a.batch);
    const int64_t slots = (int64_t)num_cus * resident_wgs(best_cfg);
    int64_t grid = cdiv(slots, (int64_t)best_split * batch);
    if (batch > 1 && num_tiles > 0) {
        // batched: the (split, batch) grids already spread over the XCDs;
        // the fewest workgroups per batch that keeps each one's tile count
        // (every workgroup walks the same number of tiles, +-1).  Rounding up
        // to a multiple of 8 here left 8 workgroups per batch walking 12
        // tiles of 256 (1024 x 768 per batch, 64 batches): 109 vs 135 TFLOP/s.
        grid = cdiv(num_tiles, cdiv(num_tiles, grid));
    } else {
        grid = cdiv(grid, 8) * 8;
    }
    grid = std::min(grid, num_tiles);
    // Triangular tiles differ in length: one tile per workgroup, and the
    // hardware's dispatch as slots free up balances them better than a
    // static stride.  The chunked work list with cap >= 2 claims its items
    // from a counter instead: one persistent workgroup per CU.
    if (a.structure != MI_DENSE)
        grid = tri_cap >= 2 ? std::min<int64_t>(num_cus, num_tiles) : num_tiles;
    // Panel configs: each work item is one resident panel times a run of streamed
    // tiles; enough runs per panel to give every resident workgroup one.
    int64_t col_splits = 1;
    if (is_panel_cfg(best_cfg)) {
        // (B-resident panels: one per column tile, runs of row tiles)
        const int64_t panels = is_panel_b_cfg(best_cfg) ? tiles_n : tiles_m;
        const int64_t streamed = is_panel_b_cfg(best_cfg) ? tiles_m : tiles_n;
        col_splits = std::min<int64_t>(streamed, std::max<int64_t>(1, cdiv(slots, panels * batch)));
        grid = std::min<int64_t>(panels * col_splits, std::max<int64_t>(1, slots / batch));
    }
    // The direct-staged 128 tile with at least two waves of work items runs
    // one tile per workgroup instead: a finished tile's stores then leave
    // with its waves and do not hold up the next tile's slice waits (gfx9's
    // vmcnt counts a wave's stores with its loads), while the other two
    // workgroups on the CU cover the next one's start.  Measured in one
    // process: 65536 x 512 x 256 129.9 vs 127.0 TFLOP/s, 8192^2 x 512 141.5
    // vs 137.1, 16384^2 x 256 133.5 vs 127.2, 32768 x 1024 x 192 122.7 vs
    // 118.9; with about one wave (4096^2 x 512, 16384 x 768 x 512) equal.
    // (The 256 and 32-deep 128 tiles, one and two workgroups per CU, lose
    // 2 % that way on 65536 x 512 x 256.)
    if (best_cfg == kCfg128 && a.structure == MI_DENSE && choose_vec(a) == 4 && a.K % 16 == 0 &&
        num_tiles * best_split * batch >= 2 * slots)
        grid = num_tiles;
    // Stream-K: every resident workgroup takes part (its K-slice range),
    // whatever the tile count.
    if (best_sk.tiles > 0) grid = best_sk.grid;

    out.plan_id = best_cfg;
    out.block_m = ci.bm;
    out.block_n = ci.bn;
    out.block_k = ci.bk;
    out.tiles_m = (int32_t)tiles_m;
    out.tiles_n = (int32_t)tiles_n;
    out.split_k = best_split;
    out.k_chunk = k_chunk;
    out.group_m = (int32_t)std::min<int64_t>(tiles_m, override_group > 0 ? override_group : 8);
    if (out.group_m < 1) out.group_m = 1;
    out.num_tiles = num_tiles;
    out.grid = grid;
    out.workspace_bytes =
        best_split > 1 ? (size_t)best_split * batch * a.M * a.N * sizeof(float) : best_sk.ws;
    sk_choose_phases(a, best_sk);
    out.stream_k = best_sk.tiles > 0 ? 1 : 0;
    out.sk_tiles = best_sk.tiles;
    out.sk_phases = best_sk.tiles > 0 ? best_sk.nph : 0;

    if (launch) {
        GemmLaunch& g = *launch;
        g.A = a.A;
        g.B = a.B;
        g.C = a.C;
        g.ws = static_cast<float*>(a.workspace);
        g.bias = a.bias_m;
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
        g.num_tiles = (int)num_tiles;
        g.col_splits = (int)col_splits;
        g.grid_x = (int)grid;
        g.tri_cap = tri_cap;
        g.sk_dp = best_sk.dp;
        g.sk_tiles = best_sk.tiles;
        g.sk_ipt = best_sk.ipt;
        g.sk_nph = best_sk.nph;
        for (int q = 0; q < kSkMaxPhases; ++q) g.sk_ph[q] = best_sk.ph[q];
    }
    out.packed = 0;
    out.packed_k = 0;
    if (cost) *cost = model_t;
    return MI_OK;
}

// Packing: operands the 16-byte loaders cannot stage (rows or K not a
// multiple of 4 floats, or K not of 32 -- the 256 tile's slice depth) are
// first copied into the workspace K-contiguous, with K zero-padded to a
// multiple of 32 (launch_pack_rows: a copy for K-contiguous sources, a
// transpose through LDS for MN-contiguous ones), and the product runs as
// the N/T problem A'[M][Kp] x B'[N][Kp]^T on the 16-byte kernels; the zero
// padding adds exact zeros.  Dense products only, batch 1, no row bias.
bool pack_eligible(const mi_gemm_args& a) {
    if (a.structure != MI_DENSE || a.batch > 1 || a.bias_m != nullptr) return false;
    if (a.M <= 0 || a.N <= 0 || a.K <= 0) return false;
    if (choose_vec(a) == 4 && a.K % 32 == 0) return false;  // already 16-byte staged
    const int64_t kp = cdiv(a.K, 32) * 32;
    return cdiv(kp, 64) <= 65535;  // the transpose kernel's grid.y
}

// workspace layout of a packed plan: A' at 0, B' and then the product's own
// workspace at 256-byte boundaries
size_t pack_a_bytes(const mi_gemm_args& a, int64_t kp) {
    return (size_t)cdiv(a.M * kp * (int64_t)sizeof(float), 256) * 256;
}
size_t pack_bytes(const mi_gemm_args& a, int64_t kp) {
    return pack_a_bytes(a, kp) + (size_t)cdiv(a.N * kp * (int64_t)sizeof(float), 256) * 256;
}

}  // namespace

int packed_k(const mi_gemm_args& a) { return (int)(cdiv(a.K, 32) * 32); }

mi_gemm_args packed_problem(const mi_gemm_args& a, void* workspace, size_t workspace_bytes) {
    const int64_t kp = packed_k(a);
    mi_gemm_args p = a;
    char* const ws = static_cast<char*>(workspace);
    p.A = ws ? reinterpret_cast<const float*>(ws) : nullptr;
    p.B = ws ? reinterpret_cast<const float*>(ws + pack_a_bytes(a, kp)) : nullptr;
    p.K = kp;
    p.op_a = MI_OP_N;
    p.op_b = MI_OP_T;
    p.lda = kp;
    p.ldb = kp;
    p.batch = 1;
    p.stride_a = p.stride_b = 0;
    // forced packing keeps the other override bits for the packed product;
    // the planner's own choice keeps the raster grouping and "never
    // stream-K" (bit 5), which holds for whatever product runs
    const int32_t keep =
        (a.plan_override & MI_PLAN_PACK) ? ~(MI_PLAN_NO_PACK | MI_PLAN_PACK)
                                         : ((0x3FF << 20) | 0x20 | MI_PLAN_SK_RANGES);
    p.plan_override = (a.plan_override & keep) | MI_PLAN_NO_PACK;
    const size_t pb = pack_bytes(a, kp);
    p.workspace = ws && workspace_bytes > pb ? ws + pb : nullptr;
    p.workspace_bytes = workspace_bytes > pb ? workspace_bytes - pb : 0;
    return p;
}

size_t packed_operand_bytes(const mi_gemm_args& a) { return pack_bytes(a, packed_k(a)); }

int plan_gemm(const mi_gemm_args& a, int num_cus, mi_plan& out, GemmLaunch* launch) {
    double t0 = -1.0;
    int rc = plan_core(a, num_cus, out, launch, &t0);
    if (rc != MI_OK) return rc;
    const bool no_pack = (a.plan_override & MI_PLAN_NO_PACK) != 0;
    const bool force_pack = (a.plan_override & MI_PLAN_PACK) != 0;
    if (no_pack || !pack_eligible(a) || (t0 < 0 && !force_pack)) return MI_OK;
    if (!force_pack && a.K < kPackMinK) return MI_OK;
    const int64_t kp = packed_k(a);
    const size_t pb = pack_bytes(a, kp);
    if (a.workspace_bytes < pb || (a.workspace && ((uintptr_t)a.workspace & 255u) != 0)) return MI_OK;
    const mi_gemm_args pa = packed_problem(a, nullptr, a.workspace_bytes);
    mi_plan pp{};
    GemmLaunch pg{};
    double t1 = -1.0;
    if (plan_core(pa, num_cus, pp, launch ? &pg : nullptr, &t1) != MI_OK) return MI_OK;
    // the packing pass: read both operands, write them padded, two launches
    const double moved = 4.0 * (double)(a.M + a.N) * (double)(a.K + kp);
    t1 += moved / kPackBytesPerNs + 2.0 * kPackLaunchNs;
    const bool four_byte_sk = out.stream_k && !(choose_vec(a) == 4 && a.K % 16 == 0);
    const double margin = four_byte_sk ? kPackMarginSk : kPackMargin;
    if (!force_pack && !(t1 >= 0 && t1 < margin * t0)) return MI_OK;
    if (pp.workspace_bytes > SIZE_MAX - pb) return MI_OK;
    out = pp;
    out.workspace_bytes = pb + pp.workspace_bytes;
    out.packed = 1;
    out.packed_k = kp;
    if (launch) *launch = pg;
    return MI_OK;
}

}  // namespace mi
