// gemm_tt.hip -- instantiations of the fp32 MFMA engine for op_a = t, op_b = t
// (one translation unit per operand layout so they compile in parallel).
#include "gemm_direct.hpp"
#include "gemm_panel.hpp"
#include "gemm_small.hpp"

namespace mi {
hipError_t launch_gemm_tt(const GemmLaunch& g, hipStream_t s) {
    if (g.cfg == kCfg64W) return launch_ksplit<true, true>(g, s);
    if (is_panel_cfg(g.cfg)) return launch_panel<true, true>(g, s);
    if (direct_ok(g) || direct4_ok(g)) return launch_direct<true, true>(g, s);
    return launch_layout<true, true>(g, s);
}
}  // namespace mi
