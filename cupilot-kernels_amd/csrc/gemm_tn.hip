// gemm_tn.hip -- instantiations of the fp32 MFMA engine for op_a = t, op_b = n
// (one translation unit per operand layout so they compile in parallel).
#include "gemm_direct.hpp"
#include "gemm_panel.hpp"
#include "gemm_small.hpp"

namespace mi {
hipError_t launch_gemm_tn(const GemmLaunch& g, hipStream_t s) {
    if (g.cfg == kCfg64W) return launch_ksplit<true, false>(g, s);
    if (is_panel_cfg(g.cfg)) return launch_panel<true, false>(g, s);
    if (direct_ok(g) || direct4_ok(g)) return launch_direct<true, false>(g, s);
    return launch_layout<true, false>(g, s);
}
}  // namespace mi
