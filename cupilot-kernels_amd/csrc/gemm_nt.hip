// gemm_nt.hip -- instantiations of the fp32 MFMA engine for op_a = n, op_b = t
// (one translation unit per operand layout so they compile in parallel).
#include "gemm_direct.hpp"
#include "gemm_panel.hpp"
#include "gemm_small.hpp"

namespace mi {
hipError_t launch_gemm_nt(const GemmLaunch& g, hipStream_t s) {
    if (g.cfg == kCfg64W) return launch_ksplit<false, true>(g, s);
    if (is_panel_cfg(g.cfg)) return launch_panel<false, true>(g, s);
    if (direct_ok(g) || direct4_ok(g)) return launch_direct<false, true>(g, s);
    return launch_layout<false, true>(g, s);
}
}  // namespace mi
