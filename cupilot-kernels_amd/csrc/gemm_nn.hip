// gemm_nn.hip -- instantiations of the fp32 MFMA engine for op_a = n, op_b = n
// (one translation unit per operand layout so they compile in parallel).
#include "gemm_direct.hpp"
#include "gemm_panel.hpp"
#include "gemm_small.hpp"

namespace mi {
hipError_t launch_gemm_nn(const GemmLaunch& g, hipStream_t s) {
    if (g.cfg == kCfg64W) return launch_ksplit<false, false>(g, s);
    if (is_panel_cfg(g.cfg)) return launch_panel<false, false>(g, s);
    if (g.tri_cap > 0) return launch_direct_tri(g, s);
    if (direct_ok(g) || direct4_ok(g)) return launch_direct<false, false>(g, s);
    return launch_layout<false, false>(g, s);
}
}  // namespace mi
