// gemm_tn.hip -- instantiations of the fp32 MFMA engine for op_a = t, op_b = n
// (one translation unit per operand layout so they compile in parallel).
#include "gemm_panel.hpp"

namespace mi {
hipError_t launch_gemm_tn(const GemmLaunch& g, hipStream_t s) {
    return is_panel_cfg(g.cfg) ? launch_panel<true, false>(g, s) : launch_layout<true, false>(g, s);
}
}  // namespace mi
