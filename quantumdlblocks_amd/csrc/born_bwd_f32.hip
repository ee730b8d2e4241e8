// Backward kernel instantiations for fp32 inputs.
#include "born_bwd.h"
#include "born_launch.h"

namespace qdl {

hipError_t bwd_launch_f32(const BwdArgs& a, hipStream_t s) {
    const int dp = padded_head_dim(a.D);
    const int mode = mask_mode(a.is_causal, a.window, a.doc);
#define QDL_MODE_BODY(M) return launch_bwd32<DPV, M>(a, s);
#define QDL_DP_BODY(D_) { constexpr int DPV = D_; QDL_SWITCH_MODE(mode, QDL_MODE_BODY) }
    QDL_SWITCH_DP(dp, QDL_DP_BODY)
#undef QDL_DP_BODY
#undef QDL_MODE_BODY
    return hipErrorInvalidValue;
}

}  // namespace qdl
