// Forward kernel instantiations for bf16 inputs.
#include "born_fwd.h"
#include "born_fwd_d128.h"
#include "born_fwd_doc.h"
#include "born_fwd_fast.h"
#include "born_launch.h"

namespace qdl {

hipError_t fwd_launch_bf16(const FwdArgs& a, hipStream_t s) {
    const int dp = padded_head_dim(a.D);
    const int mode = mask_mode(a.is_causal, a.window, a.doc);
    // Hot path: D == 64 exactly, dense or causal, per-head slice addressable
    // with 32-bit buffer offsets.
    const bool addr32 = ((int64_t)a.T + 256) * a.D * 2 < ((int64_t)1 << 31);
    // Documents (no window): the document-aware fast kernel.
    if (a.D == 64 && a.doc != nullptr && a.window == 0 && addr32) return launch_fwd16_doc<BF16, 64>(a, s);
    // Documents with a causal sliding window: the same kernel's window mode.
    if (a.D == 64 && a.doc != nullptr && a.window > 0 && a.is_causal && addr32)
        return launch_fwd16_doc<BF16, 64, true>(a, s);
    // Causal sliding window (no documents): the fast kernel's window mode.
    if (a.D == 64 && a.doc == nullptr && a.window > 0 && a.is_causal && addr32)
        return launch_fwd16_fast<BF16, 64, kWindow>(a, s);
    // Sliding window without causality (no documents): its kWindowNC mode.
    if (a.D == 64 && a.doc == nullptr && a.window > 0 && !a.is_causal && addr32)
        return launch_fwd16_fast<BF16, 64, kWindowNC>(a, s);
    // D == 128 with document ids (and a causal window): the D == 128 kernel's
    // document mode.
    // 64 < D < 128 with documents on the same kernel with zero columns past D.
    if (a.D > 64 && a.D <= 128 && a.doc != nullptr && addr32 && (a.window == 0 || a.is_causal)) {
        if (a.D < 128) {
            if (a.window > 0) return launch_fwd16_d128_doc<BF16, kWindow, true>(a, s);
            return a.is_causal ? launch_fwd16_d128_doc<BF16, kCausal, true>(a, s)
                               : launch_fwd16_d128_doc<BF16, kDense, true>(a, s);
        }
        if (a.window > 0) return launch_fwd16_d128_doc<BF16, kWindow>(a, s);
        return a.is_causal ? launch_fwd16_d128_doc<BF16, kCausal>(a, s) : launch_fwd16_d128_doc<BF16, kDense>(a, s);
    }
    // D == 128: dense, causal or a sliding window with or without causality
    // (no documents).
    if (a.D == 128 && a.doc == nullptr && addr32) {
        if (a.window > 0)
            return a.is_causal ? launch_fwd16_d128<BF16, kWindow>(a, s) : launch_fwd16_d128<BF16, kWindowNC>(a, s);
        return a.is_causal ? launch_fwd16_d128<BF16, kCausal>(a, s) : launch_fwd16_d128<BF16, kDense>(a, s);
    }
    // 128 < D <= 256 (documents with a causal window or none): the DMA-ring
    // kernel for wide rows.
    if (a.D > 128 && addr32 && (a.doc == nullptr || a.window == 0 || a.is_causal))
        return launch_fwd16_wide<BF16>(a, s);
    if (a.D == 64 && mode != kGeneral && addr32)
        return mode == kCausal ? launch_fwd16_fast<BF16, 64, kCausal>(a, s) : launch_fwd16_fast<BF16, 64, kDense>(a, s);
#define QDL_MODE_BODY(M) return launch_fwd16<BF16, DPV, M>(a, s);
#define QDL_DP_BODY(D_) { constexpr int DPV = D_; QDL_SWITCH_MODE(mode, QDL_MODE_BODY) }
    QDL_SWITCH_DP(dp, QDL_DP_BODY)
#undef QDL_DP_BODY
#undef QDL_MODE_BODY
    return hipErrorInvalidValue;
}

hipError_t fwd_prologue_launch_bf16(const FwdProArgs& a, hipStream_t s) {
    if (a.D != 64) return hipErrorInvalidValue;
    // Documents (with or without a causal window): the document kernel.
    if (a.doc != nullptr) {
        if (a.window == 0) return launch_fwd16_doc_prologue<false>(a, s);
        return a.is_causal ? launch_fwd16_doc_prologue<true>(a, s) : hipErrorInvalidValue;
    }
    if (a.window != 0) return hipErrorInvalidValue;
    return a.is_causal ? launch_fwd16_fast_prologue<kCausal>(a, s) : launch_fwd16_fast_prologue<kDense>(a, s);
}

}  // namespace qdl
