// Host-side launch helpers: pick the compiled kernel for (dtype, padded head
// dim, mask mode) and launch it on the caller's stream.
#pragma once

#include "born_common.h"

namespace qdl {

// Padded head dim served by the kernels: D rounded up to a multiple of 32.
inline int padded_head_dim(int D) { return (D + 31) / 32 * 32; }

inline int mask_mode(int is_causal, int window, const int32_t* doc) {
    if (doc != nullptr || window > 0) return kGeneral;
    return is_causal ? kCausal : kDense;
}

// Entry points of the per-dtype translation units.
hipError_t fwd_launch_bf16(const FwdArgs& a, hipStream_t s);
hipError_t fwd_launch_f16(const FwdArgs& a, hipStream_t s);
hipError_t fwd_launch_f32(const FwdArgs& a, hipStream_t s);
hipError_t bwd_launch_bf16(const BwdArgs& a, hipStream_t s);
// The forward with the Q/K prologue fused into its loads (bf16, D == 64, dense
// or causal); hipErrorInvalidValue for anything else.
hipError_t fwd_prologue_launch_bf16(const FwdProArgs& a, hipStream_t s);
hipError_t bwd_launch_f16(const BwdArgs& a, hipStream_t s);
hipError_t bwd_launch_f32(const BwdArgs& a, hipStream_t s);

}  // namespace qdl

// Expands `BODY(DPV)` for the runtime padded head dim `dp`.
#define QDL_SWITCH_DP(dp, BODY)                       \
    switch (dp) {                                     \
        case 32: { BODY(32); } break;                 \
        case 64: { BODY(64); } break;                 \
        case 96: { BODY(96); } break;                 \
        case 128: { BODY(128); } break;               \
        case 160: { BODY(160); } break;               \
        case 192: { BODY(192); } break;               \
        case 224: { BODY(224); } break;               \
        case 256: { BODY(256); } break;               \
        default: return hipErrorInvalidValue;         \
    }

#define QDL_SWITCH_MODE(mode, BODY)                   \
    switch (mode) {                                   \
        case qdl::kDense: { BODY(qdl::kDense); } break;     \
        case qdl::kCausal: { BODY(qdl::kCausal); } break;   \
        default: { BODY(qdl::kGeneral); } break;      \
    }

namespace qdl {
// Backward workspace (each region 256-byte aligned):
//   ndelta  = -(dO . O)       (B*H*T fp32)
//   delta_z = dO . O / Z      (B*H*T fp32)
//   zinv    = 1 / Z           (B*H*T fp32)
//   dscale partial sums       (fp64: H * DSCALE_CHUNKS, or one per workgroup of
//                              the D = 64 dQ kernel -- 128-row blocks with
//                              documents -- whichever is more)
inline int64_t bwd_region_bytes(int64_t B, int64_t H, int64_t T) {
    return ((B * H * T * 4) + 255) / 256 * 256;
}
inline int64_t bwd_partial_bytes(int64_t B, int64_t H, int64_t T) {
    const int64_t chunks = (H > 1 ? H : 1) * DSCALE_CHUNKS;
    const int64_t groups = B * H * ((T + 127) / 128);
    const int64_t n = (chunks > groups ? chunks : groups) * 8;
    return (n + 255) / 256 * 256;
}
inline int64_t bwd_workspace_bytes(int64_t B, int64_t H, int64_t T) {
    return 3 * bwd_region_bytes(B, H, T) + bwd_partial_bytes(B, H, T);
}
inline void bwd_workspace_carve(void* ws, int64_t B, int64_t H, int64_t T, float** ndelta,
                                float** delta_z, float** zinv, double** part) {
    char* p = static_cast<char*>(ws);
    const int64_t r = bwd_region_bytes(B, H, T);
    *ndelta = reinterpret_cast<float*>(p);
    *delta_z = reinterpret_cast<float*>(p + r);
    *zinv = reinterpret_cast<float*>(p + 2 * r);
    *part = reinterpret_cast<double*>(p + 3 * r);
}
}  // namespace qdl

namespace qdl {
// Zero `n` floats with a kernel (graph-capture friendly; no memset node).
hipError_t zero_fill(float* p, int64_t n, hipStream_t s);
}  // namespace qdl
