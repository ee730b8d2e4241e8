// qdl_flash_born_bwd_noalloc: the Born backward with its workspace taken from
// a fixed device array inside the library instead of from the caller.
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).  The
// workspace (-delta, delta/Z, 1/Z and the dscale partials) lives in the
// file-scope array `scratch`; each GPU the library runs on holds its own copy
// of it until the process ends.  The host never passes the array's name to a
// kernel: its device address is looked up once per device with
// hipGetSymbolAddress and kept.  Every region of the workspace is written by
// a call before that call reads it, so nothing has to be cleared between
// calls; calls that overlap on one GPU share the array and race.
#include <stdint.h>

#include <mutex>

#include "../../include/qdl_flash_born.h"
#include "born_launch.h"

static __device__ __align__(256) uint8_t scratch[QDL_BORN_BWD_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call on that device, with that device current).
int scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (p == nullptr) return (int)hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return QDL_BORN_OK;
}

}  // namespace

extern "C" int qdl_flash_born_bwd_noalloc(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, const void* q,
                                          const void* k, const void* v, const void* out, const void* dout,
                                          const float* z, const float* scale, int64_t n_scale,
                                          const int32_t* doc_ids, int is_causal, int64_t window_size,
                                          double eps, void* dq, void* dk, void* dv, float* dscale,
                                          qdl_stream_t stream) {
    // Shape checks first, so an oversized problem is rejected before any HIP call.
    if (B >= 0 && H >= 0 && T >= 0 && B * H * T > 0 && B * H * T <= ((int64_t)1 << 31) - 1 &&
        qdl::bwd_workspace_bytes(B, H, T) > (int64_t)QDL_BORN_BWD_SCRATCH_BYTES)
        return QDL_BORN_E_SCRATCH;
    void* ws = nullptr;
    if (B > 0 && H > 0 && T > 0) {
        const int rc = scratch_address(&ws);
        if (rc != QDL_BORN_OK) return rc;
    }
    return qdl_flash_born_bwd(dtype, B, H, T, D, q, k, v, out, dout, z, scale, n_scale, doc_ids, is_causal,
                              window_size, eps, dq, dk, dv, dscale, ws, (int64_t)QDL_BORN_BWD_SCRATCH_BYTES, stream);
}
