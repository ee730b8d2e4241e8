// C ABI of the purified-Born entry points of libqdl_flash_born.so (declared
// in include/qdl_flash_born.h).  Same conventions as the Born entry points:
// argument checks, no allocation, launches on the caller's stream.
#include <stdint.h>

#include "../../include/qdl_flash_born.h"
#include "born_launch.h"
#include "purified_args.h"

namespace qdl {
hipError_t purified_fwd_launch(int dtype, const PurArgs& a, hipStream_t s);
hipError_t purified_bwd_launch(int dtype, const PurArgs& a, hipStream_t s);
int64_t purified_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D);
}  // namespace qdl

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_purified(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, int64_t n_scale, int64_t n_tau,
                   int64_t window_size, double eps, double eps_base) {
    if (dtype != QDL_BORN_DTYPE_F32 && dtype != QDL_BORN_DTYPE_F16 && dtype != QDL_BORN_DTYPE_BF16)
        return QDL_BORN_E_DTYPE;
    if (B < 0 || H < 0 || T < 0) return QDL_BORN_E_SHAPE;
    if (B * H > (int64_t)1 << 24 || T > (int64_t)1 << 28 || B * H * T > ((int64_t)1 << 31) - 1)
        return QDL_BORN_E_SHAPE;
    if (D < 8 || D > 256 || D % 8 != 0) return QDL_BORN_E_HEADDIM;
    if (n_scale != 1 && n_scale != H) return QDL_BORN_E_SCALE;
    if (n_tau != 1 && n_tau != H) return QDL_BORN_E_TAU;
    if (window_size < 0 || window_size > ((int64_t)1 << 30)) return QDL_BORN_E_WINDOW;
    if (!(eps >= 0.0) || !(eps_base == eps_base)) return QDL_BORN_E_SHAPE;
    return QDL_BORN_OK;
}

int hip_status(hipError_t e) { return e == hipSuccess ? QDL_BORN_OK : (int)e; }

}  // namespace

extern "C" {

int qdl_flash_purified_born_fwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, const void* q,
                                const void* k, const void* v, float* out, float* z, const float* scale,
                                int64_t n_scale, const float* tau, int64_t n_tau, double eps_base,
                                const int32_t* doc_ids, int is_causal, int64_t window_size, double eps,
                                qdl_stream_t stream) {
    int rc = check_purified(dtype, B, H, T, D, n_scale, n_tau, window_size, eps, eps_base);
    if (rc != QDL_BORN_OK) return rc;
    if (B * H * T == 0) return QDL_BORN_OK;
    if (!q || !k || !v || !out || !z || !scale || !tau) return QDL_BORN_E_NULL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return QDL_BORN_E_ALIGN;
    qdl::PurArgs a = {};
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = out;
    a.z = z;
    a.scale = scale;
    a.tau = tau;
    a.doc = doc_ids;
    a.per_head_scale = n_scale > 1 ? 1 : 0;
    a.per_head_tau = n_tau > 1 ? 1 : 0;
    a.B = (int)B;
    a.H = (int)H;
    a.T = (int)T;
    a.D = (int)D;
    a.is_causal = is_causal ? 1 : 0;
    a.window = (int)window_size;
    a.eps = (float)eps;
    a.eps_base = (float)eps_base;
    return hip_status(qdl::purified_fwd_launch(dtype, a, reinterpret_cast<hipStream_t>(stream)));
}

int64_t qdl_flash_purified_born_bwd_workspace_size(int dtype, int64_t B, int64_t H, int64_t T, int64_t D) {
    (void)dtype;
    if (B <= 0 || H <= 0 || T <= 0 || D <= 0) return 256;
    return qdl::purified_bwd_workspace_bytes(B, H, T, D);
}

int qdl_flash_purified_born_bwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, const void* q,
                                const void* k, const void* v, const float* out, const void* dout,
                                const float* z, const float* scale, int64_t n_scale, const float* tau,
                                int64_t n_tau, double eps_base, const int32_t* doc_ids, int is_causal,
                                int64_t window_size, void* dq, void* dk, void* dv, float* dscale, float* dtau,
                                void* workspace, int64_t workspace_bytes, qdl_stream_t stream) {
    int rc = check_purified(dtype, B, H, T, D, n_scale, n_tau, window_size, 0.0, eps_base);
    if (rc != QDL_BORN_OK) return rc;
    if (!dscale || !dtau) return QDL_BORN_E_NULL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (B * H * T == 0) {
        hipError_t e = qdl::zero_fill(dscale, n_scale, s);
        if (e != hipSuccess) return hip_status(e);
        return hip_status(qdl::zero_fill(dtau, n_tau, s));
    }
    if (!q || !k || !v || !out || !dout || !z || !scale || !tau || !dq || !dk || !dv) return QDL_BORN_E_NULL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || !aligned16(dout) ||
        !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
        return QDL_BORN_E_ALIGN;
    const int64_t need = qdl::purified_bwd_workspace_bytes(B, H, T, D);
    if (!workspace || workspace_bytes < need) return QDL_BORN_E_WORKSPACE;
    if (!aligned16(workspace)) return QDL_BORN_E_ALIGN;
    qdl::PurArgs a = {};
    a.q = q;
    a.k = k;
    a.v = v;
    a.o_in = out;
    a.dout = dout;
    a.z_in = z;
    a.scale = scale;
    a.tau = tau;
    a.doc = doc_ids;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.dscale = dscale;
    a.dtau = dtau;
    const int64_t region = (B * H * T * 4 + 255) / 256 * 256;
    char* w = static_cast<char*>(workspace);
    a.ndelta = reinterpret_cast<float*>(w);
    a.zinv = reinterpret_cast<float*>(w + region);
    a.part = reinterpret_cast<float*>(w + 2 * region);
    a.per_head_scale = n_scale > 1 ? 1 : 0;
    a.per_head_tau = n_tau > 1 ? 1 : 0;
    a.B = (int)B;
    a.H = (int)H;
    a.T = (int)T;
    a.D = (int)D;
    a.is_causal = is_causal ? 1 : 0;
    a.window = (int)window_size;
    a.eps_base = (float)eps_base;
    return hip_status(qdl::purified_bwd_launch(dtype, a, s));
}

}  // extern "C"
