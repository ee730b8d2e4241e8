// C ABI of libqdl_flash_born.so (declared in include/qdl_flash_born.h).
//
// Validates arguments, fills the kernel argument blocks and launches on the
// caller's stream.  No allocation, no synchronisation, no global state.
#include <stdint.h>

#include "../../include/qdl_flash_born.h"
#include "born_launch.h"

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, int64_t n_scale,
                 int64_t window_size, double eps) {
    if (dtype != QDL_BORN_DTYPE_F32 && dtype != QDL_BORN_DTYPE_F16 &&
        dtype != QDL_BORN_DTYPE_BF16)
        return QDL_BORN_E_DTYPE;
    if (B < 0 || H < 0 || T < 0) return QDL_BORN_E_SHAPE;
    // Grid and per-row indices are 32-bit inside the kernels.
    if (B * H > (int64_t)1 << 24 || T > (int64_t)1 << 28 || B * H * T > ((int64_t)1 << 31) - 1)
        return QDL_BORN_E_SHAPE;
    if (D < 8 || D > 256 || D % 8 != 0) return QDL_BORN_E_HEADDIM;
    if (n_scale != 1 && n_scale != H) return QDL_BORN_E_SCALE;
    if (window_size < 0 || window_size > ((int64_t)1 << 30)) return QDL_BORN_E_WINDOW;
    if (!(eps >= 0.0)) return QDL_BORN_E_SHAPE;
    return QDL_BORN_OK;
}

int hip_status(hipError_t e) { return e == hipSuccess ? QDL_BORN_OK : (int)e; }

}  // namespace

extern "C" {

const char* qdl_flash_born_version(void) { return "qdl_flash_born 0.1.0 gfx950"; }

const char* qdl_flash_born_strerror(int code) {
    switch (code) {
        case QDL_BORN_OK: return "success";
        case QDL_BORN_E_DTYPE: return "unsupported dtype (expected f32, f16 or bf16)";
        case QDL_BORN_E_SHAPE: return "invalid shape, size beyond the 32-bit index range, or negative eps";
        case QDL_BORN_E_HEADDIM: return "head dim must be a multiple of 8 in [8, 256]";
        case QDL_BORN_E_ALIGN: return "tensor base address is not 16-byte aligned";
        case QDL_BORN_E_NULL: return "required pointer is NULL";
        case QDL_BORN_E_SCALE: return "scale must hold 1 value or exactly H values";
        case QDL_BORN_E_WINDOW: return "window_size out of range";
        case QDL_BORN_E_WORKSPACE: return "workspace missing or too small";
        case QDL_BORN_E_TAU: return "tau must hold 1 value or exactly H values";
        case QDL_BORN_E_TABLE: return "rotary table invalid (n_freq above D/2, table_ld below n_freq, or sin missing)";
        case QDL_BORN_E_ROPEDIM: return "Q/K prologue head dim must be even and in [2, 256]";
        case QDL_BORN_E_SCRATCH:
            return "problem needs more backward workspace than the fixed 16 MiB array of "
                   "qdl_flash_born_bwd_noalloc (use qdl_flash_born_bwd with a caller workspace)";
        default: break;
    }
    if (code > 0) return hipGetErrorString((hipError_t)code);
    return "unknown error";
}

int qdl_flash_born_supported(int dtype, int64_t head_dim) {
    return check_common(dtype, 1, 1, 1, head_dim, 1, 0, 0.0) == QDL_BORN_OK ? 1 : 0;
}

int qdl_flash_born_fwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, const void* q,
                       const void* k, const void* v, void* out, float* z, const float* scale,
                       int64_t n_scale, const int32_t* doc_ids, int is_causal,
                       int64_t window_size, double eps, qdl_stream_t stream) {
    int rc = check_common(dtype, B, H, T, D, n_scale, window_size, eps);
    if (rc != QDL_BORN_OK) return rc;
    if (B * H * T == 0) return QDL_BORN_OK;
    if (!q || !k || !v || !out || !z || !scale) return QDL_BORN_E_NULL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return QDL_BORN_E_ALIGN;

    qdl::FwdArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = out;
    a.z = z;
    a.scale = scale;
    a.doc = doc_ids;
    a.per_head_scale = n_scale > 1 ? 1 : 0;
    a.B = (int)B;
    a.H = (int)H;
    a.T = (int)T;
    a.D = (int)D;
    a.is_causal = is_causal ? 1 : 0;
    a.window = (int)window_size;
    a.eps = (float)eps;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (dtype) {
        case QDL_BORN_DTYPE_BF16: return hip_status(qdl::fwd_launch_bf16(a, s));
        case QDL_BORN_DTYPE_F16: return hip_status(qdl::fwd_launch_f16(a, s));
        default: return hip_status(qdl::fwd_launch_f32(a, s));
    }
}

int64_t qdl_flash_born_bwd_workspace_size(int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                                          int64_t n_scale) {
    (void)dtype;
    (void)D;
    (void)n_scale;
    return qdl::bwd_workspace_bytes(B, H, T);
}

int qdl_flash_born_bwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, const void* q,
                       const void* k, const void* v, const void* out, const void* dout,
                       const float* z, const float* scale, int64_t n_scale,
                       const int32_t* doc_ids, int is_causal, int64_t window_size, double eps,
                       void* dq, void* dk, void* dv, float* dscale, void* workspace,
                       int64_t workspace_bytes, qdl_stream_t stream) {
    int rc = check_common(dtype, B, H, T, D, n_scale, window_size, eps);
    if (rc != QDL_BORN_OK) return rc;
    if (!dscale) return QDL_BORN_E_NULL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (B * H * T == 0) {
        // Empty problem: the only output with elements is dscale.
        return hip_status(qdl::zero_fill(dscale, n_scale, s));
    }
    if (!q || !k || !v || !out || !dout || !z || !scale || !dq || !dk || !dv) return QDL_BORN_E_NULL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || !aligned16(dout) ||
        !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
        return QDL_BORN_E_ALIGN;
    if (!workspace || workspace_bytes < qdl::bwd_workspace_bytes(B, H, T)) return QDL_BORN_E_WORKSPACE;
    if (!aligned16(workspace)) return QDL_BORN_E_ALIGN;

    qdl::BwdArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = out;
    a.dout = dout;
    a.z = z;
    a.scale = scale;
    a.doc = doc_ids;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    qdl::bwd_workspace_carve(workspace, B, H, T, &a.ndelta, &a.delta_z, &a.zinv, &a.dscale_part);
    a.dscale = dscale;
    a.per_head_scale = n_scale > 1 ? 1 : 0;
    a.B = (int)B;
    a.H = (int)H;
    a.T = (int)T;
    a.D = (int)D;
    a.is_causal = is_causal ? 1 : 0;
    a.window = (int)window_size;
    a.eps = (float)eps;
    switch (dtype) {
        case QDL_BORN_DTYPE_BF16: return hip_status(qdl::bwd_launch_bf16(a, s));
        case QDL_BORN_DTYPE_F16: return hip_status(qdl::bwd_launch_f16(a, s));
        default: return hip_status(qdl::bwd_launch_f32(a, s));
    }
}

int qdl_flash_born_fwd_qk_prologue(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, const void* q,
                                   const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                   const void* v, const float* cos_table, const float* sin_table,
                                   int64_t n_freq, int64_t table_ld, double norm_eps, const float* scale,
                                   int64_t n_scale, const int32_t* doc_ids, int is_causal,
                                   int64_t window_size, double eps, void* out, float* z, void* q_out,
                                   void* k_out, float* q_rinv, float* k_rinv, qdl_stream_t stream) {
    int rc = check_common(dtype, B, H, T, D, n_scale, window_size, eps);
    if (rc != QDL_BORN_OK) return rc;
    if (cos_table && (!sin_table || n_freq < 0 || n_freq > D / 2 || table_ld < n_freq)) return QDL_BORN_E_TABLE;
    if (!(norm_eps >= 0.0)) return QDL_BORN_E_SHAPE;
    if (B * H * T == 0) return QDL_BORN_OK;
    if (!q || !k || !v || !q_strides || !k_strides || !out || !z || !scale || !q_out || !k_out)
        return QDL_BORN_E_NULL;
    if (!aligned16(v) || !aligned16(out) || !aligned16(q_out) || !aligned16(k_out)) return QDL_BORN_E_ALIGN;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // bf16, D = 64, dense or causal, with or without document ids (with
    // documents also a causal window): K is normalised by the prologue kernel
    // (K alone), then one attention kernel normalises each query block as it
    // loads it (raw rows 16-byte aligned, (T + 256) rows of their time stride
    // within 32-bit offsets) and, when q_rinv is given (a backward follows),
    // writes the normalised rows and their 1/norm.
    const bool q_rows_ok = aligned16(q) && q_strides[0] % 8 == 0 && q_strides[1] % 8 == 0 &&
                           q_strides[2] % 8 == 0 && q_strides[2] >= D &&
                           (T + 256) * q_strides[2] * 2 < ((int64_t)1 << 31);
    const bool masks_ok = doc_ids ? (window_size == 0 || is_causal) : window_size == 0;
    if (dtype == QDL_BORN_DTYPE_BF16 && D == 64 && masks_ok && q_rows_ok &&
        (!cos_table || n_freq >= 1) && (T + 256) * D * 2 < ((int64_t)1 << 31)) {
        rc = qdl_flash_born_qk_prologue_fwd(dtype, B, H, T, D, nullptr, nullptr, k, k_strides, cos_table, sin_table,
                                            n_freq, table_ld, norm_eps, nullptr, k_out, nullptr, k_rinv, stream);
        if (rc != QDL_BORN_OK) return rc;
        qdl::FwdProArgs a;
        a.q = q;
        a.k = k_out;
        a.v = v;
        a.o = out;
        a.z = z;
        a.scale = scale;
        a.doc = doc_ids;
        a.per_head_scale = n_scale > 1 ? 1 : 0;
        a.B = (int)B;
        a.H = (int)H;
        a.T = (int)T;
        a.D = (int)D;
        a.is_causal = is_causal ? 1 : 0;
        a.window = (int)window_size;
        a.eps = (float)eps;
        a.q_sb = q_strides[0];
        a.q_sh = q_strides[1];
        a.q_st = q_strides[2];
        a.cos = cos_table;
        a.sin = cos_table ? sin_table : nullptr;
        a.ld = (int)table_ld;
        a.nfreq = (int)n_freq;
        a.norm_eps = (float)norm_eps;
        a.q_out = q_out;
        a.q_rinv = q_rinv;
        return hip_status(qdl::fwd_prologue_launch_bf16(a, s));
    }
    // Every other case: the prologue kernel, then the attention kernels on
    // its output (the same rows and results, two launches).
    rc = qdl_flash_born_qk_prologue_fwd(dtype, B, H, T, D, q, q_strides, k, k_strides, cos_table, sin_table,
                                        n_freq, table_ld, norm_eps, q_out, k_out, q_rinv, k_rinv, stream);
    if (rc != QDL_BORN_OK) return rc;
    return qdl_flash_born_fwd(dtype, B, H, T, D, q_out, k_out, v, out, z, scale, n_scale, doc_ids, is_causal,
                              window_size, eps, stream);
}

}  // extern "C"
