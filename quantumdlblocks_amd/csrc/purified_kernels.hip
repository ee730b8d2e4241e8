// Purified-Born kernel instantiations: element type x padded head dim
// (32, 64, 128, 256; the host zero-pads D to a multiple of 8 and the kernels
// bound-check columns past D).
#include "born_bwd_d128.h"
#include "born_bwd_fast.h"
#include "born_fwd_d128.h"
#include "born_fwd_doc.h"
#include "purified.h"

namespace qdl {

inline int purified_padded_dim(int D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256; }

// 16-bit inputs with document ids at head dims below 128 other than 64 (or
// with a window without causality): the generic 16-bit-MFMA kernels'
// purified mode (purified_wide.hip).
hipError_t purified_wide_fwd_launch(int dtype, const PurArgs& a, hipStream_t s);
hipError_t purified_wide_bwd_launch(int dtype, const PurArgs& a, hipStream_t s);
// 128 < D <= 256 (documents with a causal window or none): the wide-row
// DMA-ring kernels' purified mode (born_fwd_d256.hip, born_bwd_d256.hip).
hipError_t purified_fwd_d256_launch(int dtype, const PurArgs& a, hipStream_t s);
hipError_t purified_bwd_d256_launch(int dtype, const PurArgs& a, hipStream_t s);

// The bf16-MFMA kernels address one (batch, head) slice with 32-bit buffer
// offsets (rows up to T + 256 of 2 D bytes); longer slices take the generic
// kernels, as the Born dispatch does.
// Sliding windows: without documents any window (kWindow causal, kWindowNC
// not); with documents a causal one (the wavelet models' purified layers run
// causal with a window and document ids).
inline bool purified_window_ok(const PurArgs& a) { return a.window == 0 || a.is_causal; }

inline bool purified_fast_ok(const PurArgs& a) {
    return a.D == 64 && a.doc == nullptr && ((int64_t)a.T + 256) * a.D * 2 < ((int64_t)1 << 31);
}

// D < 64 (a multiple of 8) on the D = 64 kernels with the columns past D zero.
inline bool purified_narrow_ok(const PurArgs& a) {
    return a.D < 64 && a.doc == nullptr && ((int64_t)a.T + 256) * 64 * 2 < ((int64_t)1 << 31);
}

// D == 128, and 64 < D < 128 with the columns past D zero.
inline bool purified_d128_ok(const PurArgs& a) {
    return a.D > 64 && a.D <= 128 && a.doc == nullptr && ((int64_t)a.T + 256) * a.D * 2 < ((int64_t)1 << 31);
}

// 64 < D <= 128 with document ids: the D = 128 kernels' document mode (zero
// columns past D).
inline bool purified_d128_doc_ok(const PurArgs& a) {
    return a.D > 64 && a.D <= 128 && purified_window_ok(a) && a.doc != nullptr &&
           ((int64_t)a.T + 256) * a.D * 2 < ((int64_t)1 << 31);
}

inline bool purified_d256_ok(const PurArgs& a) {
    return a.D > 128 && a.D <= 256 && (a.doc == nullptr || purified_window_ok(a)) &&
           ((int64_t)a.T + 256) * a.D * 2 < ((int64_t)1 << 31);
}

inline bool purified_doc_fast_ok(const PurArgs& a) {
    return a.D == 64 && purified_window_ok(a) && a.doc != nullptr && ((int64_t)a.T + 256) * a.D * 2 < ((int64_t)1 << 31);
}

template <class IN>
static hipError_t purified_fwd_dispatch(const PurArgs& a, hipStream_t s) {
    // 16-bit inputs, D <= 128: the 16-bit-MFMA kernels with each weight split
    // into two bf16 terms for P.V (fp16: the overlap on the fp16 MFMA, V split
    // exactly into two bf16 terms).
    using E = typename std::conditional<std::is_same<IN, F16>::value, F16, BF16>::type;
    constexpr bool k16 = !std::is_same<IN, float>::value;
    // D = 64 (and below, zero columns), dense, causal or a window.
    if (k16 && purified_fast_ok(a)) {
        if (a.window > 0)
            return a.is_causal ? launch_purified_fwd_fast<kWindow, false, E>(a, s)
                               : launch_purified_fwd_fast<kWindowNC, false, E>(a, s);
        return a.is_causal ? launch_purified_fwd_fast<kCausal, false, E>(a, s)
                           : launch_purified_fwd_fast<kDense, false, E>(a, s);
    }
    if (k16 && purified_narrow_ok(a)) {
        if (a.window > 0)
            return a.is_causal ? launch_purified_fwd_fast<kWindow, true, E>(a, s)
                               : launch_purified_fwd_fast<kWindowNC, true, E>(a, s);
        return a.is_causal ? launch_purified_fwd_fast<kCausal, true, E>(a, s)
                           : launch_purified_fwd_fast<kDense, true, E>(a, s);
    }
    // 64 < D <= 128, dense, causal or a window: the D = 128 kernel's purified
    // mode.
    if (k16 && purified_d128_ok(a)) {
        if (a.D == 128) {
            if (a.window > 0)
                return a.is_causal ? launch_purified_fwd_d128<kWindow, false, E>(a, s)
                                   : launch_purified_fwd_d128<kWindowNC, false, E>(a, s);
            return a.is_causal ? launch_purified_fwd_d128<kCausal, false, E>(a, s)
                               : launch_purified_fwd_d128<kDense, false, E>(a, s);
        }
        if (a.window > 0)
            return a.is_causal ? launch_purified_fwd_d128<kWindow, true, E>(a, s)
                               : launch_purified_fwd_d128<kWindowNC, true, E>(a, s);
        return a.is_causal ? launch_purified_fwd_d128<kCausal, true, E>(a, s)
                           : launch_purified_fwd_d128<kDense, true, E>(a, s);
    }
    // D = 128, document ids (with or without a causal window): its document
    // mode.
    if (k16 && purified_d128_doc_ok(a)) {
        if (a.D < 128) {
            if (a.window > 0) return launch_purified_fwd_d128_doc<kWindow, E, true>(a, s);
            return a.is_causal ? launch_purified_fwd_d128_doc<kCausal, E, true>(a, s)
                               : launch_purified_fwd_d128_doc<kDense, E, true>(a, s);
        }
        if (a.window > 0) return launch_purified_fwd_d128_doc<kWindow, E>(a, s);
        return a.is_causal ? launch_purified_fwd_d128_doc<kCausal, E>(a, s)
                           : launch_purified_fwd_d128_doc<kDense, E>(a, s);
    }
    // D = 64, document ids (with or without a causal window): the document
    // kernel's purified mode.
    if (k16 && purified_doc_fast_ok(a))
        return a.window > 0 ? launch_purified_fwd_doc<true, E>(a, s) : launch_purified_fwd_doc<false, E>(a, s);
    // Above D = 128, and documents at other head dims: the generic
    // 16-bit-MFMA kernels' purified mode.
    if (k16 && purified_d256_ok(a)) return purified_fwd_d256_launch(E::kDtype, a, s);
    if (k16 && (a.D > 128 || a.doc != nullptr)) return purified_wide_fwd_launch(E::kDtype, a, s);
    switch (purified_padded_dim(a.D)) {
        case 32: return launch_purified_fwd<IN, 32>(a, s);
        case 64: return launch_purified_fwd<IN, 64>(a, s);
        case 128: return launch_purified_fwd<IN, 128>(a, s);
        default: return launch_purified_fwd<IN, 256>(a, s);
    }
}
// 16-bit, D = 64: the 16-bit-MFMA dQ kernel (which also writes -delta and
// 1/Z) before the dK/dV kernel (which writes the dgamma / dtau partials), then
// the fixed-order reduction.  E: the input dtype, to which the reference
// rounds p/Z and dR before their contractions (flash_born.py:926, 939, 1058).
template <int MODE, bool DOC = false, bool PAD = false, class E = BF16>
static hipError_t purified_bwd_fast(const PurArgs& a, hipStream_t s) {
    // dQ: 256-row blocks of 4 waves, 128-row blocks of 2 with documents.
    constexpr int NW = DOC ? 2 : 4;
    hipLaunchKernelGGL((born_bwd16_dq_fast_kernel<E, 64, MODE, true, DOC, PAD, NW>),
                       dim3((unsigned)bwd16_dq_fast_groups(a.B, a.H, a.T, DOC)), dim3(64 * NW), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nwg = purified_dkdv_groups(a.B, a.H, a.T, 64);
    hipLaunchKernelGGL((born_bwd16_dkdv_fast_kernel<E, 64, MODE, true, DOC, PAD>), dim3((unsigned)nwg), dim3(256), 0,
                       s, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int n_scale = a.per_head_scale ? a.H : 1, n_tau = a.per_head_tau ? a.H : 1;
    hipLaunchKernelGGL(purified_param_reduce_kernel<0>, dim3((unsigned)(n_scale + n_tau)), dim3(256), 0, s, a, nwg, n_scale);
    return hipGetLastError();
}

// 16-bit, 64 < D <= 128: the D = 128 dQ and dK/dV kernels' purified mode,
// then the same reduction.
template <int MODE, bool DOC = false, class E = BF16>
static hipError_t purified_bwd_d128(const PurArgs& a, hipStream_t s) {
    hipError_t e = a.D == 128 ? launch_purified_bwd_d128<MODE, false, DOC, E>(a, s)
                              : launch_purified_bwd_d128<MODE, true, DOC, E>(a, s);
    if (e != hipSuccess) return e;
    // dK/dV workgroups: 128-key blocks, 64-key blocks with documents.
    const int nwg = DOC ? ((a.T + 63) / 64) * a.B * a.H : purified_dkdv_groups(a.B, a.H, a.T, 128);
    const int n_scale = a.per_head_scale ? a.H : 1, n_tau = a.per_head_tau ? a.H : 1;
    hipLaunchKernelGGL(purified_param_reduce_kernel<0>, dim3((unsigned)(n_scale + n_tau)), dim3(256), 0, s, a, nwg, n_scale);
    return hipGetLastError();
}

template <class IN>
static hipError_t purified_bwd_dispatch(const PurArgs& a, hipStream_t s) {
    // 16-bit inputs: the 16-bit-MFMA backward kernels (bf16 and fp16 alike:
    // the reference rounds p/Z and dR to the input dtype before its dots).
    using E = typename std::conditional<std::is_same<IN, F16>::value, F16, BF16>::type;
    constexpr bool k16 = !std::is_same<IN, float>::value;
    if (k16 && purified_fast_ok(a)) {
        if (a.window > 0)
            return a.is_causal ? purified_bwd_fast<kWindow, false, false, E>(a, s)
                               : purified_bwd_fast<kWindowNC, false, false, E>(a, s);
        return a.is_causal ? purified_bwd_fast<kCausal, false, false, E>(a, s)
                           : purified_bwd_fast<kDense, false, false, E>(a, s);
    }
    if (k16 && purified_narrow_ok(a)) {
        if (a.window > 0)
            return a.is_causal ? purified_bwd_fast<kWindow, false, true, E>(a, s)
                               : purified_bwd_fast<kWindowNC, false, true, E>(a, s);
        return a.is_causal ? purified_bwd_fast<kCausal, false, true, E>(a, s)
                           : purified_bwd_fast<kDense, false, true, E>(a, s);
    }
    if (k16 && purified_d128_ok(a)) {
        if (a.window > 0)
            return a.is_causal ? purified_bwd_d128<kWindow, false, E>(a, s) : purified_bwd_d128<kWindowNC, false, E>(a, s);
        return a.is_causal ? purified_bwd_d128<kCausal, false, E>(a, s) : purified_bwd_d128<kDense, false, E>(a, s);
    }
    if (k16 && purified_d128_doc_ok(a)) {
        if (a.window > 0) return purified_bwd_d128<kWindow, true, E>(a, s);
        return a.is_causal ? purified_bwd_d128<kCausal, true, E>(a, s) : purified_bwd_d128<kDense, true, E>(a, s);
    }
    // D = 64, document ids (with or without a causal window): the same
    // kernels' document variants.
    if (k16 && purified_doc_fast_ok(a)) {
        if (a.window > 0) return purified_bwd_fast<kWindow, true, false, E>(a, s);
        return a.is_causal ? purified_bwd_fast<kCausal, true, false, E>(a, s)
                           : purified_bwd_fast<kDense, true, false, E>(a, s);
    }
    if (k16 && purified_d256_ok(a)) {
        hipError_t e = purified_bwd_d256_launch(E::kDtype, a, s);
        if (e != hipSuccess) return e;
        const int nwg = ((a.T + 127) / 128) * a.B * a.H;
        const int n_scale = a.per_head_scale ? a.H : 1, n_tau = a.per_head_tau ? a.H : 1;
        hipLaunchKernelGGL(purified_param_reduce_kernel<0>, dim3((unsigned)(n_scale + n_tau)), dim3(256), 0, s, a, nwg,
                           n_scale);
        return hipGetLastError();
    }
    if (k16 && (a.D > 128 || a.doc != nullptr)) return purified_wide_bwd_launch(E::kDtype, a, s);
    switch (purified_padded_dim(a.D)) {
        case 32: return launch_purified_bwd<IN, 32>(a, s);
        case 64: return launch_purified_bwd<IN, 64>(a, s);
        case 128: return launch_purified_bwd<IN, 128>(a, s);
        default: return launch_purified_bwd<IN, 256>(a, s);
    }
}

// dtype codes as in qdl_flash_born.h: 0 fp32, 1 fp16, 2 bf16.
hipError_t purified_fwd_launch(int dtype, const PurArgs& a, hipStream_t s) {
    if (dtype == 0) return purified_fwd_dispatch<float>(a, s);
    if (dtype == 1) return purified_fwd_dispatch<F16>(a, s);
    return purified_fwd_dispatch<BF16>(a, s);
}
hipError_t purified_bwd_launch(int dtype, const PurArgs& a, hipStream_t s) {
    if (dtype == 0) return purified_bwd_dispatch<float>(a, s);
    if (dtype == 1) return purified_bwd_dispatch<F16>(a, s);
    return purified_bwd_dispatch<BF16>(a, s);
}
int64_t purified_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D) {
    const int64_t region = (B * H * T * 4 + 255) / 256 * 256;
    const int64_t nwg = purified_dkdv_groups_max((int)B, (int)H, (int)T, purified_padded_dim((int)D));
    return 2 * region + (2 * nwg * 4 + 255) / 256 * 256;
}

}  // namespace qdl
