// Purified-Born attention at head dims above 128, and with document ids at
// head dims other than 64 and 128 (bf16 / fp16 inputs), on the
// register-staged 16-bit-MFMA kernels of the Born generic path (born_fwd.h,
// born_bwd.h), in their purified mode: the overlap, dP and the backward's
// three contractions on the 16-bit MFMA (the reference rounds p/Z and dR to
// the input dtype before its dots, flash_born.py:926, 939, 1058), the
// forward's P.V on the bf16 MFMA with the fp32 weights split into two bf16
// terms (and fp16 V split exactly into two).  One instantiation per padded
// head dim (32 to 256 in steps of 32), with the masks (causal, window,
// documents) as runtime flags.
#include "born_bwd.h"
#include "born_fwd.h"
#include "born_launch.h"
#include "purified.h"

namespace qdl {

namespace {

// One wave per SIMD at every head dim (the purified elementwise pass and the
// split weights need more registers than Born's: at two waves per SIMD the
// DP = 64 and 128 kernels spill 56-148 bytes per lane).
template <class E, int DP>
hipError_t wide_fwd(const PurArgs& a, hipStream_t st) {
    using C = Fwd16Cfg<DP>;
    const unsigned nmb = (unsigned)((a.T + C::BM - 1) / C::BM);
    hipLaunchKernelGGL((born_fwd16_kernel<E, DP, C::NQB, C::NW, C::BN, kGeneral, 1, true>),
                       dim3(nmb * (unsigned)(a.B * a.H)), dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

// -delta and 1/Z per row, then dK/dV (with the dgamma / dtau partials), dQ,
// and the fixed-order reduction of the partials.
template <class E, int DP>
hipError_t wide_bwd(const PurArgs& a, hipStream_t st) {
    using C = Bwd16Cfg<DP>;
    const unsigned BH = (unsigned)(a.B * a.H);
    {
        int n = (a.D + 3) / 4, G = 1;
        while (G < n && G < 32) G <<= 1;
        const int64_t rows = (int64_t)a.B * a.H * a.T;
        const int per_block = 256 / G;
        hipLaunchKernelGGL((purified_delta_kernel<E>), dim3((unsigned)((rows + per_block - 1) / per_block)),
                           dim3(256), 0, st, a, G);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // dK/dV in two column halves above DP = 128 (the purified elementwise
    // pass needs more registers than Born's: unsplit, DP = 160 spills 92
    // bytes per lane).
    constexpr int BK = C::NW * 32, CS = DP > 128 ? 2 : 1;
    const int nwg = ((a.T + BK - 1) / BK) * (int)BH;
    hipLaunchKernelGGL((born_bwd_dkdv16_kernel<E, DP, C::NW, C::KV_BQ, kGeneral, 1, CS, true>),
                       dim3((unsigned)nwg * CS), dim3(C::NW * 64), 0, st, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    constexpr int BM = C::NW * 32 * C::DQ_NQB;
    hipLaunchKernelGGL((born_bwd_dq16_kernel<E, DP, C::DQ_NQB, C::NW, C::DQ_BN, kGeneral, 1, true>),
                       dim3((unsigned)((a.T + BM - 1) / BM) * BH), dim3(C::NW * 64), 0, st, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int n_scale = a.per_head_scale ? a.H : 1, n_tau = a.per_head_tau ? a.H : 1;
    hipLaunchKernelGGL(purified_param_reduce_kernel<0>, dim3((unsigned)(n_scale + n_tau)), dim3(256), 0, st, a, nwg,
                       n_scale);
    return hipGetLastError();
}

template <class E>
hipError_t wide_fwd_dp(const PurArgs& a, hipStream_t st) {
    switch (padded_head_dim(a.D)) {
        case 32: return wide_fwd<E, 32>(a, st);
        case 64: return wide_fwd<E, 64>(a, st);
        case 96: return wide_fwd<E, 96>(a, st);
        case 128: return wide_fwd<E, 128>(a, st);
        case 160: return wide_fwd<E, 160>(a, st);
        case 192: return wide_fwd<E, 192>(a, st);
        case 224: return wide_fwd<E, 224>(a, st);
        case 256: return wide_fwd<E, 256>(a, st);
        default: return hipErrorInvalidValue;
    }
}

template <class E>
hipError_t wide_bwd_dp(const PurArgs& a, hipStream_t st) {
    switch (padded_head_dim(a.D)) {
        case 32: return wide_bwd<E, 32>(a, st);
        case 64: return wide_bwd<E, 64>(a, st);
        case 96: return wide_bwd<E, 96>(a, st);
        case 128: return wide_bwd<E, 128>(a, st);
        case 160: return wide_bwd<E, 160>(a, st);
        case 192: return wide_bwd<E, 192>(a, st);
        case 224: return wide_bwd<E, 224>(a, st);
        case 256: return wide_bwd<E, 256>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

// dtype codes as in qdl_flash_born.h: 1 fp16, 2 bf16 (fp32 is not taken here).
hipError_t purified_wide_fwd_launch(int dtype, const PurArgs& a, hipStream_t s) {
    return dtype == 1 ? wide_fwd_dp<F16>(a, s) : wide_fwd_dp<BF16>(a, s);
}

hipError_t purified_wide_bwd_launch(int dtype, const PurArgs& a, hipStream_t s) {
    return dtype == 1 ? wide_bwd_dp<F16>(a, s) : wide_bwd_dp<BF16>(a, s);
}

}  // namespace qdl
