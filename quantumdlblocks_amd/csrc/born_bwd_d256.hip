// Backward kernels for head dims 128 < D <= 256 (bf16 and fp16 inputs): the
// DMA-ring dQ and dK/dV kernels of born_bwd_d256.h, one instantiation per
// mask mode, with and without document ids, unpadded (D == 256) and padded.
#include "born_bwd.h"
#include "born_bwd_d256.h"

namespace qdl {

namespace {

template <class E, bool PAD>
hipError_t wide_modes(const BwdArgs& a, hipStream_t s) {
    if (a.doc != nullptr) {  // documents: with a causal window or none
        if (a.window > 0) return launch_bwd16_d256<E, kWindow, PAD, true>(a, s);
        return a.is_causal ? launch_bwd16_d256<E, kCausal, PAD, true>(a, s) : launch_bwd16_d256<E, kDense, PAD, true>(a, s);
    }
    if (a.window > 0)
        return a.is_causal ? launch_bwd16_d256<E, kWindow, PAD>(a, s) : launch_bwd16_d256<E, kWindowNC, PAD>(a, s);
    return a.is_causal ? launch_bwd16_d256<E, kCausal, PAD>(a, s) : launch_bwd16_d256<E, kDense, PAD>(a, s);
}

// 128 < D <= 256, a multiple of 8; documents only with a causal window or none.
template <class A>
bool wide_ok(const A& a) {
    return a.D > 128 && a.D <= 256 && a.D % 8 == 0 && (a.doc == nullptr || a.window == 0 || a.is_causal);
}

}  // namespace

template <class E>
hipError_t launch_bwd16_wide(const BwdArgs& a, hipStream_t st) {
    if (!wide_ok(a)) return hipErrorInvalidValue;
    return a.D == 256 ? wide_modes<E, false>(a, st) : wide_modes<E, true>(a, st);
}

template hipError_t launch_bwd16_wide<BF16>(const BwdArgs&, hipStream_t);
template hipError_t launch_bwd16_wide<F16>(const BwdArgs&, hipStream_t);

namespace {

template <class E, bool PAD>
hipError_t purified_modes(const PurArgs& a, hipStream_t s) {
    if (a.doc != nullptr) {
        if (a.window > 0) return launch_purified_bwd_d256<E, kWindow, PAD, true>(a, s);
        return a.is_causal ? launch_purified_bwd_d256<E, kCausal, PAD, true>(a, s)
                           : launch_purified_bwd_d256<E, kDense, PAD, true>(a, s);
    }
    if (a.window > 0)
        return a.is_causal ? launch_purified_bwd_d256<E, kWindow, PAD>(a, s)
                           : launch_purified_bwd_d256<E, kWindowNC, PAD>(a, s);
    return a.is_causal ? launch_purified_bwd_d256<E, kCausal, PAD>(a, s)
                       : launch_purified_bwd_d256<E, kDense, PAD>(a, s);
}

}  // namespace

// Purified-Born dQ and dK/dV, 128 < D <= 256 (dtype codes as in
// qdl_flash_born.h: 1 fp16, 2 bf16); the caller reduces the dgamma / dtau
// partials of the B H ceil(T / 128) dK/dV workgroups.
hipError_t purified_bwd_d256_launch(int dtype, const PurArgs& a, hipStream_t s) {
    if (!wide_ok(a)) return hipErrorInvalidValue;
    if (dtype == 1) return a.D == 256 ? purified_modes<F16, false>(a, s) : purified_modes<F16, true>(a, s);
    return a.D == 256 ? purified_modes<BF16, false>(a, s) : purified_modes<BF16, true>(a, s);
}

}  // namespace qdl
