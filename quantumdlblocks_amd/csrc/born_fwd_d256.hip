// Forward kernels for head dims 128 < D <= 256 (bf16 and fp16 inputs): the
// DMA-ring kernel of born_fwd_d256.h, one instantiation per mask mode, with
// and without document ids, unpadded (D == 256) and padded.
#include "born_fwd.h"
#include "born_fwd_d256.h"

namespace qdl {

namespace {

template <class E, bool PAD, bool PUR, class A>
hipError_t wide_modes(const A& a, hipStream_t s) {
    if (a.doc != nullptr) {  // documents: with a causal window or none
        if (a.window > 0) return launch_fwd16_d256<E, kWindow, PAD, PUR, true>(a, s);
        return a.is_causal ? launch_fwd16_d256<E, kCausal, PAD, PUR, true>(a, s)
                           : launch_fwd16_d256<E, kDense, PAD, PUR, true>(a, s);
    }
    if (a.window > 0)
        return a.is_causal ? launch_fwd16_d256<E, kWindow, PAD, PUR>(a, s) : launch_fwd16_d256<E, kWindowNC, PAD, PUR>(a, s);
    return a.is_causal ? launch_fwd16_d256<E, kCausal, PAD, PUR>(a, s) : launch_fwd16_d256<E, kDense, PAD, PUR>(a, s);
}

// 128 < D <= 256, a multiple of 8; documents only with a causal window or none.
template <class A>
bool wide_ok(const A& a) {
    return a.D > 128 && a.D <= 256 && a.D % 8 == 0 && (a.doc == nullptr || a.window == 0 || a.is_causal);
}

}  // namespace

template <class E>
hipError_t launch_fwd16_wide(const FwdArgs& a, hipStream_t st) {
    if (!wide_ok(a)) return hipErrorInvalidValue;
    return a.D == 256 ? wide_modes<E, false, false>(a, st) : wide_modes<E, true, false>(a, st);
}

template hipError_t launch_fwd16_wide<BF16>(const FwdArgs&, hipStream_t);
template hipError_t launch_fwd16_wide<F16>(const FwdArgs&, hipStream_t);

// Purified-Born forward, 128 < D <= 256 (dtype codes as in qdl_flash_born.h:
// 1 fp16, 2 bf16).
hipError_t purified_fwd_d256_launch(int dtype, const PurArgs& a, hipStream_t s) {
    if (!wide_ok(a)) return hipErrorInvalidValue;
    if (dtype == 1) return a.D == 256 ? wide_modes<F16, false, true>(a, s) : wide_modes<F16, true, true>(a, s);
    return a.D == 256 ? wide_modes<BF16, false, true>(a, s) : wide_modes<BF16, true, true>(a, s);
}

}  // namespace qdl
