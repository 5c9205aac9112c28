// The verify kernel's instantiations with an affine 4-bit (gs 64) shared expert (the reference checkpoint's format:
// gate / up / down as packed words with bf16 group scales and biases), dispatched from launch_verify when sh_gs is
// set. Kept apart from the bf16-shared instantiations so that neither pays for the other's branches.
#include "ss_verify_kernel.hpp"

namespace ss {

template <int NJG, int NJD>
static hipError_t launch_x_q4(const VerifyArgs& a, hipStream_t st) {
  return a.x_f32 ? launch_nj<NJG, NJD, true, true>(a, st) : launch_nj<NJG, NJD, false, true>(a, st);
}

hipError_t launch_verify_q4(const VerifyArgs& a, hipStream_t st) {
  const int njg = a.H / 128, njd = a.I / 128;
#define SS_CASE(G_, D_) \
  if (njg == G_ && njd == D_) return launch_x_q4<G_, D_>(a, st);
#define SS_ROW(G_) SS_CASE(G_, 1) SS_CASE(G_, 2) SS_CASE(G_, 4) SS_CASE(G_, 5) SS_CASE(G_, 8)
  SS_ROW(8)
  SS_ROW(16)
  SS_ROW(20)
  SS_ROW(32)
#undef SS_ROW
#undef SS_CASE
  return hipErrorInvalidValue;
}

}  // namespace ss
