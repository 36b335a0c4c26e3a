// Batched-decode linear with LDS-staged operands (skinny_lds.h) for 33..64 tokens: four 16-token tiles
// per weight fragment (plain linear, codes path; activations staged one step at a time where the LDS
// holds them, else in registers).
#include "skinny_lds.h"

namespace wfb {

hipError_t launch_skinny_lds_mr64(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                   const Epilogue& e, int act, int nt_pref, const NormSrc& ns, hipStream_t s) {
  if (act != 0) return hipErrorNotSupported;  // the gated form pairs two row tiles per workgroup
  return skinny_lds::launch_modes<64, 0>(W, n, C, A, m, lda, e, nt_pref, ns, s);
}

}  // namespace wfb
