// Batched-decode linear with LDS-staged operands (skinny_lds.h) for up to 4 tokens.
#include "skinny_lds.h"

namespace wfb {

hipError_t launch_skinny_lds_mr4(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                   const Epilogue& e, int act, int nt_pref, const NormSrc& ns, hipStream_t s) {
  if (act == WFB_ACT_SILU) return skinny_lds::launch_modes<4, WFB_ACT_SILU>(W, n, C, A, m, lda, e, nt_pref, ns, s);
  if (act == WFB_ACT_RELU2) return skinny_lds::launch_modes<4, WFB_ACT_RELU2>(W, n, C, A, m, lda, e, nt_pref, ns, s);
  return skinny_lds::launch_modes<4, 0>(W, n, C, A, m, lda, e, nt_pref, ns, s);
}

}  // namespace wfb
