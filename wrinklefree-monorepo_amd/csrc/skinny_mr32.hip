// Batched-decode linear with LDS-staged operands (skinny_lds.h) for 17..32 tokens: two 16-token tiles
// per weight fragment (codes path, activations staged in LDS).
#include "skinny_lds.h"

namespace wfb {

hipError_t launch_skinny_lds_mr32(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                   const Epilogue& e, int act, int nt_pref, const NormSrc& ns, hipStream_t s) {
  if (act == WFB_ACT_SILU) return skinny_lds::launch_modes<32, WFB_ACT_SILU>(W, n, C, A, m, lda, e, nt_pref, ns, s);
  if (act == WFB_ACT_RELU2) return skinny_lds::launch_modes<32, WFB_ACT_RELU2>(W, n, C, A, m, lda, e, nt_pref, ns, s);
  return skinny_lds::launch_modes<32, 0>(W, n, C, A, m, lda, e, nt_pref, ns, s);
}

}  // namespace wfb
