// Gated activation (silu(gate) * up or relu(gate)^2 * up) fused with RMSNorm/SubLN and the
// per-token int8 quantiser: the middle of the BitNet MLP between the gate|up and down projections
// (bitnet_mlp_fused, SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:200-216).  Own translation unit
// so the kernel variants compile in parallel with quant.hip.
#include "quant_rows.h"

namespace wfb {

hipError_t launch_glu_quant_rows(const void* gate, const void* up, int dt, int64_t ldx, int act, const void* gamma,
                                 int gdt, float eps, int64_t m, int64_t h, int8_t* q, int64_t k_pad, int64_t ldq,
                                 float* a_scale, hipStream_t s) {
  if (m == 0) return hipSuccess;
#define WFB_GLU(D, A) launch_rows_g<D, true, A>(gate, up, ldx, gamma, gdt, eps, m, h, q, k_pad, ldq, a_scale, s)
  if (act == WFB_ACT_SILU) {
    if (dt == WFB_F32) return WFB_GLU(WFB_F32, 1);
    if (dt == WFB_BF16) return WFB_GLU(WFB_BF16, 1);
    return WFB_GLU(WFB_F16, 1);
  }
  if (dt == WFB_F32) return WFB_GLU(WFB_F32, 2);
  if (dt == WFB_BF16) return WFB_GLU(WFB_BF16, 2);
  return WFB_GLU(WFB_F16, 2);
#undef WFB_GLU
}

}  // namespace wfb
