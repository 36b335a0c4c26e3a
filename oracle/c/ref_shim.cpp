// extern "C" entry points over the reference's own CPU kernels -- TEST INFRASTRUCTURE ONLY.
// Compiled by oracle/Makefile together with the reference source
//   packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp
// where it lies under the reference tree; the output goes to oracle/_ref/ (never committed).
#include <cstdint>
#include <exception>

#include "bitnet_gemv.h"

namespace sk = sgl_kernel::bitnet;

extern "C" {

int ref_vec_dot_i2_i8(int n, float* result, const uint8_t* w, const int8_t* a) {
  try {
    sk::bitnet_vec_dot_i2_i8(n, result, w, a);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// bitnet_gemm_i2_i8: out[m * n_batch + b] (the reference's [out, batch] layout).
int ref_gemm_i2_i8(int m_out, int n_batch, int k, float* out, const uint8_t* w, const int8_t* a, float scale) {
  try {
    sk::bitnet_gemm_i2_i8(m_out, n_batch, k, out, w, a, scale);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// The op-level GEMV loop of bitnet_gemv_cpu (torch_extension_cpu.cpp:355-366): OpenMP over rows.
int ref_gemv_op(int out_features, int k, float* out, const uint8_t* w, const int8_t* a, float scale) {
  int bad = 0;
#pragma omp parallel for
  for (int i = 0; i < out_features; i++) {
    float r;
    try {
      sk::bitnet_vec_dot_i2_i8(k, &r, w + (int64_t)i * (k / 4), a);
      out[i] = r * scale;
    } catch (const std::exception&) {
      bad = 1;
    }
  }
  return bad ? -1 : 0;
}

void ref_quantize_activations_i8(int n, int8_t* out, const float* in, float* scale) {
  sk::quantize_activations_i8(n, out, in, scale);
}

}  // extern "C"
