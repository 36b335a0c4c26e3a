// Activation quantisation entry points: per-token absmax int8 (optionally fused behind RMSNorm/SubLN;
// kernels in quant_rows.h) and the per-tensor variant of the reference torch op
// (SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:409-426).
#include "quant_rows.h"

namespace wfb {

namespace {

// ---- per-tensor (one scale for the whole buffer) -------------------------------------------

__global__ void zero_u32_kernel(uint32_t* p) { *p = 0u; }

template <int DT>
__global__ __launch_bounds__(256) void absmax_tensor_kernel(const void* __restrict__ x, int64_t numel,
                                                            uint32_t* __restrict__ mx_bits) {
  __shared__ float red[4];
  float mx = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel; i += (int64_t)gridDim.x * blockDim.x)
    mx = fmaxf(mx, fabsf(load_elem<DT>(x, i)));
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // non-negative floats order like their bit patterns
    atomicMax(mx_bits, __float_as_uint(mx));
  }
}

template <int DT>
__global__ __launch_bounds__(256) void quant_tensor_kernel(const void* __restrict__ x, int64_t numel,
                                                           const uint32_t* __restrict__ mx_bits,
                                                           int8_t* __restrict__ q) {
  float mx = __uint_as_float(*mx_bits);
  if (mx < 1e-6f) mx = 1.0f;
  const float inv = __fdiv_rn(127.0f, mx);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel; i += (int64_t)gridDim.x * blockDim.x)
    q[i] = (int8_t)quant_i8(load_elem<DT>(x, i), inv);
}

__global__ void finish_tensor_scale_kernel(float* a_scale) {
  float mx = a_scale[0];  // still holds the absmax bits
  if (mx < 1e-6f) mx = 1.0f;
  a_scale[0] = __fdiv_rn(mx, 127.0f);
}

template <int DT>
hipError_t launch_tensor_t(const void* x, int64_t numel, int8_t* q, float* a_scale, hipStream_t s) {
  uint32_t* bits = reinterpret_cast<uint32_t*>(a_scale);
  hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(1), 0, s, bits);
  int64_t blocks = (numel + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((absmax_tensor_kernel<DT>), dim3((unsigned)blocks), dim3(256), 0, s, x, numel, bits);
  hipLaunchKernelGGL((quant_tensor_kernel<DT>), dim3((unsigned)blocks), dim3(256), 0, s, x, numel, bits, q);
  hipLaunchKernelGGL(finish_tensor_scale_kernel, dim3(1), dim3(1), 0, s, a_scale);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quant_rows(const void* x, int dt, int64_t ldx, const void* gamma, int gdt, bool norm,
                             float eps, int64_t m, int64_t h, int8_t* q, int64_t k_pad, int64_t ldq,
                             float* a_scale, hipStream_t s) {
  if (m == 0) return hipSuccess;
  if (norm) {
    if (dt == WFB_F32)
      return launch_rows_g<WFB_F32, true, 0>(x, nullptr, ldx, gamma, gdt, eps, m, h, q, k_pad, ldq, a_scale, s);
    if (dt == WFB_BF16)
      return launch_rows_g<WFB_BF16, true, 0>(x, nullptr, ldx, gamma, gdt, eps, m, h, q, k_pad, ldq, a_scale, s);
    return launch_rows_g<WFB_F16, true, 0>(x, nullptr, ldx, gamma, gdt, eps, m, h, q, k_pad, ldq, a_scale, s);
  }
  if (dt == WFB_F32)
    return launch_rows_g<WFB_F32, false, 0>(x, nullptr, ldx, nullptr, 0, 0.f, m, h, q, k_pad, ldq, a_scale, s);
  if (dt == WFB_BF16)
    return launch_rows_g<WFB_BF16, false, 0>(x, nullptr, ldx, nullptr, 0, 0.f, m, h, q, k_pad, ldq, a_scale, s);
  return launch_rows_g<WFB_F16, false, 0>(x, nullptr, ldx, nullptr, 0, 0.f, m, h, q, k_pad, ldq, a_scale, s);
}

hipError_t launch_quant_tensor(const void* x, int dt, int64_t numel, int8_t* q, float* a_scale, hipStream_t s) {
  if (dt == WFB_F32) return launch_tensor_t<WFB_F32>(x, numel, q, a_scale, s);
  if (dt == WFB_BF16) return launch_tensor_t<WFB_BF16>(x, numel, q, a_scale, s);
  return launch_tensor_t<WFB_F16>(x, numel, q, a_scale, s);
}

}  // namespace wfb
