// Offline weight pack on the device: per-tensor absmean scale and the I2_S 2-bit layout.
//
// Follows pack_ternary_sglkernel (packages/inference/scripts/convert_to_sglkernel.py:51-123):
//   s = mean(|W|) (s < 1e-8 -> 1.0), q = clamp(round_half_even(W / s), -1, 1), code = q + 1,
//   byte j of 128-weight block b = code[128b+j]<<6 | code[128b+32+j]<<4 | code[128b+64+j]<<2 | code[128b+96+j].
#include "wfb_common.h"

namespace wfb {

namespace {

constexpr int kAbsBlocks = WFB_ABSMEAN_WS_DOUBLES;

// Stage 1: block b sums |w| over the grid-stride set {i : i % (blocks*256) in block b's range},
// in fp64, each thread sequentially, then a fixed tree.  Deterministic for a given numel.
template <int DT>
__global__ __launch_bounds__(256) void absmean_partial_kernel(const void* __restrict__ w, int64_t numel,
                                                              double* __restrict__ partial) {
  __shared__ double red[256];
  double acc = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < numel; i += (int64_t)kAbsBlocks * 256)
    acc += (double)fabsf(load_elem<DT>(w, i));
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(256) void absmean_final_kernel(const double* __restrict__ partial, int64_t numel,
                                                            float* __restrict__ scale) {
  __shared__ double red[256];
  double acc = 0.0;
  for (int i = threadIdx.x; i < kAbsBlocks; i += 256) acc += partial[i];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float s = numel > 0 ? (float)(red[0] / (double)numel) : 0.0f;
    if ((double)s < 1e-8) s = 1.0f;
    scale[0] = s;
  }
}

__device__ __forceinline__ uint32_t ternary_code(float w, float s) {
  float q = __builtin_rintf(__fdiv_rn(w, s));
  q = fminf(fmaxf(q, -1.0f), 1.0f);
  return (uint32_t)((int)q + 1);
}

// One thread per output dword: bytes j..j+3 (j = 4*(p % 8)) of block b = p / 8 of row `row`.
template <int DT>
__global__ __launch_bounds__(256) void pack_i2s_kernel(const void* __restrict__ w, int64_t n, int64_t k,
                                                       int64_t ldw, const float* __restrict__ scale,
                                                       uint32_t* __restrict__ qw) {
  const int64_t dw_per_row = k / 16;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= n * dw_per_row) return;
  const int64_t row = gid / dw_per_row;
  const int64_t p = gid % dw_per_row;
  const int64_t b = p >> 3;
  const int j = (int)(p & 7) * 4;
  const float s = scale[0];
  const int64_t base = row * ldw + 128 * b + j;
  uint32_t out = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint32_t byte = 0;
#pragma unroll
    for (int f = 0; f < 4; ++f) byte |= ternary_code(load_elem<DT>(w, base + 32 * f + t), s) << (6 - 2 * f);
    out |= byte << (8 * t);
  }
  qw[gid] = out;
}

__global__ __launch_bounds__(256) void unpack_i2s_kernel(const uint8_t* __restrict__ qw, int64_t n, int64_t k,
                                                         int8_t* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one packed byte
  const int64_t kb = k / 4;
  if (gid >= n * kb) return;
  const int64_t row = gid / kb, p = gid % kb;
  const int64_t b = p / 32;
  const int j = (int)(p % 32);
  const uint32_t byte = qw[gid];
  int8_t* o = out + row * k + 128 * b + j;
#pragma unroll
  for (int f = 0; f < 4; ++f) o[32 * f] = (int8_t)((int)((byte >> (6 - 2 * f)) & 3u) - 1);
}

template <int DT>
hipError_t absmean_t(const void* w, int64_t numel, float* scale, double* ws, hipStream_t s) {
  hipLaunchKernelGGL((absmean_partial_kernel<DT>), dim3(kAbsBlocks), dim3(256), 0, s, w, numel, ws);
  hipLaunchKernelGGL(absmean_final_kernel, dim3(1), dim3(256), 0, s, ws, numel, scale);
  return hipGetLastError();
}

template <int DT>
hipError_t pack_t(const void* w, int64_t n, int64_t k, int64_t ldw, const float* scale, uint8_t* qw,
                  hipStream_t s) {
  const int64_t total = n * (k / 16);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL((pack_i2s_kernel<DT>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, w, n, k, ldw,
                     scale, reinterpret_cast<uint32_t*>(qw));
  return hipGetLastError();
}

}  // namespace

hipError_t launch_weight_absmean(const void* w, int dt, int64_t numel, float* scale, double* ws, hipStream_t s) {
  if (dt == WFB_F32) return absmean_t<WFB_F32>(w, numel, scale, ws, s);
  if (dt == WFB_BF16) return absmean_t<WFB_BF16>(w, numel, scale, ws, s);
  return absmean_t<WFB_F16>(w, numel, scale, ws, s);
}

hipError_t launch_pack_i2s(const void* w, int dt, int64_t n, int64_t k, int64_t ldw, const float* scale,
                           uint8_t* qw, hipStream_t s) {
  if (dt == WFB_F32) return pack_t<WFB_F32>(w, n, k, ldw, scale, qw, s);
  if (dt == WFB_BF16) return pack_t<WFB_BF16>(w, n, k, ldw, scale, qw, s);
  return pack_t<WFB_F16>(w, n, k, ldw, scale, qw, s);
}

hipError_t launch_unpack_i2s(const uint8_t* qw, int64_t n, int64_t k, int8_t* out, hipStream_t s) {
  const int64_t total = n * (k / 4);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(unpack_i2s_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, qw, n, k, out);
  return hipGetLastError();
}

}  // namespace wfb
