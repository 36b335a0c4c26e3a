// Diagnostic: the rate of back-to-back int8 MFMA on this device, the practical ceiling next to the
// nominal dense int8 peak.  Not part of the BitLinear path; no counterpart in the reference.
//
// Each wave keeps 8 independent 32x32 int32 accumulators and issues v_mfma_i32_32x32x32_i8 on them in
// turn.  With random_operands = 0 every MFMA reads the same constant operands; with 1 the 8 chains
// read distinct pseudo-random int8 values (the A operand also rotates between chains each
// iteration), as the operands of a GEMM do.  On MI355X the difference is large: input toggling raises
// MFMA power, and the clock drops under it.
#include "wfb_common.h"

namespace wfb {

namespace {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

constexpr int kDiagChains = 8;

template <bool RANDOM>
__global__ __launch_bounds__(256) void mfma_rate_kernel(int64_t iters, int* __restrict__ sink) {
  v4i a[kDiagChains], b[kDiagChains];
  const uint32_t t = threadIdx.x + 977u * blockIdx.x;
#pragma unroll
  for (int c = 0; c < kDiagChains; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[c][e] = RANDOM ? (int)mix32(t * 131u + c * 17u + e) : 0x01020304;
      b[c][e] = RANDOM ? (int)mix32(t * 7919u + c * 3u + e + 99991u) : 0x01000100;
    }
  v16i acc[kDiagChains];
#pragma unroll
  for (int c = 0; c < kDiagChains; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0;
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kDiagChains; ++c)
      acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[c], a[(c + it) % kDiagChains], acc[c], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int c = 0; c < kDiagChains; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

hipError_t launch_mfma_rate(bool random_operands, int64_t blocks, int64_t iters, int* sink, hipStream_t s) {
  if (random_operands)
    hipLaunchKernelGGL((mfma_rate_kernel<true>), dim3((unsigned)blocks), dim3(256), 0, s, iters, sink);
  else
    hipLaunchKernelGGL((mfma_rate_kernel<false>), dim3((unsigned)blocks), dim3(256), 0, s, iters, sink);
  return hipGetLastError();
}

}  // namespace wfb
