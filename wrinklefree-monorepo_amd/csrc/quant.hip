// Activation quantisation kernels: per-token absmax int8 (optionally fused behind RMSNorm/SubLN)
// and the per-tensor variant of the reference torch op.
//
// Quantiser semantics follow quantize_activations_i8
// (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:880-1135, vector path): mx = max|x|, mx < 1e-6 -> 1,
// scale = mx / 127, inv = 127 / mx, q = saturate_i8(round_half_even(x * inv)).
// The norm follows SubLN/RMSNorm (packages/training/src/wrinklefree/models/subln.py:42-59, 64-97):
// y = x * (1 / sqrt(mean(x^2) + eps)) * gamma, computed here in fp32.
#include "wfb_common.h"

namespace wfb {

namespace {

constexpr int kTPB = 256;      // threads per row
constexpr int kVec = 8;        // elements per thread per iteration
constexpr int kMaxIt = WFB_NORM_MAX_H / (kTPB * kVec);

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum in a fixed xor-butterfly order; every lane ends with the same value.
__device__ __forceinline__ float wave_sum_fixed(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, 64));
  return v;
}

template <int DT, int GDT, bool NORM>
__global__ __launch_bounds__(kTPB) void quant_rows_kernel(const void* __restrict__ x, int64_t ldx,
                                                          const void* __restrict__ gamma, float eps,
                                                          int h, int8_t* __restrict__ q, int64_t k_pad,
                                                          int64_t ldq, float* __restrict__ a_scale,
                                                          bool vec) {
  __shared__ float red[kTPB / 64];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  const void* xr = reinterpret_cast<const char*>(x) + row * ldx * (DT == WFB_F32 ? 4 : 2);

  float v[kMaxIt][kVec];
#pragma unroll
  for (int it = 0; it < kMaxIt; ++it) {
    const int e0 = (it * kTPB + t) * kVec;
    if (it * kTPB * kVec >= h) {  // uniform over the block
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[it][e] = 0.0f;
    } else if (vec && e0 + kVec <= h) {
      load8<DT>(xr, e0, v[it]);
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[it][e] = (e0 + e < h) ? load_elem<DT>(xr, e0 + e) : 0.0f;
    }
  }

  if constexpr (NORM) {
    // Sum of squares: thread-sequential over (it, e), then the fixed butterfly, then waves in order.
    float ss = 0.0f;
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it)
#pragma unroll
      for (int e = 0; e < kVec; ++e) ss = __fadd_rn(ss, __fmul_rn(v[it][e], v[it][e]));
    ss = wave_sum_fixed(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = red[0];
#pragma unroll
    for (int w = 1; w < kTPB / 64; ++w) tot = __fadd_rn(tot, red[w]);
    __syncthreads();
    const float r = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, (float)h), eps)));
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
      if (it * kTPB * kVec >= h) break;  // uniform over the block
      const int e0 = (it * kTPB + t) * kVec;
      float g[kVec];
      if (gamma == nullptr) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[e] = 1.0f;
      } else if (vec && e0 + kVec <= h) {
        load8<GDT>(gamma, e0, g);
      } else {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[e] = (e0 + e < h) ? load_elem<GDT>(gamma, e0 + e) : 1.0f;
      }
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[it][e] = __fmul_rn(__fmul_rn(v[it][e], r), g[e]);
    }
  }

  float mx = 0.0f;
#pragma unroll
  for (int it = 0; it < kMaxIt; ++it)
#pragma unroll
    for (int e = 0; e < kVec; ++e) mx = fmaxf(mx, fabsf(v[it][e]));
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < kTPB / 64; ++w) mx = fmaxf(mx, red[w]);
  if (mx < 1e-6f) mx = 1.0f;
  const float inv = __fdiv_rn(127.0f, mx);
  if (t == 0) a_scale[row] = __fdiv_rn(mx, 127.0f);

  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int it = 0; it < kMaxIt; ++it) {
    const int e0 = (it * kTPB + t) * kVec;
    if (e0 >= h) break;
    if (e0 + kVec <= h) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) lo |= (uint32_t)(quant_i8(v[it][e], inv) & 0xff) << (8 * e);
#pragma unroll
      for (int e = 0; e < 4; ++e) hi |= (uint32_t)(quant_i8(v[it][4 + e], inv) & 0xff) << (8 * e);
      *reinterpret_cast<uint2*>(qr + e0) = make_uint2(lo, hi);
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e)
        if (e0 + e < h) qr[e0 + e] = (int8_t)quant_i8(v[it][e], inv);
    }
  }
  for (int64_t e = h + t; e < k_pad; e += kTPB) qr[e] = 0;
}

// One wave per row for H <= kWaveMaxH (4 rows per 256-thread workgroup, no barriers): lane l holds
// the 8-element vectors v = l + 64*j (j < VPL).  Sum of squares: lane-sequential over (j, e), then
// the fixed xor butterfly.  Used for every row length up to kWaveMaxH.
constexpr int kWaveMaxH = 4096;

template <int DT, int GDT, bool NORM, int VPL>
__global__ __launch_bounds__(256) void quant_rows_wave_kernel(const void* __restrict__ x, int64_t ldx,
                                                              const void* __restrict__ gamma, float eps, int h,
                                                              int m, int8_t* __restrict__ q, int64_t k_pad,
                                                              int64_t ldq, float* __restrict__ a_scale, bool vec) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m) return;
  const void* xr = reinterpret_cast<const char*>(x) + row * ldx * (DT == WFB_F32 ? 4 : 2);

  float v[VPL][kVec];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e0 = (lane + 64 * j) * kVec;
    if (vec && e0 + kVec <= h) {
      load8<DT>(xr, e0, v[j]);
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[j][e] = (e0 + e < h) ? load_elem<DT>(xr, e0 + e) : 0.0f;
    }
  }
  if constexpr (NORM) {
    float g[VPL][kVec];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e0 = (lane + 64 * j) * kVec;
      if (gamma == nullptr) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[j][e] = 1.0f;
      } else if (vec && e0 + kVec <= h) {
        load8<GDT>(gamma, e0, g[j]);
      } else {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[j][e] = (e0 + e < h) ? load_elem<GDT>(gamma, e0 + e) : 1.0f;
      }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < kVec; ++e) ss = __fadd_rn(ss, __fmul_rn(v[j][e], v[j][e]));
    ss = wave_sum_fixed(ss);
    const float r = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(ss, (float)h), eps)));
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[j][e] = __fmul_rn(__fmul_rn(v[j][e], r), g[j][e]);
  }
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int e = 0; e < kVec; ++e) mx = fmaxf(mx, fabsf(v[j][e]));
  mx = wave_max(mx);
  if (mx < 1e-6f) mx = 1.0f;
  const float inv = __fdiv_rn(127.0f, mx);
  if (lane == 0) a_scale[row] = __fdiv_rn(mx, 127.0f);
  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e0 = (lane + 64 * j) * kVec;
    if (e0 + kVec <= h) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) lo |= (uint32_t)(quant_i8(v[j][e], inv) & 0xff) << (8 * e);
#pragma unroll
      for (int e = 0; e < 4; ++e) hi |= (uint32_t)(quant_i8(v[j][4 + e], inv) & 0xff) << (8 * e);
      *reinterpret_cast<uint2*>(qr + e0) = make_uint2(lo, hi);
    } else if (e0 < h) {
#pragma unroll
      for (int e = 0; e < kVec; ++e)
        if (e0 + e < h) qr[e0 + e] = (int8_t)quant_i8(v[j][e], inv);
    }
  }
  for (int64_t e = h + lane; e < k_pad; e += 64) qr[e] = 0;
}

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

template <int DT, int GDT, bool NORM, int VPL>
void launch_wave(const void* x, int64_t ldx, const void* gamma, float eps, int64_t m, int64_t h, int8_t* q,
                 int64_t k_pad, int64_t ldq, float* a_scale, bool vec, hipStream_t s) {
  hipLaunchKernelGGL((quant_rows_wave_kernel<DT, GDT, NORM, VPL>), dim3((unsigned)((m + 3) / 4)), dim3(256), 0, s, x,
                     ldx, gamma, eps, (int)h, (int)m, q, k_pad, ldq, a_scale, vec);
}

template <int DT, int GDT, bool NORM>
hipError_t launch_rows_t(const void* x, int64_t ldx, const void* gamma, float eps, int64_t m, int64_t h,
                         int8_t* q, int64_t k_pad, int64_t ldq, float* a_scale, hipStream_t s) {
  const int esz = DT == WFB_F32 ? 4 : 2;
  const int gsz = GDT == WFB_F32 ? 4 : 2;
  const bool vec = ((uintptr_t)x % 16 == 0) && ((ldx * esz) % 16 == 0) &&
                   (gamma == nullptr || (uintptr_t)gamma % (8 * gsz > 16 ? 16 : 8 * gsz) == 0);
  const int vpl = (int)((h + 64 * kVec - 1) / (64 * kVec));
  if (h <= kWaveMaxH) {
    switch (vpl) {
      case 1: launch_wave<DT, GDT, NORM, 1>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
      case 2: launch_wave<DT, GDT, NORM, 2>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
      case 3: launch_wave<DT, GDT, NORM, 3>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
      case 4: launch_wave<DT, GDT, NORM, 4>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
      case 5: launch_wave<DT, GDT, NORM, 5>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
      case 6: launch_wave<DT, GDT, NORM, 6>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
      case 7: case 8: launch_wave<DT, GDT, NORM, 8>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
      case 9: case 10: case 11: case 12:
        launch_wave<DT, GDT, NORM, 12>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
      default: launch_wave<DT, GDT, NORM, 16>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s); break;
    }
  } else {
    hipLaunchKernelGGL((quant_rows_kernel<DT, GDT, NORM>), dim3((unsigned)m), dim3(kTPB), 0, s, x, ldx, gamma,
                       eps, (int)h, q, k_pad, ldq, a_scale, vec);
  }
  return hipGetLastError();
}

template <int DT, bool NORM>
hipError_t launch_rows_g(const void* x, int64_t ldx, const void* gamma, int gdt, float eps, int64_t m,
                         int64_t h, int8_t* q, int64_t k_pad, int64_t ldq, float* a_scale, hipStream_t s) {
  if (!NORM || gamma == nullptr || gdt == WFB_F32)
    return launch_rows_t<DT, WFB_F32, NORM>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, s);
  if (gdt == WFB_BF16)
    return launch_rows_t<DT, WFB_BF16, NORM>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, s);
  return launch_rows_t<DT, WFB_F16, NORM>(x, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, s);
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
    if (dt == WFB_F32) return launch_rows_g<WFB_F32, true>(x, ldx, gamma, gdt, eps, m, h, q, k_pad, ldq, a_scale, s);
    if (dt == WFB_BF16) return launch_rows_g<WFB_BF16, true>(x, ldx, gamma, gdt, eps, m, h, q, k_pad, ldq, a_scale, s);
    return launch_rows_g<WFB_F16, true>(x, ldx, gamma, gdt, eps, m, h, q, k_pad, ldq, a_scale, s);
  }
  if (dt == WFB_F32) return launch_rows_g<WFB_F32, false>(x, ldx, nullptr, 0, 0.f, m, h, q, k_pad, ldq, a_scale, s);
  if (dt == WFB_BF16) return launch_rows_g<WFB_BF16, false>(x, ldx, nullptr, 0, 0.f, m, h, q, k_pad, ldq, a_scale, s);
  return launch_rows_g<WFB_F16, false>(x, ldx, nullptr, 0, 0.f, m, h, q, k_pad, ldq, a_scale, s);
}

hipError_t launch_quant_tensor(const void* x, int dt, int64_t numel, int8_t* q, float* a_scale, hipStream_t s) {
  if (dt == WFB_F32) return launch_tensor_t<WFB_F32>(x, numel, q, a_scale, s);
  if (dt == WFB_BF16) return launch_tensor_t<WFB_BF16>(x, numel, q, a_scale, s);
  return launch_tensor_t<WFB_F16>(x, numel, q, a_scale, s);
}

}  // namespace wfb
