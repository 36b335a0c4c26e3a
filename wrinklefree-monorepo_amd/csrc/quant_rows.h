// Row quantisation kernels (shared by quant.hip and quant_glu.hip): per-token absmax int8 (optionally fused behind RMSNorm/SubLN)
// and the per-tensor variant of the reference torch op.
//
// Quantiser semantics follow quantize_activations_i8
// (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:880-1135, vector path): mx = max|x|, mx < 1e-6 -> 1,
// scale = mx / 127, inv = 127 / mx, q = saturate_i8(round_half_even(x * inv)).
// The norm follows SubLN/RMSNorm (packages/training/src/wrinklefree/models/subln.py:42-59, 64-97):
// y = x * (1 / sqrt(mean(x^2) + eps)) * gamma, computed here in fp32.  The gated variants form
// x = act(gate) * up on the fly (the BitNet MLP middle: bitnet_mlp_fused,
// SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:200-216).
#pragma once

#include "wfb_common.h"

namespace wfb {
namespace {

constexpr int kTPB = 256;      // threads per row
constexpr int kVec = 8;        // elements per thread per iteration
constexpr int kMaxIt = WFB_NORM_MAX_H / (kTPB * kVec);

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor_lanes_f32<32>(v));
  v = fmaxf(v, xor_lanes_f32<16>(v));
  v = fmaxf(v, xor_lanes_f32<8>(v));
  v = fmaxf(v, xor_lanes_f32<4>(v));
  v = fmaxf(v, xor_lanes_f32<2>(v));
  return fmaxf(v, xor_lanes_f32<1>(v));
}

// Sum in a fixed xor-butterfly order (partners 32, 16, 8, 4, 2, 1); every lane ends with the same value.
__device__ __forceinline__ float wave_sum_fixed(float v) {
  v = __fadd_rn(v, xor_lanes_f32<32>(v));
  v = __fadd_rn(v, xor_lanes_f32<16>(v));
  v = __fadd_rn(v, xor_lanes_f32<8>(v));
  v = __fadd_rn(v, xor_lanes_f32<4>(v));
  v = __fadd_rn(v, xor_lanes_f32<2>(v));
  return __fadd_rn(v, xor_lanes_f32<1>(v));
}

// 8 consecutive row elements from element e0 (h = row length): x itself (GLU = 0) or the gated
// product of x (gate) and u (up).
template <int DT, int GLU>
__device__ __forceinline__ void load_row8(const void* xr, const void* ur, int e0, int h, bool vec, float (&v)[kVec]) {
  if (vec && e0 + kVec <= h) {
    load8<DT>(xr, e0, v);
    if constexpr (GLU != 0) {
      float u[kVec];
      load8<DT>(ur, e0, u);
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[e] = glu<GLU>(v[e], u[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < kVec; ++e) {
      if (e0 + e < h) {
        v[e] = load_elem<DT>(xr, e0 + e);
        if constexpr (GLU != 0) v[e] = glu<GLU>(v[e], load_elem<DT>(ur, e0 + e));
      } else {
        v[e] = 0.0f;
      }
    }
  }
}

// Whole-vector rows (16-byte aligned, h % kVec == 0): 8 elements through a buffer descriptor bounded at
// the row end, so vectors past it read as zeros without a branch.  With no element-wise alternative in
// the same code path, every load of a thread is issued before the first one is waited for.
template <int DT>
__device__ __forceinline__ void load8_buf(buf_t b, int e0, float (&v)[kVec]) {
  if constexpr (DT == WFB_F32) {
    const v4i a = buf_load16(b, (uint32_t)e0 * 4), c = buf_load16(b, (uint32_t)e0 * 4 + 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __int_as_float(a[e]);
      v[4 + e] = __int_as_float(c[e]);
    }
  } else {
    const v4i a = buf_load16(b, (uint32_t)e0 * 2);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = (uint32_t)a[e];
      if constexpr (DT == WFB_BF16) {
        v[2 * e] = __uint_as_float(w << 16);
        v[2 * e + 1] = __uint_as_float(w & 0xffff0000u);
      } else {
        v[2 * e] = f16_bits_to_f32((uint16_t)(w & 0xffffu));
        v[2 * e + 1] = f16_bits_to_f32((uint16_t)(w >> 16));
      }
    }
  }
}

// 8 elements from the raw 16-byte words of load8_buf (fp32: two words, 16-bit types: one)
template <int DT>
__device__ __forceinline__ void widen_raw8(const v4i (&a)[DT == WFB_F32 ? 2 : 1], float (&v)[kVec]) {
  if constexpr (DT == WFB_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __int_as_float(a[0][e]);
      v[4 + e] = __int_as_float(a[1][e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = (uint32_t)a[0][e];
      if constexpr (DT == WFB_BF16) {
        v[2 * e] = __uint_as_float(w << 16);
        v[2 * e + 1] = __uint_as_float(w & 0xffff0000u);
      } else {
        v[2 * e] = f16_bits_to_f32((uint16_t)(w & 0xffffu));
        v[2 * e + 1] = f16_bits_to_f32((uint16_t)(w >> 16));
      }
    }
  }
}

template <int DT, int GLU>
__device__ __forceinline__ void load_row8_full(buf_t xb, buf_t ub, int e0, float (&v)[kVec]) {
  load8_buf<DT>(xb, e0, v);
  if constexpr (GLU != 0) {
    float u[kVec];
    load8_buf<DT>(ub, e0, u);
#pragma unroll
    for (int e = 0; e < kVec; ++e) v[e] = glu<GLU>(v[e], u[e]);
  }
}

template <int DT>
__device__ __forceinline__ buf_t row_buf(const void* r, int h) {
  return make_buf(r, (uint32_t)h * (DT == WFB_F32 ? 4u : 2u));
}

template <int DT, int GDT, bool NORM, int GLU>
__global__ __launch_bounds__(kTPB) void quant_rows_kernel(const void* __restrict__ x, const void* __restrict__ up,
                                                          int64_t ldx, const void* __restrict__ gamma, float eps,
                                                          int h, int8_t* __restrict__ q, int64_t k_pad,
                                                          int64_t ldq, float* __restrict__ a_scale,
                                                          bool vec) {
  __shared__ float red[kTPB / 64];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  const int64_t roff = row * ldx * (DT == WFB_F32 ? 4 : 2);
  const void* xr = reinterpret_cast<const char*>(x) + roff;
  const void* ur = GLU != 0 ? reinterpret_cast<const char*>(up) + roff : nullptr;

  float v[kMaxIt][kVec];
  const bool full = vec && h % kVec == 0;  // uniform
  // (whole-vector rows with gamma) gamma's 8 elements per iteration as raw 16-byte words, requested right
  // after the row's: issued after the reduction inside the per-iteration loop below, each load was
  // followed by a wait of its own, one cache round trip per iteration
  constexpr int GW = GDT == WFB_F32 ? 2 : 1;
  v4i graw[NORM ? kMaxIt : 1][GW];
  const bool gpre = NORM && full && gamma != nullptr;  // uniform
  if (full) {
    const buf_t xb = row_buf<DT>(xr, h), ub = GLU != 0 ? row_buf<DT>(ur, h) : xb;
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
      if (it * kTPB * kVec >= h) {  // uniform over the block
#pragma unroll
        for (int e = 0; e < kVec; ++e) v[it][e] = 0.0f;
      } else {
        load_row8_full<DT, GLU>(xb, ub, (it * kTPB + t) * kVec, v[it]);
      }
    }
    if constexpr (NORM) {
      if (gpre) {
        // every iteration's words, without branches (vectors past the row read zeros through the range)
        const buf_t gb = row_buf<GDT>(gamma, h);
#pragma unroll
        for (int it = 0; it < kMaxIt; ++it)
#pragma unroll
          for (int q = 0; q < GW; ++q)
            graw[it][q] = buf_load16(gb, (uint32_t)((it * kTPB + t) * kVec) * (GDT == WFB_F32 ? 4u : 2u) + 16u * q);
      }
    }
  } else {
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
      const int e0 = (it * kTPB + t) * kVec;
      if (it * kTPB * kVec >= h) {  // uniform over the block
#pragma unroll
        for (int e = 0; e < kVec; ++e) v[it][e] = 0.0f;
      } else {
        load_row8<DT, GLU>(xr, ur, e0, h, vec, v[it]);
      }
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
      } else if (gpre) {
        widen_raw8<GDT>(graw[it], g);
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
      const uint32_t lo = quant4_i8(&v[it][0], inv), hi = quant4_i8(&v[it][4], inv);
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

template <int DT, int GDT, bool NORM, int VPL, int GLU>
__global__ __launch_bounds__(256) void quant_rows_wave_kernel(const void* __restrict__ x, const void* __restrict__ up,
                                                              int64_t ldx, const void* __restrict__ gamma, float eps,
                                                              int h, int m, int8_t* __restrict__ q, int64_t k_pad,
                                                              int64_t ldq, float* __restrict__ a_scale, bool vec) {
  const int lane = threadIdx.x & 63;
  // wave-uniform row (readfirstlane), so the row's buffer descriptor lives in scalar registers
  const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= m) return;
  const int64_t roff = row * ldx * (DT == WFB_F32 ? 4 : 2);
  const void* xr = reinterpret_cast<const char*>(x) + roff;
  const void* ur = GLU != 0 ? reinterpret_cast<const char*>(up) + roff : nullptr;

  float v[VPL][kVec];
  const bool full = vec && h % kVec == 0;  // uniform
  if (full) {
    const buf_t xb = row_buf<DT>(xr, h), ub = GLU != 0 ? row_buf<DT>(ur, h) : xb;
#pragma unroll
    for (int j = 0; j < VPL; ++j) load_row8_full<DT, GLU>(xb, ub, (lane + 64 * j) * kVec, v[j]);
  } else {
#pragma unroll
    for (int j = 0; j < VPL; ++j) load_row8<DT, GLU>(xr, ur, (lane + 64 * j) * kVec, h, vec, v[j]);
  }
  if constexpr (NORM) {
    float g[VPL][kVec];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e0 = (lane + 64 * j) * kVec;
      if (gamma == nullptr) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[j][e] = 1.0f;
      } else if (full) {
        load8_buf<GDT>(row_buf<GDT>(gamma, h), e0, g[j]);
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
      const uint32_t lo = quant4_i8(&v[j][0], inv), hi = quant4_i8(&v[j][4], inv);
      *reinterpret_cast<uint2*>(qr + e0) = make_uint2(lo, hi);
    } else if (e0 < h) {
#pragma unroll
      for (int e = 0; e < kVec; ++e)
        if (e0 + e < h) qr[e0 + e] = (int8_t)quant_i8(v[j][e], inv);
    }
  }
  for (int64_t e = h + lane; e < k_pad; e += 64) qr[e] = 0;
}

// Few rows (M <= kWideMaxM): one 1024-thread workgroup per row, so the per-element work (loads, gated
// activation, scaling, quantisation, stores) is spread over 16 waves instead of one (at M = 8 a wave per
// row leaves the GPU nearly idle and every wave instruction-latency-bound).  The element values go
// through LDS so that the sum of squares is still taken in exactly the documented order of the kernel
// the row length selects (the wave order for H <= kWaveMaxH, the 256-thread block order above it):
// results are bit-identical to quant_rows_wave_kernel / quant_rows_kernel, whatever the batch size.
constexpr int kWideThreads = 1024;
constexpr int kWideMaxM = 64;

template <int DT, int GDT, bool NORM, int GLU>
__global__ __launch_bounds__(kWideThreads) void quant_rows_wide_kernel(
    const void* __restrict__ x, const void* __restrict__ up, int64_t ldx, const void* __restrict__ gamma, float eps,
    int h, int8_t* __restrict__ q, int64_t k_pad, int64_t ldq, float* __restrict__ a_scale, bool vec) {
  extern __shared__ float xs[];  // the row, fp32 (after the gated activation)
  __shared__ float red[kWideThreads / 64];
  __shared__ float bcast;
  constexpr int VPT = 2;  // 8-element vectors per thread (h <= 16384)
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t row = blockIdx.x;
  const int64_t roff = row * ldx * (DT == WFB_F32 ? 4 : 2);
  const void* xr = reinterpret_cast<const char*>(x) + roff;
  const void* ur = GLU != 0 ? reinterpret_cast<const char*>(up) + roff : nullptr;
  const int nvec = (h + kVec - 1) / kVec;

  float v[VPT][kVec];
  const bool full = vec && h % kVec == 0;  // uniform
  // (whole-vector rows with gamma) gamma's words requested with the row's, as in quant_rows_kernel
  constexpr int GW = GDT == WFB_F32 ? 2 : 1;
  v4i graw[NORM ? VPT : 1][GW];
  const bool gpre = NORM && full && gamma != nullptr;  // uniform
  if (full) {  // every load in flight before the first wait (vectors past the row read as zeros)
    const buf_t xb = row_buf<DT>(xr, h), ub = GLU != 0 ? row_buf<DT>(ur, h) : xb;
#pragma unroll
    for (int i = 0; i < VPT; ++i) load_row8_full<DT, GLU>(xb, ub, (t + kWideThreads * i) * kVec, v[i]);
    if constexpr (NORM) {
      if (gpre) {
        const buf_t gb = row_buf<GDT>(gamma, h);
#pragma unroll
        for (int i = 0; i < VPT; ++i)
#pragma unroll
          for (int q = 0; q < GW; ++q)
            graw[i][q] = buf_load16(gb, (uint32_t)((t + kWideThreads * i) * kVec) * (GDT == WFB_F32 ? 4u : 2u) + 16u * q);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int vi = t + kWideThreads * i;
    if (vi < nvec) {
      if (!full) load_row8<DT, GLU>(xr, ur, vi * kVec, h, vec, v[i]);
      if constexpr (NORM) {
        if (vi * kVec + kVec <= h) {
          float4* d = reinterpret_cast<float4*>(xs + vi * kVec);
          d[0] = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
          d[1] = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
        } else {
#pragma unroll
          for (int e = 0; e < kVec; ++e)
            if (vi * kVec + e < h) xs[vi * kVec + e] = v[i][e];
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[i][e] = 0.0f;
    }
  }

  if constexpr (NORM) {
    __syncthreads();
    // adds the squares of elements base .. base+7 to ss in order (elements past h count as 0)
    auto add8 = [&](float ss, int base) {
      float a[kVec];
      if (base + kVec <= h) {
        const float4* p = reinterpret_cast<const float4*>(xs + base);
        const float4 lo = p[0], hi = p[1];
        a[0] = lo.x; a[1] = lo.y; a[2] = lo.z; a[3] = lo.w; a[4] = hi.x; a[5] = hi.y; a[6] = hi.z; a[7] = hi.w;
      } else {
#pragma unroll
        for (int e = 0; e < kVec; ++e) a[e] = base + e < h ? xs[base + e] : 0.0f;
      }
#pragma unroll
      for (int e = 0; e < kVec; ++e) ss = __fadd_rn(ss, __fmul_rn(a[e], a[e]));
      return ss;
    };
    if (h <= kWaveMaxH) {  // wave order: lane l adds elements (l + 64j)*8 + e, j ascending, e = 0..7
      if (w == 0) {
        float ss = 0.0f;
        for (int j = 0; j * 64 * kVec < h; ++j) ss = add8(ss, (lane + 64 * j) * kVec);
        ss = wave_sum_fixed(ss);
        if (lane == 0) bcast = ss;
      }
    } else {  // block order: thread t < 256 adds elements (it*256 + t)*8 + e, then waves 0..3 in order
      if (w < kTPB / 64) {
        float ss = 0.0f;
        for (int it = 0; it * kTPB * kVec < h; ++it) ss = add8(ss, (it * kTPB + t) * kVec);
        ss = wave_sum_fixed(ss);
        if (lane == 0) red[w] = ss;
      }
      __syncthreads();
      if (t == 0) {
        float tot = red[0];
#pragma unroll
        for (int k = 1; k < kTPB / 64; ++k) tot = __fadd_rn(tot, red[k]);
        bcast = tot;
      }
    }
    __syncthreads();
    const float r = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(bcast, (float)h), eps)));
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int vi = t + kWideThreads * i;
      if (vi >= nvec) continue;
      const int e0 = vi * kVec;
      float g[kVec];
      if (gamma == nullptr) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[e] = 1.0f;
      } else if (gpre) {
        widen_raw8<GDT>(graw[i], g);
      } else if (vec && e0 + kVec <= h) {
        load8<GDT>(gamma, e0, g);
      } else {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[e] = (e0 + e < h) ? load_elem<GDT>(gamma, e0 + e) : 1.0f;
      }
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[i][e] = __fmul_rn(__fmul_rn(v[i][e], r), g[e]);
    }
  }

  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < VPT; ++i)
#pragma unroll
    for (int e = 0; e < kVec; ++e)
      if ((t + kWideThreads * i) * kVec + e < h) mx = fmaxf(mx, fabsf(v[i][e]));
  mx = wave_max(mx);
  if (lane == 0) red[w] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int k = 1; k < kWideThreads / 64; ++k) mx = fmaxf(mx, red[k]);
  if (mx < 1e-6f) mx = 1.0f;
  const float inv = __fdiv_rn(127.0f, mx);
  if (t == 0) a_scale[row] = __fdiv_rn(mx, 127.0f);

  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e0 = (t + kWideThreads * i) * kVec;
    if (e0 >= h) break;
    if (e0 + kVec <= h) {
      const uint32_t lo = quant4_i8(&v[i][0], inv), hi = quant4_i8(&v[i][4], inv);
      *reinterpret_cast<uint2*>(qr + e0) = make_uint2(lo, hi);
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e)
        if (e0 + e < h) qr[e0 + e] = (int8_t)quant_i8(v[i][e], inv);
    }
  }
  for (int64_t e = h + t; e < k_pad; e += kWideThreads) qr[e] = 0;
}

template <int DT, int GDT, bool NORM, int VPL, int GLU>
void launch_wave(const void* x, const void* up, int64_t ldx, const void* gamma, float eps, int64_t m, int64_t h,
                 int8_t* q, int64_t k_pad, int64_t ldq, float* a_scale, bool vec, hipStream_t s) {
  hipLaunchKernelGGL((quant_rows_wave_kernel<DT, GDT, NORM, VPL, GLU>), dim3((unsigned)((m + 3) / 4)), dim3(256), 0, s,
                     x, up, ldx, gamma, eps, (int)h, (int)m, q, k_pad, ldq, a_scale, vec);
}

template <int DT, int GDT, bool NORM, int GLU>
hipError_t launch_rows_t(const void* x, const void* up, int64_t ldx, const void* gamma, float eps, int64_t m,
                         int64_t h, int8_t* q, int64_t k_pad, int64_t ldq, float* a_scale, hipStream_t s) {
  const int esz = DT == WFB_F32 ? 4 : 2;
  const int gsz = GDT == WFB_F32 ? 4 : 2;
  const bool vec = ((uintptr_t)x % 16 == 0) && (GLU == 0 || (uintptr_t)up % 16 == 0) && ((ldx * esz) % 16 == 0) &&
                   (gamma == nullptr || (uintptr_t)gamma % (8 * gsz > 16 ? 16 : 8 * gsz) == 0);
  const int vpl = (int)((h + 64 * kVec - 1) / (64 * kVec));
#define WFB_WAVE(V) launch_wave<DT, GDT, NORM, V, GLU>(x, up, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, vec, s)
  // wide kernel where a wave per row has the most serial work: rows of the wave order with 5-8 vectors
  // per lane (H > 2048) and gated rows (measured on MI355X; above kWaveMaxH the 256-thread block kernel
  // stays faster for plain rows, 5.2 vs 5.9 us at H = 6912, M = 8, while the gated ones gain from 16
  // waves, 9.5 vs 9.8 us at H = 14336; the row is staged in LDS as fp32, kept under 64 KB)
  const bool wide = m <= kWideMaxM && ((h <= kWaveMaxH && (h > 2048 || (GLU != 0 && (m > 1 || h > 1024)))) ||
                                       (GLU != 0 && h > kWaveMaxH && h <= 15360));
  if (wide) {
    const size_t lds = NORM ? (size_t)h * sizeof(float) : 0;
    hipLaunchKernelGGL((quant_rows_wide_kernel<DT, GDT, NORM, GLU>), dim3((unsigned)m), dim3(kWideThreads), lds, s, x,
                       up, ldx, gamma, eps, (int)h, q, k_pad, ldq, a_scale, vec);
  } else if (h <= kWaveMaxH) {
    switch (vpl) {
      case 1: WFB_WAVE(1); break;
      case 2: WFB_WAVE(2); break;
      case 3: WFB_WAVE(3); break;
      case 4: WFB_WAVE(4); break;
      case 5: WFB_WAVE(5); break;
      case 6: WFB_WAVE(6); break;
      case 7: case 8: WFB_WAVE(8); break;
      case 9: case 10: case 11: case 12: WFB_WAVE(12); break;
      default: WFB_WAVE(16); break;
    }
  } else {
    hipLaunchKernelGGL((quant_rows_kernel<DT, GDT, NORM, GLU>), dim3((unsigned)m), dim3(kTPB), 0, s, x, up, ldx, gamma,
                       eps, (int)h, q, k_pad, ldq, a_scale, vec);
  }
#undef WFB_WAVE
  return hipGetLastError();
}

template <int DT, bool NORM, int GLU>
hipError_t launch_rows_g(const void* x, const void* up, int64_t ldx, const void* gamma, int gdt, float eps, int64_t m,
                         int64_t h, int8_t* q, int64_t k_pad, int64_t ldq, float* a_scale, hipStream_t s) {
  if (!NORM || gamma == nullptr || gdt == WFB_F32)
    return launch_rows_t<DT, WFB_F32, NORM, GLU>(x, up, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, s);
  if (gdt == WFB_BF16)
    return launch_rows_t<DT, WFB_BF16, NORM, GLU>(x, up, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, s);
  return launch_rows_t<DT, WFB_F16, NORM, GLU>(x, up, ldx, gamma, eps, m, h, q, k_pad, ldq, a_scale, s);
}

}  // namespace
}  // namespace wfb
