// Greedy decoding on the device: the LM head with the next-token argmax fused in.
//
// Replaces the engine's final steps (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:539-553: final
// rms_norm, then the LM head as a packed BitLinear or an fp32 linear over the vocabulary) and its greedy
// pick (bitnet_engine.cpp:774-779, std::max_element: the first maximal logit).
//
// Every producer writes, per 16 vocabulary rows and token, the largest 64-bit key of
// (logit, row) (amax_key: orderable float bits above the inverted row index, so ties go to the smaller
// row) into a workspace of ceil(N/16) x M slots; argmax_finalize_kernel reduces the slots of each
// token and writes the row index.  No atomics, so the result does not depend on workgroup order, and
// no workspace initialisation is needed (every slot is written).
//
// lm_head_kernel is the dense head (tied bf16/fp32 embedding): each workgroup recomputes the final
// RMSNorm of the M token rows (y = x * (1/sqrt(mean(x^2) + eps)) * gamma, rounded to the x dtype as the
// torch glue does) into LDS, then streams 64 vocabulary rows: 8 lanes per row, each lane a 16-byte
// (bf16) or 32-byte (fp32) piece of the row per step against the normalised rows in LDS, fp32
// accumulation, a DPP sum over the 8 lanes; each wave covers 16 rows = one workspace slot.
#include "wfb_common.h"

namespace wfb {

namespace {

__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  if (dt == WFB_F32) return load_elem<WFB_F32>(p, i);
  if (dt == WFB_BF16) return load_elem<WFB_BF16>(p, i);
  return load_elem<WFB_F16>(p, i);
}

// One workgroup per token; each thread keeps kFinLoads independent slot loads in flight per round (a
// 128256-row head has 8016 slots: one round), then a wave and a workgroup maximum.  BUF: the loads go
// through a buffer descriptor bounded at the workspace's end (workspaces under 4 GiB), so slots past it
// read 0 without a branch -- guarded loads compiled to one wait per load.
constexpr int kFinThreads = 1024, kFinLoads = 8;
typedef uint32_t u32x2_fin __attribute__((ext_vector_type(2)));
template <bool BUF>
__global__ __launch_bounds__(kFinThreads) void argmax_finalize_kernel(const uint64_t* __restrict__ parts, int64_t np,
                                                                      int m, int64_t* __restrict__ tokens) {
  __shared__ uint64_t sb[kFinThreads / 64];
  const int mm = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint32_t pbytes = BUF ? (uint32_t)(np * m) * 8u : 0u;
  const buf_t pb = make_buf(parts, pbytes);
  uint64_t best = 0;
  for (int64_t p0 = 0; p0 < np; p0 += (int64_t)kFinThreads * kFinLoads) {
    uint64_t v[kFinLoads];
#pragma unroll
    for (int i = 0; i < kFinLoads; ++i) {
      const int64_t p = p0 + t + (int64_t)kFinThreads * i;
      if constexpr (BUF) {
        const u32x2_fin a =
            __builtin_amdgcn_raw_buffer_load_b64(pb, p < np ? (uint32_t)(p * m + mm) * 8u : pbytes, 0, 0);
        v[i] = ((uint64_t)a[1] << 32) | a[0];
      } else {
        v[i] = p < np ? parts[p * m + mm] : 0;
      }
    }
#pragma unroll
    for (int i = 0; i < kFinLoads; ++i) best = v[i] > best ? v[i] : best;
  }
  best = group_max_u64<64>(best);
  if (lane == 0) sb[w] = best;
  __syncthreads();
  if (t == 0) {
    uint64_t b = sb[0];
#pragma unroll
    for (int i = 1; i < kFinThreads / 64; ++i) b = sb[i] > b ? sb[i] : b;
    tokens[mm] = b ? (int64_t)(0xFFFFFFFFu - (uint32_t)b) : -1;
  }
}

template <int XT, int WT, int MM>
__global__ __launch_bounds__(256) void lm_head_kernel(const void* __restrict__ x, int64_t ldx,
                                                      const void* __restrict__ gamma, int gdt, float eps,
                                                      const void* __restrict__ W, int64_t ldw, int m, int n, int h,
                                                      float* __restrict__ logits, int64_t ldo,
                                                      uint64_t* __restrict__ parts) {
  extern __shared__ float xn[];  // [m][h]
  __shared__ float rs[16];
  __shared__ float red[4][MM];
  constexpr int ESZ = WT == WFB_F32 ? 4 : 2;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);

  // The final norm of the m rows: 8-element chunks of the rows spread over all 256 threads, each batch's
  // loads issued before any is used (a load-then-add loop waits one cache round trip per element).
  // Pass 1: each row's sum of squares (per-thread partials per row, then the wave and the 4 waves).
  const int C8 = h >> 3, nch = m * C8;
  float ssr[MM];
#pragma unroll
  for (int mm = 0; mm < MM; ++mm) ssr[mm] = 0.0f;
  for (int j0 = 0; j0 * 256 < nch; j0 += 2) {
    float v[2][8];
    int mrow[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = (j0 + u) * 256 + t;
      const int ic = i < nch ? i : 0;
      const int mm = ic / C8, c = ic - mm * C8;
      mrow[u] = i < nch ? mm : -1;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[u][e] = load_elem<XT>(x, (int64_t)mm * ldx + 8 * c + e);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float sq = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sq += v[u][e] * v[u][e];
#pragma unroll
      for (int mm = 0; mm < MM; ++mm) ssr[mm] += mrow[u] == mm ? sq : 0.0f;
    }
  }
#pragma unroll
  for (int mm = 0; mm < MM; ++mm) {
    float v = ssr[mm];
    v += xor_lanes_f32<32>(v);
    v += xor_lanes_f32<16>(v);
    v += xor_lanes_f32<8>(v);
    v += xor_lanes_f32<4>(v);
    v += xor_lanes_f32<2>(v);
    v += xor_lanes_f32<1>(v);
    if (lane == 0) red[w][mm] = v;
  }
  __syncthreads();
  if (t < m) rs[t] = 1.0f / sqrtf((((red[0][t] + red[1][t]) + red[2][t]) + red[3][t]) / (float)h + eps);
  __syncthreads();
  // Pass 2: y = x * rs * gamma, rounded to x's dtype as the torch glue does, into LDS.
  for (int j0 = 0; j0 * 256 < nch; j0 += 2) {
    float v[2][8], gv[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = (j0 + u) * 256 + t;
      const int ic = i < nch ? i : 0;
      const int mm = ic / C8, c = ic - mm * C8;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[u][e] = load_elem<XT>(x, (int64_t)mm * ldx + 8 * c + e);
      // gamma's dtype tested once per chunk, so the 8 loads of a chunk go out together
      if (gamma == nullptr) {
#pragma unroll
        for (int e = 0; e < 8; ++e) gv[u][e] = 1.0f;
      } else if (gdt == WFB_F32) {
#pragma unroll
        for (int e = 0; e < 8; ++e) gv[u][e] = load_elem<WFB_F32>(gamma, 8 * c + e);
      } else if (gdt == WFB_BF16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) gv[u][e] = load_elem<WFB_BF16>(gamma, 8 * c + e);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) gv[u][e] = load_elem<WFB_F16>(gamma, 8 * c + e);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = (j0 + u) * 256 + t;
      if (i >= nch) break;
      const int mm = i / C8, c = i - mm * C8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float y = v[u][e] * rs[mm];
        if (gamma) y = y * gv[u][e];
        if constexpr (XT == WFB_BF16) y = bf16_bits_to_f32(f32_to_bf16_rne(y));
        xn[mm * h + 8 * c + e] = y;
      }
    }
  }
  __syncthreads();

  const int s = lane & 7, rsub = lane >> 3, C = h >> 3;
  const buf_t wb = make_buf(W, (uint32_t)((int64_t)n * ldw * ESZ));
  uint64_t best[MM];
#pragma unroll
  for (int mm = 0; mm < MM; ++mm) best[mm] = 0;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int row = blockIdx.x * 64 + w * 16 + p * 8 + rsub;
    const uint32_t roff = (uint32_t)((int64_t)row * ldw * ESZ);
    float acc[MM];
#pragma unroll
    for (int mm = 0; mm < MM; ++mm) acc[mm] = 0.0f;
    // U chunks' loads in flight per lane, then their arithmetic in chunk order (a one-load-then-wait loop
    // kept a single 16-byte load in flight per lane); chunks past the row read zeros from an out-of-range
    // offset (below 2^31, so offset + 16 cannot wrap) and add exactly +0
    constexpr int U = 4;
    for (int c0 = s; c0 < C; c0 += 8 * U) {
      v4i r0[U], r1[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + 8 * u;
        const uint32_t off = c < C ? roff + (uint32_t)(8 * c * ESZ) : 0x7FFFFF00u;
        r0[u] = buf_load16(wb, off);
        if constexpr (WT == WFB_F32) r1[u] = buf_load16(wb, off + 16);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + 8 * u < C ? c0 + 8 * u : 0;  // the LDS index stays in range (its weights are 0)
        float wv[8];
        if constexpr (WT == WFB_F32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            wv[e] = __int_as_float(r0[u][e]);
            wv[4 + e] = __int_as_float(r1[u][e]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            wv[2 * e] = __uint_as_float((uint32_t)r0[u][e] << 16);
            wv[2 * e + 1] = __uint_as_float((uint32_t)r0[u][e] & 0xffff0000u);
          }
        }
#pragma unroll
        for (int mm = 0; mm < MM; ++mm) {
          if (mm < m) {
            const float4* xp = reinterpret_cast<const float4*>(xn + mm * h + 8 * c);
            const float4 a = xp[0], b = xp[1];
            acc[mm] += wv[0] * a.x + wv[1] * a.y + wv[2] * a.z + wv[3] * a.w + wv[4] * b.x + wv[5] * b.y +
                       wv[6] * b.z + wv[7] * b.w;
          }
        }
      }
    }
    const bool valid = row < n && s == 0;
#pragma unroll
    for (int mm = 0; mm < MM; ++mm) {
      if (mm < m) {
        const float y = group_sum_f32<8>(acc[mm]);
        if (valid && logits) logits[(int64_t)mm * ldo + row] = y;
        const uint64_t key = group_max_u64<64>(valid ? amax_key(y, row) : 0);
        best[mm] = key > best[mm] ? key : best[mm];
      }
    }
  }
  const int slot = blockIdx.x * 4 + w;
  if (lane == 0 && slot < (n + 15) / 16) {
#pragma unroll
    for (int mm = 0; mm < MM; ++mm)
      if (mm < m) parts[(int64_t)slot * m + mm] = best[mm];
  }
}

template <int XT, int WT>
hipError_t launch_head_t(const void* x, int64_t ldx, const void* gamma, int gdt, float eps, const void* w, int64_t ldw,
                         int m, int n, int h, float* logits, int64_t ldo, uint64_t* parts, hipStream_t s) {
  const dim3 grid((n + 63) / 64);
  const size_t lds = (size_t)m * h * sizeof(float);
#define WFB_HEAD(MMV) \
  hipLaunchKernelGGL((lm_head_kernel<XT, WT, MMV>), grid, dim3(256), lds, s, x, ldx, gamma, gdt, eps, w, ldw, m, n, h, \
                     logits, ldo, parts)
  if (m <= 1) WFB_HEAD(1);
  else if (m <= 2) WFB_HEAD(2);
  else if (m <= 4) WFB_HEAD(4);
  else if (m <= 8) WFB_HEAD(8);
  else WFB_HEAD(16);
#undef WFB_HEAD
  return hipGetLastError();
}

}  // namespace

hipError_t launch_argmax_finalize(const uint64_t* parts, int64_t n_parts, int64_t m, int64_t* tokens, hipStream_t s) {
  if (n_parts * m * 8 < ((int64_t)1 << 32))
    hipLaunchKernelGGL((argmax_finalize_kernel<true>), dim3((unsigned)m), dim3(kFinThreads), 0, s, parts, n_parts, (int)m,
                       tokens);
  else
    hipLaunchKernelGGL((argmax_finalize_kernel<false>), dim3((unsigned)m), dim3(kFinThreads), 0, s, parts, n_parts, (int)m,
                       tokens);
  return hipGetLastError();
}

hipError_t launch_lm_head_argmax(const void* x, int xdt, int64_t ldx, const void* gamma, int gdt, float eps,
                                 const void* w, int wdt, int64_t ldw, int64_t m, int64_t n, int64_t h, float* logits,
                                 int64_t ldo, uint64_t* parts, hipStream_t s) {
  if (xdt == WFB_F32 && wdt == WFB_F32)
    return launch_head_t<WFB_F32, WFB_F32>(x, ldx, gamma, gdt, eps, w, ldw, (int)m, (int)n, (int)h, logits, ldo, parts, s);
  if (xdt == WFB_F32 && wdt == WFB_BF16)
    return launch_head_t<WFB_F32, WFB_BF16>(x, ldx, gamma, gdt, eps, w, ldw, (int)m, (int)n, (int)h, logits, ldo, parts, s);
  if (xdt == WFB_BF16 && wdt == WFB_F32)
    return launch_head_t<WFB_BF16, WFB_F32>(x, ldx, gamma, gdt, eps, w, ldw, (int)m, (int)n, (int)h, logits, ldo, parts, s);
  return launch_head_t<WFB_BF16, WFB_BF16>(x, ldx, gamma, gdt, eps, w, ldw, (int)m, (int)n, (int)h, logits, ldo, parts, s);
}

}  // namespace wfb
