// GQA decode attention over a KV cache, one new token per sequence, with the rotary embedding of
// the new query/key and the cache append fused in.
//
// Replaces attention_forward (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:381-441: GQA with
// kv_h = h / (heads / kv_heads), scores q.k * 1/sqrt(head_dim) over positions 0..pos, softmax, weighted
// sum of V) and the cache writes kv_cache_update_key / kv_cache_update_value
// (SGB/sgl-kernel/csrc/inference/kv_cache.h:81-101).  The C engine has no rotary embedding; the stage-1
// model does (HF rotate-half form, packages/training/src/wrinklefree/training/stage1.py:169-214), so it
// is applied here when tables are given:
//   y[j] = x[j] * cos[pos, j] + (-x[j + D/2]) * sin[pos, j],  y[j + D/2] = x[j + D/2] * cos[pos, j] + x[j] * sin[pos, j]
// each product and sum rounded to fp32 (the same operations as the torch formula), then rounded to
// the storage type.
//
// Cache layout: [batch, kv_heads, max_len, head_dim] for K and V (one key = head_dim contiguous
// elements).  One workgroup per (kv head, sequence) owns that cache slice: it writes the new key and
// value at pos and attends over keys 0..pos, taking key pos from its own LDS copy (no read-back of its
// own global store).  The G = heads / kv_heads query heads of the group share every K/V load.
//
// Work mapping (4 waves).  A key is read by LPK = D/8 lanes, 8 elements each (one 16-byte load for
// 16-bit caches), so one wave instruction covers 64/LPK whole keys and a wave's loads are contiguous.
// Keys are processed in chunks of CH; per chunk each wave loads its CH/4 keys of K and V up front,
// forms the G partial dot products per lane against its 8 query elements (held in registers), sums them
// over the key's LPK lanes with DPP, and parks the scores in LDS.  A running (online) softmax per head
// -- chunk max, rescale factor exp(m_old - m_new), exp(s - m_new), running sum -- is kept by the wave
// that owns the head; then each lane accumulates p * v for its keys and 8 elements.  At the end the
// per-lane partial outputs are summed over the lanes of a wave sharing the same elements (xor
// shuffles), then over the 4 waves in LDS, and divided by the softmax sum.
#include "wfb_common.h"

namespace wfb {

namespace {

constexpr int kAttnThreads = 256;

template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == WFB_F32) return x;
  else return bf16_bits_to_f32(f32_to_bf16_rne(x));
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
  if constexpr (DT == WFB_F32) reinterpret_cast<float*>(p)[i] = v;
  else reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(v);
}

// 8 elements of a cache row as raw bits: one 16-byte load (16-bit types) or two (fp32).
template <int CT>
struct Raw8 {
  v4i r[CT == WFB_F32 ? 2 : 1];
};

template <int CT>
__device__ __forceinline__ Raw8<CT> load_raw8(buf_t b, uint32_t off) {
  Raw8<CT> x;
  x.r[0] = buf_load16(b, off);
  if constexpr (CT == WFB_F32) x.r[1] = buf_load16(b, off + 16);
  return x;
}

template <int CT>
__device__ __forceinline__ void widen8(const Raw8<CT>& x, float (&v)[8]) {
  if constexpr (CT == WFB_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __int_as_float(x.r[0][e]);
      v[4 + e] = __int_as_float(x.r[1][e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t u = (uint32_t)x.r[0][e];
      v[2 * e] = __uint_as_float(u << 16);
      v[2 * e + 1] = __uint_as_float(u & 0xffff0000u);
    }
  }
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int DT, int D, int G>
__global__ __launch_bounds__(kAttnThreads) void gqa_decode_kernel(
    const void* __restrict__ q, int64_t ldq, const void* __restrict__ kn, int64_t ldk, const void* __restrict__ vn,
    int64_t ldv, const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, void* __restrict__ kc,
    void* __restrict__ vc, int64_t max_len, const int64_t* __restrict__ pos_arr, int hkv, float scale,
    void* __restrict__ out, int64_t ldo) {
  constexpr int LPK = D / 8;           // lanes per key
  constexpr int KPW = 64 / LPK;        // keys per wave instruction
  constexpr int CH = DT == WFB_F32 ? 128 : 256;  // keys per chunk
  constexpr int KW = CH / 4;           // keys per wave per chunk
  constexpr int R = KW / KPW;          // load rounds per wave per chunk
  constexpr int ESZ = DT == WFB_F32 ? 4 : 2;
  constexpr int HD = D / 2;
  constexpr int HPW = (G + 3) / 4;     // heads per wave in the softmax step
  static_assert(R * KPW * 4 == CH, "chunk must tile the waves");

  __shared__ float qs[G][D];
  __shared__ float knew[D], vnew[D];
  __shared__ float sc[G][CH];
  __shared__ float alpha_s[G], lsum_s[G];
  __shared__ float red[4][G][D];

  const int kvh = blockIdx.x, b = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t pos = pos_arr[b];
  const int64_t obase = (int64_t)b * ldo + (int64_t)kvh * G * D;
  if (pos < 0 || pos >= max_len) {  // uniform over the workgroup: flag the rows, touch no cache
    for (int i = t; i < G * D; i += kAttnThreads) store_elem<DT>(out, obase + i, __builtin_nanf(""));
    return;
  }
  const int64_t cbase = ((int64_t)b * hkv + kvh) * max_len * D;  // element offset of this cache slice

  // ---- rotary embedding of the new query heads and key; append key and value ------------------
  const float* cs = rope_cos ? rope_cos + pos * HD : nullptr;
  const float* sn = rope_sin ? rope_sin + pos * HD : nullptr;
  for (int i = t; i < G * HD; i += kAttnThreads) {
    const int g = i / HD, j = i % HD;
    const int64_t qo = (int64_t)b * ldq + (int64_t)(kvh * G + g) * D;
    float x1 = load_elem<DT>(q, qo + j), x2 = load_elem<DT>(q, qo + j + HD);
    if (cs) {
      const float c = cs[j], s = sn[j];
      const float y1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(-x2, s));
      const float y2 = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));
      x1 = round_to<DT>(y1);
      x2 = round_to<DT>(y2);
    }
    qs[g][j] = x1;
    qs[g][j + HD] = x2;
  }
  if (t < HD) {
    const int64_t ko = (int64_t)b * ldk + (int64_t)kvh * D;
    float x1 = load_elem<DT>(kn, ko + t), x2 = load_elem<DT>(kn, ko + t + HD);
    if (cs) {
      const float c = cs[t], s = sn[t];
      const float y1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(-x2, s));
      const float y2 = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));
      x1 = round_to<DT>(y1);
      x2 = round_to<DT>(y2);
    }
    knew[t] = x1;
    knew[t + HD] = x2;
    store_elem<DT>(kc, cbase + pos * D + t, x1);
    store_elem<DT>(kc, cbase + pos * D + t + HD, x2);
  } else if (t >= 64 && t < 64 + D) {
    const int j = t - 64;
    const float x = load_elem<DT>(vn, (int64_t)b * ldv + (int64_t)kvh * D + j);
    vnew[j] = x;
    store_elem<DT>(vc, cbase + pos * D + j, x);
  }
  __syncthreads();

  const int kl = lane / LPK;        // key slot of the lane within a wave instruction
  const int d0 = 8 * (lane % LPK);  // first of the lane's 8 elements
  float qf[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[g][e] = qs[g][d0 + e];
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
  float m_run[HPW], l_run[HPW];
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    m_run[h] = -__builtin_inff();
    l_run[h] = 0.0f;
  }

  // keys 0..pos-1 come from the cache (loads past them read zeros); key pos from knew / vnew
  const uint32_t kbytes = (uint32_t)(pos * D * ESZ);
  const buf_t kb = make_buf(reinterpret_cast<const char*>(kc) + cbase * ESZ, kbytes);
  const buf_t vb = make_buf(reinterpret_cast<const char*>(vc) + cbase * ESZ, kbytes);
  const int nk = (int)pos + 1;

  for (int c0 = 0; c0 < nk; c0 += CH) {
    Raw8<DT> kr[R], vr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int key = c0 + w * KW + r * KPW + kl;
      const uint32_t off = (uint32_t)(key * D + d0) * ESZ;
      kr[r] = load_raw8<DT>(kb, off);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int key = c0 + w * KW + r * KPW + kl;
      const uint32_t off = (uint32_t)(key * D + d0) * ESZ;
      vr[r] = load_raw8<DT>(vb, off);
    }
    // scores
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int key = c0 + w * KW + r * KPW + kl;
      float kf[8];
      widen8<DT>(kr[r], kf);
      if (key == pos) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[e] = knew[d0 + e];
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += qf[g][e] * kf[e];
        s = group_sum_f32<LPK>(s);
        if (lane % LPK == 0) sc[g][key - c0] = key <= pos ? s * scale : -__builtin_inff();
      }
    }
    __syncthreads();
    // online softmax: wave w owns heads w, w + 4
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      const int g = w + 4 * h;
      if (g < G) {
        float v[CH / 64];
        float mx = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < CH / 64; ++i) {
          v[i] = sc[g][lane + 64 * i];
          mx = fmaxf(mx, v[i]);
        }
        const float m_new = fmaxf(m_run[h], wave_max_f32(mx));
        const float a = __expf(m_run[h] - m_new);
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < CH / 64; ++i) {
          const float p = __expf(v[i] - m_new);
          sc[g][lane + 64 * i] = p;
          ps += p;
        }
        l_run[h] = l_run[h] * a + wave_sum_f32(ps);
        m_run[h] = m_new;
        if (lane == 0) alpha_s[g] = a;
      }
    }
    __syncthreads();
    // weighted sum of values
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float a = alpha_s[g];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= a;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int key = c0 + w * KW + r * KPW + kl;
      float vf[8];
      widen8<DT>(vr[r], vf);
      if (key == pos) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[e] = vnew[d0 + e];
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = sc[g][key - c0];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] += p * vf[e];
      }
    }
    __syncthreads();  // sc and alpha_s are rewritten by the next chunk
  }

  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < HPW; ++h)
      if (w + 4 * h < G) lsum_s[w + 4 * h] = l_run[h];
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[g][e];
#pragma unroll
      for (int o = LPK; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
      if (kl == 0) red[w][g][d0 + e] = v;
    }
  __syncthreads();
  for (int i = t; i < G * D; i += kAttnThreads) {
    const int g = i / D, d = i % D;
    const float s = (red[0][g][d] + red[1][g][d]) + (red[2][g][d] + red[3][g][d]);
    store_elem<DT>(out, obase + i, s / lsum_s[g]);
  }
}

template <int DT, int D, int G>
hipError_t launch_attn_g(const void* q, int64_t ldq, const void* kn, int64_t ldk, const void* vn, int64_t ldv,
                         const float* rc, const float* rs, void* kc, void* vc, int64_t max_len, const int64_t* pos,
                         int b, int hkv, float scale, void* out, int64_t ldo, hipStream_t s) {
  hipLaunchKernelGGL((gqa_decode_kernel<DT, D, G>), dim3(hkv, b), dim3(kAttnThreads), 0, s, q, ldq, kn, ldk, vn, ldv,
                     rc, rs, kc, vc, max_len, pos, hkv, scale, out, ldo);
  return hipGetLastError();
}

template <int DT, int D>
hipError_t launch_attn_d(int g, const void* q, int64_t ldq, const void* kn, int64_t ldk, const void* vn, int64_t ldv,
                         const float* rc, const float* rs, void* kc, void* vc, int64_t max_len, const int64_t* pos,
                         int b, int hkv, float scale, void* out, int64_t ldo, hipStream_t s) {
#define WFB_ATTN_G(GG) \
  case GG: return launch_attn_g<DT, D, GG>(q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, s)
  switch (g) {
    WFB_ATTN_G(1);
    WFB_ATTN_G(2);
    WFB_ATTN_G(3);
    WFB_ATTN_G(4);
    WFB_ATTN_G(5);
    WFB_ATTN_G(6);
    WFB_ATTN_G(7);
    WFB_ATTN_G(8);
    default: return hipErrorInvalidValue;
  }
#undef WFB_ATTN_G
}

}  // namespace

hipError_t launch_gqa_decode(int dt, int d, int g, const void* q, int64_t ldq, const void* kn, int64_t ldk,
                             const void* vn, int64_t ldv, const float* rc, const float* rs, void* kc, void* vc,
                             int64_t max_len, const int64_t* pos, int b, int hkv, float scale, void* out, int64_t ldo,
                             hipStream_t s) {
  if (dt == WFB_F32 && d == 64)
    return launch_attn_d<WFB_F32, 64>(g, q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, s);
  if (dt == WFB_F32 && d == 128)
    return launch_attn_d<WFB_F32, 128>(g, q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, s);
  if (dt == WFB_BF16 && d == 64)
    return launch_attn_d<WFB_BF16, 64>(g, q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, s);
  if (dt == WFB_BF16 && d == 128)
    return launch_attn_d<WFB_BF16, 128>(g, q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, s);
  return hipErrorInvalidValue;
}

}  // namespace wfb
