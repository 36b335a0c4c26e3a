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
// Split context (flash decoding).  With few sequences and kv heads a workgroup per (kv head, sequence)
// leaves most of the GPU idle, so the keys are cut into splits of KS keys, one workgroup each (grid z);
// split s covers keys [s*KS, min(pos+1, (s+1)*KS)) and writes its unnormalised output with its running
// max m and sum l to a workspace, and gqa_combine_kernel merges the splits that hold keys
// (out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M), M = max_s m_s).  The split holding pos appends
// the new key and value.  The grid holds ceil(max_len / KS_MIN) splits (KS_MIN = 64 keys unless the
// combine's staging would outgrow its LDS), fixed by max_len; KS itself is read from pos on the device
// (KS_MIN doubled while the sequence would need more splits than its share of the GPU), so a captured
// HIP graph stays valid as pos advances; splits past pos exit at once.
//
// Work mapping (4 waves).  A key is read by LPK = D/8 lanes, 8 elements each (one 16-byte load for
// 16-bit caches), so one wave instruction covers 64/LPK whole keys and a wave's loads are contiguous.
// Keys are processed in chunks of CH; per chunk each wave loads its CH/4 keys of K and V up front.
// bf16 caches: the scores go through the matrix cores, S[head, key] = Q K^T per 16 keys of a wave
// (v_mfma_f32_16x16x32_bf16: A = the group's query heads as rows, zero past G; B = the 16 keys as
// columns, a lane's fragment being 16 contiguous bytes of its key's row; k = 32 head dimensions per
// step), the products of bf16 operands exact in fp32 and summed in fp32.  The appended key pos is not
// among the cache reads; its G scores are computed once per workgroup from the LDS copy of the key.
// fp32 caches: each lane forms the G partial dot products against its 8 query elements (held in
// registers) and they are summed over the key's LPK lanes with DPP.  The scores are parked in LDS.  A
// running (online) softmax per head -- chunk max, rescale factor exp(m_old - m_new), exp(s - m_new),
// running sum -- is kept by the wave that owns the head; then each lane accumulates p * v for its keys
// and 8 elements.  At the end the per-lane partial outputs are summed over the lanes of a wave sharing
// the same elements (xor shuffles), then over the 4 waves in LDS, and divided by the softmax sum.
#include <mutex>

#include "wfb_common.h"

// Split partials of wfb_gqa_decode_attention_noalloc, the entry point that allocates nothing: one copy
// per GPU, held for the life of the process (a device global of the code object).  Host code never
// passes this name to a kernel or a copy: it is a host-side stand-in, and the device address comes
// from hipGetSymbolAddress (wfb::gqa_decode_scratch below).
static __device__ __align__(256) float scratch[wfb::kAttnScratchFloats];

namespace wfb {

namespace {

constexpr int kAttnThreads = 256;
constexpr int64_t kAttnMaxSplitHeads = 4096;  // splits x heads staged by the combine (32 KB of LDS)

// Keys per split: 64, doubled only while the combine's LDS staging of the split weights (splits x
// query heads per kv head) would pass kAttnMaxSplitHeads.
int64_t split_keys(int64_t max_len, int g) {
  int64_t ks = 64;
  while (ks < max_len && ((max_len + ks - 1) / ks) * g > kAttnMaxSplitHeads) ks *= 2;
  return ks;
}

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
  v = fmaxf(v, xor_lanes_f32<32>(v));
  v = fmaxf(v, xor_lanes_f32<16>(v));
  v = fmaxf(v, xor_lanes_f32<8>(v));
  v = fmaxf(v, xor_lanes_f32<4>(v));
  v = fmaxf(v, xor_lanes_f32<2>(v));
  return fmaxf(v, xor_lanes_f32<1>(v));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  v += xor_lanes_f32<32>(v);
  v += xor_lanes_f32<16>(v);
  v += xor_lanes_f32<8>(v);
  v += xor_lanes_f32<4>(v);
  v += xor_lanes_f32<2>(v);
  return v + xor_lanes_f32<1>(v);
}

// sum over the lanes l, l ^ LPK, l ^ 2 LPK, ... (partners LPK, 2 LPK, .., 32 in that order)
template <int LPK>
__device__ __forceinline__ float sum_across_keys(float v) {
  if constexpr (LPK <= 1) v += xor_lanes_f32<1>(v);
  if constexpr (LPK <= 2) v += xor_lanes_f32<2>(v);
  if constexpr (LPK <= 4) v += xor_lanes_f32<4>(v);
  if constexpr (LPK <= 8) v += xor_lanes_f32<8>(v);
  if constexpr (LPK <= 16) v += xor_lanes_f32<16>(v);
  if constexpr (LPK <= 32) v += xor_lanes_f32<32>(v);
  return v;
}

// Keys per split of a sequence at position pos: ks doubled while the keys 0..pos would need more than spt
// splits (spt = 0: ks as given).  Read from the device-side position by the split and combine kernels
// alike, so a captured launch adapts to the position it is replayed at.
__device__ inline int split_len(int64_t pos, int ks, int spt) {
  if (spt > 0)
    while ((pos + ks) / ks > spt) ks *= 2;  // ceil((pos + 1) / ks) splits
  return ks;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// (PF, bf16: three workgroups per CU -- at most 168 registers -- where the register budget allows it)
template <int DT, int D, int G, int CH, bool PF = false>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(PF && DT == WFB_BF16 && G <= 4 ? 3 : 1)))
void gqa_decode_kernel(
    const void* __restrict__ q, int64_t ldq, const void* __restrict__ kn, int64_t ldk, const void* __restrict__ vn,
    int64_t ldv, const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, void* __restrict__ kc,
    void* __restrict__ vc, int64_t max_len, const int64_t* __restrict__ pos_arr, int hkv, float scale,
    void* __restrict__ out, int64_t ldo, int ks_min, int spt, float* __restrict__ part) {
  constexpr int LPK = D / 8;           // lanes per key
  constexpr int KPW = 64 / LPK;        // keys per wave instruction
  constexpr int KW = CH / 4;           // keys per wave per chunk (CH keys per chunk)
  constexpr int R = KW / KPW;          // load rounds per wave per chunk
  constexpr int ESZ = DT == WFB_F32 ? 4 : 2;
  constexpr int HD = D / 2;
  constexpr int HPW = (G + 3) / 4;     // heads per wave in the softmax step
  static_assert(R * KPW * 4 == CH, "chunk must tile the waves");
  constexpr bool MQ = DT == WFB_BF16;  // scores on the matrix cores
  constexpr int NTL = KW / 16;         // (MQ) 16-key MFMA tiles per wave and chunk
  static_assert(!MQ || (KW % 16 == 0 && D % 32 == 0 && G <= 16 && R == NTL * (D / 32)), "matrix-core score tiles");

  __shared__ float qs[G][D];
  __shared__ float knew[D], vnew[D];
  __shared__ float sc[G][CH];
  __shared__ float alpha_s[G], lsum_s[G];
  __shared__ float snew_s[G];  // (MQ) scores of the appended key
  __shared__ float red[4][G][D];

  const int kvh = blockIdx.x, b = blockIdx.y, split = blockIdx.z;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t pos = pos_arr[b];
  const int64_t obase = (int64_t)b * ldo + (int64_t)kvh * G * D;
  if (pos < 0 || pos >= max_len) {  // uniform over the workgroup: flag the rows, touch no cache
    if (!part)
      for (int i = t; i < G * D; i += kAttnThreads) store_elem<DT>(out, obase + i, __builtin_nanf(""));
    return;  // (split mode: the combine kernel flags the rows)
  }
  const int ks = split_len(pos, ks_min, spt);
  if ((int64_t)split * ks > pos) return;  // no keys in this split (the combine kernel skips it)
  const int k0 = split * ks;
  const int k1 = (int)(pos + 1 < (int64_t)k0 + ks ? pos + 1 : (int64_t)k0 + ks);
  const bool owns_new = pos < k1;  // the split holding key pos appends the new key and value
  const int64_t cbase = ((int64_t)b * hkv + kvh) * max_len * D;  // element offset of this cache slice

  // keys k0..min(pos, k1)-1 come from the cache (loads past them read zeros); key pos from knew / vnew.
  // The first chunk's K and V rows are requested before the rotary arithmetic and the append: the range
  // never includes pos, so they do not wait for this workgroup's own append.
  const int kl = lane / LPK;        // key slot of the lane within a wave instruction
  const int d0 = 8 * (lane % LPK);  // first of the lane's 8 elements
  const int kend = owns_new ? (int)pos : k1;
  const uint32_t kbytes = (uint32_t)((int64_t)kend * D * ESZ);
  const buf_t kb = make_buf(reinterpret_cast<const char*>(kc) + cbase * ESZ, kbytes);
  const buf_t vb = make_buf(reinterpret_cast<const char*>(vc) + cbase * ESZ, kbytes);
  // PF: two register sets of K, the next chunk's keys requested before the current chunk is used and
  // its values right after the current chunk's values are consumed
  Raw8<DT> kr[PF ? 2 : 1][R], vr[R];
  auto load_k = [&](int c0, int set) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (MQ) {  // B fragment j of tile tl: key 16 tl + lane % 16, dimensions 32 j + 8 (lane / 16) ..
        const int tl = r / (D / 32), j = r % (D / 32);
        const int key = c0 + w * KW + 16 * tl + (lane & 15);
        kr[set][r] = load_raw8<DT>(kb, (uint32_t)(key * D + 32 * j + 8 * (lane >> 4)) * ESZ);
      } else {
        const int key = c0 + w * KW + r * KPW + kl;
        kr[set][r] = load_raw8<DT>(kb, (uint32_t)(key * D + d0) * ESZ);
      }
    }
  };
  auto load_v = [&](int c0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int key = c0 + w * KW + r * KPW + kl;
      vr[r] = load_raw8<DT>(vb, (uint32_t)(key * D + d0) * ESZ);
    }
  };
  // ---- rotary embedding of the new query heads and key; append key and value ------------------
  // This phase's loads are issued before the first chunk's K and V rows: loads complete in issue order,
  // so a load issued after them would make its use wait for the chunk as well.  Indices are clamped
  // into range instead of guarding the loads, so every wave issues the same loads.
  const float* cs = rope_cos ? rope_cos + pos * HD : nullptr;
  const float* sn = rope_sin ? rope_sin + pos * HD : nullptr;
  constexpr int NQ = (G * HD + kAttnThreads - 1) / kAttnThreads;
  float qx1[NQ], qx2[NQ], qc[NQ], qsi[NQ];
#pragma unroll
  for (int it = 0; it < NQ; ++it) {
    const int i = t + it * kAttnThreads < G * HD ? t + it * kAttnThreads : G * HD - 1;
    const int g = i / HD, j = i % HD;
    const int64_t qo = (int64_t)b * ldq + (int64_t)(kvh * G + g) * D;
    qx1[it] = load_elem<DT>(q, qo + j);
    qx2[it] = load_elem<DT>(q, qo + j + HD);
    qc[it] = cs ? cs[j] : 1.0f;
    qsi[it] = cs ? sn[j] : 0.0f;
  }
  const int tk = t < HD ? t : HD - 1, tv = t < 64 ? 0 : t < 64 + D ? t - 64 : D - 1;
  const int64_t ko = (int64_t)b * ldk + (int64_t)kvh * D;
  const float kx1 = load_elem<DT>(kn, ko + tk), kx2 = load_elem<DT>(kn, ko + tk + HD);
  const float kcs = cs ? cs[tk] : 1.0f, ksn = cs ? sn[tk] : 0.0f;
  const float vx = load_elem<DT>(vn, (int64_t)b * ldv + (int64_t)kvh * D + tv);
  load_k(k0, 0);
  load_v(k0);

#pragma unroll
  for (int it = 0; it < NQ; ++it) {
    const int i = t + it * kAttnThreads;
    if (i >= G * HD) break;
    const int g = i / HD, j = i % HD;
    float x1 = qx1[it], x2 = qx2[it];
    if (cs) {
      const float y1 = __fadd_rn(__fmul_rn(x1, qc[it]), __fmul_rn(-x2, qsi[it]));
      const float y2 = __fadd_rn(__fmul_rn(x2, qc[it]), __fmul_rn(x1, qsi[it]));
      x1 = round_to<DT>(y1);
      x2 = round_to<DT>(y2);
    }
    qs[g][j] = x1;
    qs[g][j + HD] = x2;
  }
  if (!owns_new) {
  } else if (t < HD) {
    float x1 = kx1, x2 = kx2;
    if (cs) {
      const float y1 = __fadd_rn(__fmul_rn(x1, kcs), __fmul_rn(-x2, ksn));
      const float y2 = __fadd_rn(__fmul_rn(x2, kcs), __fmul_rn(x1, ksn));
      x1 = round_to<DT>(y1);
      x2 = round_to<DT>(y2);
    }
    knew[t] = x1;
    knew[t + HD] = x2;
    store_elem<DT>(kc, cbase + pos * D + t, x1);
    store_elem<DT>(kc, cbase + pos * D + t + HD, x2);
  } else if (t >= 64 && t < 64 + D) {
    const int j = t - 64;
    vnew[j] = vx;
    store_elem<DT>(vc, cbase + pos * D + j, vx);
  }
  __syncthreads();

  // the lane's 8 query elements per head; for 16-bit caches as bf16 pairs (the rotated query was rounded
  // to the storage type, so the pairs hold it exactly) to leave registers for the prefetched keys
  constexpr bool QP = DT != WFB_F32;
  float qf[QP ? 1 : G][8];
  uint32_t qp[QP && !MQ ? G : 1][4];
  v4i qa[MQ ? D / 32 : 1];  // (MQ) A fragments: row = head lane % 16, dimensions 32 j + 8 (lane / 16) ..
  if constexpr (MQ) {
    const int h = lane & 15;
#pragma unroll
    for (int j = 0; j < D / 32; ++j)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int dd = 32 * j + 8 * (lane >> 4) + e;
        qa[j][e / 2] =
            h < G ? (int)((__float_as_uint(qs[h][dd]) >> 16) | (__float_as_uint(qs[h][dd + 1]) & 0xffff0000u)) : 0;
      }
    if (owns_new) {  // the appended key's scores: wave w takes heads w, w + 4, ..
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        const int g = w + 4 * hh;
        if (g < G) {
          float p = 0.0f;
#pragma unroll
          for (int e = 0; e < D / 64; ++e) p += qs[g][lane + 64 * e] * knew[lane + 64 * e];
          p = wave_sum_f32(p);
          if (lane == 0) snew_s[g] = p;
        }
      }
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        if constexpr (QP)
          qp[g][e / 2] = (__float_as_uint(qs[g][d0 + e]) >> 16) | (__float_as_uint(qs[g][d0 + e + 1]) & 0xffff0000u);
        else {
          qf[g][e] = qs[g][d0 + e];
          qf[g][e + 1] = qs[g][d0 + e + 1];
        }
      }
  }
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

  // one chunk of CH keys from register set `set`: scores, online softmax, weighted sum of values
  auto chunk = [&](int c0, int set) {
    // scores (the empty asm keeps the query pairs packed across chunks: without it the compiler
    // widens them once, ahead of the loop, into twice the registers)
    if constexpr (QP && !MQ)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(qp[g][i]));
    if constexpr (MQ) {
#pragma unroll
      for (int tl = 0; tl < NTL; ++tl) {
        f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < D / 32; ++j)
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qa[j]),
                                                       __builtin_bit_cast(bf16x8_t, kr[set][tl * (D / 32) + j].r[0]), c,
                                                       0, 0, 0);
        // lane l holds S[head 4 (l / 16) + i, key 16 tl + l % 16]
        const int key = c0 + w * KW + 16 * tl + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int g = 4 * (lane >> 4) + i;
          if (g < G) {
            const float sv = owns_new && key == pos ? snew_s[g] : c[i];
            sc[g][key - c0] = key < k1 ? sv * scale : -__builtin_inff();
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < (MQ ? 0 : R); ++r) {
      const int key = c0 + w * KW + r * KPW + kl;
      float kf[8];
      widen8<DT>(kr[set][r], kf);
      // only the split that owns pos wrote knew / vnew; a chunk longer than the split (CH > ks) can
      // reach key pos in a split that does not own it, where the key is masked and must stay finite
      if (owns_new && key == pos) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[e] = knew[d0 + e];
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float qe;
          if constexpr (QP)
            qe = __uint_as_float(e % 2 ? qp[g][e / 2] & 0xffff0000u : qp[g][e / 2] << 16);
          else
            qe = qf[g][e];
          s += qe * kf[e];
        }
        s = group_sum_f32<LPK>(s);
        if (lane % LPK == 0) sc[g][key - c0] = key < k1 ? s * scale : -__builtin_inff();
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
      if (owns_new && key == pos) {
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
  };
  if constexpr (PF) {
    // software pipelined: chunk c + 1's keys are in flight while chunk c is used, its values from the
    // end of chunk c's weighted sum (loads complete in issue order, so each use waits only for its own)
    for (int c0 = k0; c0 < k1; c0 += 2 * CH) {
      if (c0 + CH < k1) load_k(c0 + CH, 1);
      chunk(c0, 0);
      if (c0 + CH >= k1) break;
      load_v(c0 + CH);
      if (c0 + 2 * CH < k1) load_k(c0 + 2 * CH, 0);
      chunk(c0 + CH, 1);
      if (c0 + 2 * CH < k1) load_v(c0 + 2 * CH);
    }
  } else {
    for (int c0 = k0; c0 < k1; c0 += CH) {
      if (c0 != k0) {
        load_k(c0, 0);
        load_v(c0);
      }
      chunk(c0, 0);
    }
  }

  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < HPW; ++h)
      if (w + 4 * h < G) {
        lsum_s[w + 4 * h] = l_run[h];
        alpha_s[w + 4 * h] = m_run[h];  // the running max (alpha_s is free after the last chunk)
      }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = sum_across_keys<LPK>(acc[g][e]);
      if (kl == 0) red[w][g][d0 + e] = v;
    }
  __syncthreads();
  if (part) {  // split: unnormalised output, then m and l, per head
    float* pp = part + ((((int64_t)b * hkv + kvh) * gridDim.z + split) * G) * (D + 2);
    for (int i = t; i < G * D; i += kAttnThreads) {
      const int g = i / D, d = i % D;
      pp[g * (D + 2) + d] = (red[0][g][d] + red[1][g][d]) + (red[2][g][d] + red[3][g][d]);
    }
    if (t < G) {
      pp[t * (D + 2) + D] = alpha_s[t];
      pp[t * (D + 2) + D + 1] = lsum_s[t];
    }
    return;
  }
  for (int i = t; i < G * D; i += kAttnThreads) {
    const int g = i / D, d = i % D;
    const float s = (red[0][g][d] + red[1][g][d]) + (red[2][g][d] + red[3][g][d]);
    store_elem<DT>(out, obase + i, s / lsum_s[g]);
  }
}

// Merges the splits of one (kv head, sequence) that hold keys: splits 0 .. pos / KS, KS the sequence's
// split length (split_len).
template <int DT, int D, int G>
__global__ __launch_bounds__(kAttnThreads) void gqa_combine_kernel(const float* __restrict__ part,
                                                                   const int64_t* __restrict__ pos_arr,
                                                                   int64_t max_len, int hkv, int ks_min, int spt,
                                                                   int nsplit, void* __restrict__ out, int64_t ldo) {
  // LDS: the running max m and sum l of every (split, head), then the per-head denominators.  The
  // partials are read with independent loads (m and l once per workgroup, the accumulators unrolled
  // over the splits) rather than as a chain of dependent loops per output element.
  extern __shared__ float cw[];
  const int kvh = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int64_t pos = pos_arr[b];
  const int64_t obase = (int64_t)b * ldo + (int64_t)kvh * G * D;
  if (pos < 0 || pos >= max_len) {
    for (int i = t; i < G * D; i += kAttnThreads) store_elem<DT>(out, obase + i, __builtin_nanf(""));
    return;
  }
  const int ns = (int)(pos / split_len(pos, ks_min, spt)) + 1;  // <= nsplit
  const float* pp = part + (((int64_t)b * hkv + kvh) * nsplit) * G * (D + 2);
  float* sm = cw;                // [ns * G]: m, then the split weights e^(m_s - M)
  float* sl = cw + nsplit * G;   // [ns * G]: l
  float* sden = sl + nsplit * G; // [G]
  // Up to kPre splits: the accumulators of the thread's output elements are requested together with m
  // and l (one round trip to the partials instead of two).
  constexpr int kPre = 16, EPT = (G * D + kAttnThreads - 1) / kAttnThreads;
  const bool pre = ns <= kPre;  // uniform
  float pa[EPT][kPre];
  if (pre) {
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int i = t + kAttnThreads * k;
      const int g = i / D, d = i % D;
#pragma unroll
      for (int s = 0; s < kPre; ++s) pa[k][s] = (i < G * D && s < ns) ? pp[(s * G + g) * (D + 2) + d] : 0.0f;
    }
  }
  for (int i = t; i < ns * G; i += kAttnThreads) {
    sm[i] = pp[i * (D + 2) + D];
    sl[i] = pp[i * (D + 2) + D + 1];
  }
  __syncthreads();
  if (t < G) {
    float mx = -__builtin_inff();
    for (int s = 0; s < ns; ++s) mx = fmaxf(mx, sm[s * G + t]);
    float den = 0.0f;
    for (int s = 0; s < ns; ++s) {
      const float wgt = __expf(sm[s * G + t] - mx);
      sm[s * G + t] = wgt;
      den += sl[s * G + t] * wgt;
    }
    sden[t] = den;
  }
  __syncthreads();
  if (pre) {
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int i = t + kAttnThreads * k;
      if (i >= G * D) break;
      const int g = i / D;
      float num = 0.0f;
#pragma unroll
      for (int s = 0; s < kPre; ++s)
        if (s < ns) num += pa[k][s] * sm[s * G + g];
      store_elem<DT>(out, obase + i, num / sden[g]);
    }
    return;
  }
  for (int i = t; i < G * D; i += kAttnThreads) {
    const int g = i / D, d = i % D;
    float num = 0.0f;
#pragma unroll 8
    for (int s = 0; s < ns; ++s) num += pp[(s * G + g) * (D + 2) + d] * sm[s * G + g];
    store_elem<DT>(out, obase + i, num / sden[g]);
  }
}

// Split attention and the combine.  spt = 0: splits of ks_min keys, ceil(max_len / ks_min) of them per
// (kv head, sequence).  spt > 0: a sequence at position pos uses ceil((pos + 1) / KS) <= spt splits of
// KS = split_len(pos, ks_min, spt) keys, so the grid holds min(spt, ceil(max_len / ks_min)) splits and no
// workgroups that would only find their split empty; the split kernel walks its keys in chunks of 64 with
// the next chunk's K and V loads in flight.
template <int DT, int D, int G>
hipError_t launch_attn_split(const void* q, int64_t ldq, const void* kn, int64_t ldk, const void* vn, int64_t ldv,
                             const float* rc, const float* rs, void* kc, void* vc, int64_t max_len, const int64_t* pos,
                             int b, int hkv, float scale, void* out, int64_t ldo, float* part, int64_t ks_min, int spt,
                             hipStream_t s) {
  const int64_t nsplit_max = (max_len + ks_min - 1) / ks_min;
  const int64_t nsplit = spt > 0 && spt < nsplit_max ? spt : nsplit_max;
  if (spt > 0)
    hipLaunchKernelGGL((gqa_decode_kernel<DT, D, G, 64, true>), dim3(hkv, b, nsplit), dim3(kAttnThreads), 0, s, q,
                       ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, hkv, scale, out, ldo, (int)ks_min, spt, part);
  else
    hipLaunchKernelGGL((gqa_decode_kernel<DT, D, G, 64>), dim3(hkv, b, nsplit), dim3(kAttnThreads), 0, s, q, ldq, kn,
                       ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, hkv, scale, out, ldo, (int)ks_min, 0, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t lds = (size_t)(2 * nsplit * G + G) * sizeof(float);  // nsplit * G <= kAttnMaxSplitHeads
  hipLaunchKernelGGL((gqa_combine_kernel<DT, D, G>), dim3(hkv, b), dim3(kAttnThreads), lds, s, part, pos, max_len,
                     hkv, (int)ks_min, spt, (int)nsplit, out, ldo);
  return hipGetLastError();
}

// Target of live workgroups for the split kernel: the split length grows with the position until a
// sequence's keys take at most ceil(kAttnLiveSplits / (b * hkv)) splits.
constexpr int kAttnLiveSplits = 768;

template <int DT, int D, int G>
hipError_t launch_attn_g(const void* q, int64_t ldq, const void* kn, int64_t ldk, const void* vn, int64_t ldv,
                         const float* rc, const float* rs, void* kc, void* vc, int64_t max_len, const int64_t* pos,
                         int b, int hkv, float scale, void* out, int64_t ldo, float* part, hipStream_t s) {
  // Split length: at least ks_min = 64 keys (doubled only while the combine's LDS staging of the split
  // weights would pass 32 KB).  When the batch's sequences x kv heads would otherwise hold more than
  // kAttnLiveSplits splits at max_len, the length grows with the position instead, so the live splits
  // stay near kAttnLiveSplits: short contexts get many small splits to fill the GPU, long ones fewer and
  // longer splits whose chunk loads overlap.  The grid and workspace depend on max_len only and the
  // kernels read the positions on the device, so a captured graph stays valid at every position.
  // Measured at the Llama-3-8B batch-8 shape (64 sequence-heads, 4096 slots, split + combine, eager):
  // 14.5 / 15.7 / 24.7 / 31.6 / 37.5 us at positions 700 / 1000 / 2047 / 3000 / 4095 against 14.3 /
  // 17.8 / 29.0 / 42.3 / 49.3 with fixed 64-key splits; targets of 384 / 512 / 1024 live splits were
  // slower somewhere in that range.  One split (no workspace pass) when a single split covers max_len
  // or no workspace is given.
  const int64_t ks = split_keys(max_len, G);
  const int64_t nsplit = (max_len + ks - 1) / ks;
  if (nsplit == 1 || part == nullptr) {
    constexpr int CH = DT == WFB_F32 ? 128 : 256;
    hipLaunchKernelGGL((gqa_decode_kernel<DT, D, G, CH>), dim3(hkv, b, 1), dim3(kAttnThreads), 0, s, q, ldq, kn, ldk,
                       vn, ldv, rc, rs, kc, vc, max_len, pos, hkv, scale, out, ldo, (int)(max_len + 1), 0,
                       (float*)nullptr);
    return hipGetLastError();
  }
  const int64_t seq_heads = (int64_t)b * hkv;
  const int64_t spt = (kAttnLiveSplits + seq_heads - 1) / seq_heads;
  const int dyn = spt < nsplit ? (int)spt : 0;
  return launch_attn_split<DT, D, G>(q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo,
                                     part, ks, dyn, s);
}

template <int DT, int D>
hipError_t launch_attn_d(int g, const void* q, int64_t ldq, const void* kn, int64_t ldk, const void* vn, int64_t ldv,
                         const float* rc, const float* rs, void* kc, void* vc, int64_t max_len, const int64_t* pos,
                         int b, int hkv, float scale, void* out, int64_t ldo, float* part, hipStream_t s) {
#define WFB_ATTN_G(GG) \
  case GG: return launch_attn_g<DT, D, GG>(q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, part, s)
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
                             float* part, hipStream_t s) {
  if (dt == WFB_F32 && d == 64)
    return launch_attn_d<WFB_F32, 64>(g, q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, part, s);
  if (dt == WFB_F32 && d == 128)
    return launch_attn_d<WFB_F32, 128>(g, q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, part, s);
  if (dt == WFB_BF16 && d == 64)
    return launch_attn_d<WFB_BF16, 64>(g, q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, part, s);
  if (dt == WFB_BF16 && d == 128)
    return launch_attn_d<WFB_BF16, 128>(g, q, ldq, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len, pos, b, hkv, scale, out, ldo, part, s);
  return hipErrorInvalidValue;
}

int64_t gqa_decode_workspace_floats(int64_t max_len, int g, int64_t batch, int64_t hkv, int d) {
  const int64_t ks = split_keys(max_len, g);
  const int64_t nsplit = (max_len + ks - 1) / ks;
  return nsplit == 1 ? 0 : batch * hkv * nsplit * g * (d + 2);
}

namespace {
constexpr int kScratchDevices = 256;
std::mutex g_scratch_mu;
float* g_scratch_dev[kScratchDevices];  // device address of `scratch` on each GPU, looked up once
}  // namespace

hipError_t gqa_decode_scratch(hipStream_t stream, float** ptr) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  int dev = cur;
  if (stream) {  // the scratch of the GPU the work runs on (the null stream is the current device's)
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) return e;
  }
  if (dev < 0 || dev >= kScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {  // first call on this device: its own copy's address, looked up with it current
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return e;
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *ptr = g_scratch_dev[dev];
  return hipSuccess;
}

}  // namespace wfb
