// Causal GQA attention for a prefill chunk of T tokens per sequence (bf16 caches), with the rotary
// embedding of the new queries/keys and the cache append.
//
// Same contract as the decode kernel (attention_forward, SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:381-441,
// and kv_cache_update_key / _value, SGB/sgl-kernel/csrc/inference/kv_cache.h:81-101) for every query of the
// chunk: token i of sequence b sits at position start + i and attends over keys 0..start+i (causal), the
// rotary embedding in the HF rotate-half form of the stage-1 model
// (packages/training/src/wrinklefree/training/stage1.py:169-214), applied with the same fp32 operations as
// the torch formula and rounded to bf16.
//
// Two launches.  gqa_append_kernel ropes the T new keys and writes them and the values into the cache
// (bit-identical to the torch cache writes).  gqa_prefill_kernel then runs flash attention on the matrix
// cores: one workgroup per (16 query tokens, kv head, sequence), one wave per query head of the group, so
// each 64-key block of K and V is staged in LDS once for all heads of the group.  Per key block a wave
//   S^T[key, q] = K Q^T        v_mfma_f32_16x16x32_bf16, K rows from LDS (A), roped Q in registers (B)
//   online softmax per query   the 16 queries sit in lanes l % 16; a query's 64 keys in lanes l, l^16,
//                              l^32, l^48 (4 each per 16-key block), reduced with two xor shuffles
//   O^T[d, q] += V^T P^T       V staged transposed in LDS (A); P from the S^T registers of the same
//                              lane (B), split P = hi + lo (two bf16 products, ~16 mantissa bits)
// The reduction index k of an MFMA is a free labelling as long as A and B agree: S^T takes k = head
// dimension (32ks + 8(l/16) + j, 16 contiguous bytes of a row of K and of Q); O^T takes k = key, mapped to
// the keys the lane already holds from S^T (32c + 4(l/16) + j and 32c + 16 + 4(l/16) + j - 4).
// Scores and softmax are fp32; products of bf16 operands are exact in fp32 and summed in fp32.
#include "wfb_common.h"

namespace wfb {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

union Frag8 {
  bf16x8_t v;
  uint16_t h[8];
  uint32_t u[4];
  v4i q;
};

__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// y1 = x1 c + (-x2) s, y2 = x2 c + x1 s, each product and sum rounded to fp32, then to bf16
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, uint16_t& y1, uint16_t& y2) {
  y1 = f32_to_bf16_rne(__fadd_rn(__fmul_rn(x1, c), __fmul_rn(-x2, s)));
  y2 = f32_to_bf16_rne(__fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s)));
}

// One workgroup per (token i, sequence b): rotary of the token's kv heads' keys, cache writes of key
// and value at position start + i.
template <int D>
__global__ __launch_bounds__(256) void gqa_append_kernel(const uint16_t* __restrict__ kn, int64_t ldk,
                                                         const uint16_t* __restrict__ vn, int64_t ldv,
                                                         const float* __restrict__ rope_cos,
                                                         const float* __restrict__ rope_sin, uint16_t* __restrict__ kc,
                                                         uint16_t* __restrict__ vc, int64_t max_len, int hkv, int T,
                                                         int64_t start, bool vec) {
  constexpr int HD = D / 2;
  const int i = blockIdx.x, b = blockIdx.y;
  const int64_t pos = start + i;
  const int64_t row = (int64_t)b * T + i;
  if (vec) {  // 16-byte pieces: 8 rotary pairs of a key, or 8 value elements, per thread
    constexpr int KI = HD / 8, VI = D / 8;
    for (int e = threadIdx.x; e < hkv * (KI + VI); e += blockDim.x) {
      if (e < hkv * KI) {
        const int g = e / KI, j0 = 8 * (e % KI);
        const uint16_t* kr = kn + row * ldk + (int64_t)g * D;
        uint16_t* dst = kc + (((int64_t)b * hkv + g) * max_len + pos) * D;
        Frag8 x1, x2;
        x1.q = *reinterpret_cast<const v4i*>(kr + j0);
        x2.q = *reinterpret_cast<const v4i*>(kr + j0 + HD);
        if (rope_cos) {
          const float4* cp = reinterpret_cast<const float4*>(rope_cos + pos * HD + j0);
          const float4* sp = reinterpret_cast<const float4*>(rope_sin + pos * HD + j0);
          const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
          const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
          const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
          float y1[8], y2[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float a = bf16f(x1.h[j]), c = bf16f(x2.h[j]);
            y1[j] = __fadd_rn(__fmul_rn(a, cs[j]), __fmul_rn(-c, sn[j]));
            y2[j] = __fadd_rn(__fmul_rn(c, cs[j]), __fmul_rn(a, sn[j]));
          }
#pragma unroll
          for (int j = 0; j < 8; j += 2) {  // bf16, round to nearest even (v_cvt_pk_bf16_f32)
            x1.u[j / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){y1[j], y1[j + 1]}, bf16x2_t));
            x2.u[j / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){y2[j], y2[j + 1]}, bf16x2_t));
          }
        }
        *reinterpret_cast<v4i*>(dst + j0) = x1.q;
        *reinterpret_cast<v4i*>(dst + j0 + HD) = x2.q;
      } else {
        const int e2 = e - hkv * KI, g = e2 / VI, j0 = 8 * (e2 % VI);
        *reinterpret_cast<v4i*>(vc + (((int64_t)b * hkv + g) * max_len + pos) * D + j0) =
            *reinterpret_cast<const v4i*>(vn + row * ldv + (int64_t)g * D + j0);
      }
    }
    return;
  }
  for (int e = threadIdx.x; e < hkv * HD; e += blockDim.x) {
    const int g = e / HD, j = e % HD;
    const uint16_t* kr = kn + row * ldk + (int64_t)g * D;
    uint16_t* dst = kc + (((int64_t)b * hkv + g) * max_len + pos) * D;
    if (rope_cos) {
      uint16_t y1, y2;
      rope_pair(bf16f(kr[j]), bf16f(kr[j + HD]), rope_cos[pos * HD + j], rope_sin[pos * HD + j], y1, y2);
      dst[j] = y1;
      dst[j + HD] = y2;
    } else {
      dst[j] = kr[j];
      dst[j + HD] = kr[j + HD];
    }
  }
  for (int e = threadIdx.x; e < hkv * D; e += blockDim.x) {
    const int g = e / D, j = e % D;
    vc[(((int64_t)b * hkv + g) * max_len + pos) * D + j] = vn[row * ldv + (int64_t)g * D + j];
  }
}

// At D = 128 with 4 query heads per kv head (Llama-3-8B) the kernel is held to 3 waves per SIMD
// (158 registers, no spills; 29.1 -> 26.3 us at the Llama-3-8B prompt shape, where the compiler's own
// choice was 176 registers and 2 waves); the other shapes keep the compiler's choice.
template <int D, int G>
__global__ __launch_bounds__(64 * G) __attribute__((amdgpu_waves_per_eu(D == 128 && G == 4 ? 3 : 1))) void gqa_prefill_kernel(const uint16_t* __restrict__ q, int64_t ldq,
                                                             const float* __restrict__ rope_cos,
                                                             const float* __restrict__ rope_sin,
                                                             const uint16_t* __restrict__ kc,
                                                             const uint16_t* __restrict__ vc, int64_t max_len, int hkv,
                                                             int T, int64_t start, float scale,
                                                             uint16_t* __restrict__ out, int64_t ldo) {
  constexpr int KS = D / 32;       // MFMA k-steps over the head dimension
  constexpr int DB = D / 16;       // 16-row blocks of O^T
  constexpr int KB = 64;           // keys per block
  constexpr int KROW = D + 8;      // K tile row stride (elements): 16-byte aligned, rows 4 banks apart
  constexpr int VROW = KB + 4;     // V^T tile row stride (elements): rows 2 banks apart (+ 8-byte reads)
  constexpr int NT = 64 * G;
  __shared__ __attribute__((aligned(16))) uint16_t ks_[KB * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vs_[D * VROW];

  const int i0 = blockIdx.x * 16, g = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int h = g * G + w;
  const int grp = lane >> 4;
  const int qi = i0 + (lane & 15);  // this lane's query token (S^T / O^T column)
  const bool qvalid = qi < T;
  const int64_t qpos = start + qi;
  const int qpos32 = (int)qpos;                // positions < max_len < 2^23 (host-checked)
  const int qpos_first = (int)(start + i0);    // the workgroup's first query position

  // roped query fragments: lane holds Q[qi][32ks + 8grp .. +7] for each ks
  Frag8 qf[KS];
  {
    const uint16_t* qr = q + ((int64_t)b * T + (qvalid ? qi : 0)) * ldq + (int64_t)h * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s].q = *reinterpret_cast<const v4i*>(qr + 32 * s + 8 * grp);
    if (!qvalid) {
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[s].q = v4i{0, 0, 0, 0};
    } else if (rope_cos) {
      constexpr int HD = D / 2;
#pragma unroll
      for (int s = 0; s < KS / 2; ++s) {
        // elements d = 32s + 8grp + j (< D/2) and their partners d + D/2 (fragment s + KS/2, slot j);
        // the 8 table entries of d are contiguous (16-byte aligned tables, host-checked)
        const float4* cp = reinterpret_cast<const float4*>(rope_cos + qpos * HD + 32 * s + 8 * grp);
        const float4* sp = reinterpret_cast<const float4*>(rope_sin + qpos * HD + 32 * s + 8 * grp);
        const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
        const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        float y1[8], y2[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x1 = bf16f(qf[s].h[j]), x2 = bf16f(qf[s + KS / 2].h[j]);
          y1[j] = __fadd_rn(__fmul_rn(x1, cs[j]), __fmul_rn(-x2, sn[j]));
          y2[j] = __fadd_rn(__fmul_rn(x2, cs[j]), __fmul_rn(x1, sn[j]));
        }
#pragma unroll
        for (int j = 0; j < 8; j += 2) {  // round to bf16, nearest even (v_cvt_pk_bf16_f32)
          qf[s].u[j / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){y1[j], y1[j + 1]}, bf16x2_t));
          qf[s + KS / 2].u[j / 2] =
              __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){y2[j], y2[j + 1]}, bf16x2_t));
        }
      }
    }
  }

  // keys needed by the block's last valid query; loads past them read zeros (no stale cache rows enter
  // the P V product, where a masked p = 0 would still meet them)
  const int64_t kend = start + (i0 + 16 < T ? i0 + 16 : T);
  const int nkb = (int)((kend + KB - 1) / KB);
  const int64_t slice = ((int64_t)b * hkv + g) * max_len * D;  // element offset of the (b, g) cache slice
  const buf_t kb_ = make_buf(kc + slice, (uint32_t)(kend * D * 2));
  const buf_t vb_ = make_buf(vc + slice, (uint32_t)(kend * D * 2));

  f32x4_t o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -__builtin_inff(), l_run = 0.0f;

  // Tile staging, software-pipelined: the global loads of block kb + 1 are issued right after block kb
  // is written to LDS, so they are in flight while block kb is computed.  Trip counts are compile-time
  // constants, so every load of a tile is issued before the first LDS write waits for one.
  constexpr int KP = KB * (D / 8);        // 16-byte pieces of the K tile
  constexpr int KIT = (KP + NT - 1) / NT;
  constexpr int VP = (KB / 2) * (D / 8);  // (key pair, 8-element chunk) items of the V tile
  constexpr int VIT = (VP + NT - 1) / NT;
  v4i kreg[KIT];
  Frag8 va[VIT], vb2[VIT];
  auto load_tile = [&](int key0) {
#pragma unroll
    for (int it = 0; it < KIT; ++it) {
      const int p = t + it * NT;
      if (KP % NT == 0 || p < KP) {
        const int r = p / (D / 8), c = p % (D / 8);
        kreg[it] = buf_load16(kb_, (uint32_t)(((key0 + r) * D + 8 * c) * 2));
      }
    }
    // V: 16 consecutive lanes take 16 consecutive key pairs of one 8-element chunk, the next 16 lanes
    // the next chunk, so the transposed row stores below spread over all banks (rows 8c + j of chunks
    // c and c + 1 sit 16 banks apart) while each key row is still read as 64-byte pieces
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
      const int p = t + it * NT;
      if (VP % NT == 0 || p < VP) {
        const int rest = p / 16, c = rest % (D / 8);
        const int r = 2 * ((p % 16) + 16 * (rest / (D / 8)));
        va[it].q = buf_load16(vb_, (uint32_t)(((key0 + r) * D + 8 * c) * 2));
        vb2[it].q = buf_load16(vb_, (uint32_t)(((key0 + r + 1) * D + 8 * c) * 2));
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int it = 0; it < KIT; ++it) {
      const int p = t + it * NT;
      if (KP % NT == 0 || p < KP) {
        const int r = p / (D / 8), c = p % (D / 8);
        *reinterpret_cast<v4i*>(&ks_[r * KROW + 8 * c]) = kreg[it];
      }
    }
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
      const int p = t + it * NT;
      if (VP % NT == 0 || p < VP) {
        const int rest = p / 16, c = rest % (D / 8);
        const int r = 2 * ((p % 16) + 16 * (rest / (D / 8)));
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          *reinterpret_cast<uint32_t*>(&vs_[(8 * c + jj) * VROW + r]) =
              (uint32_t)va[it].h[jj] | ((uint32_t)vb2[it].h[jj] << 16);
      }
    }
  };

  load_tile(0);
  for (int kb = 0; kb < nkb; ++kb) {
    const int key0 = kb * KB;
    __syncthreads();  // the previous block's tiles are no longer read
    store_tile();
    __syncthreads();
    if (kb + 1 < nkb) load_tile(key0 + KB);

    // S^T = K Q^T for the 4 sub-blocks of 16 keys
    f32x4_t s[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      s[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        Frag8 a;
        a.q = *reinterpret_cast<const v4i*>(&ks_[(16 * nb + (lane & 15)) * KROW + 32 * k + 8 * grp]);
        s[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, qf[k].v, s[nb], 0, 0, 0);
      }
    }
    // scale, causal mask (only blocks reaching past the workgroup's first query), block max
    float bmax = -__builtin_inff();
    const bool masked = key0 + KB - 1 > qpos_first;  // uniform
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = key0 + 16 * nb + 4 * grp + i;
        const float v = !masked || key <= qpos32 ? s[nb][i] * scale : -__builtin_inff();
        s[nb][i] = v;
        bmax = fmaxf(bmax, v);
      }
    bmax = fmaxf(bmax, xor_lanes_f32<16>(bmax));
    bmax = fmaxf(bmax, xor_lanes_f32<32>(bmax));
    const float m_new = fmaxf(m_run, bmax);  // finite: key 0 <= qpos is in block 0
    const float alpha = __expf(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __expf(s[nb][i] - m_new);
        s[nb][i] = p;
        psum += p;
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] *= alpha;

    // O^T += V^T P^T over two chunks of 32 keys (slots j < 4: sub-block 2c, j >= 4: sub-block 2c + 1)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      Frag8 phi, plo;  // hi = bf16(p), lo = bf16(p - hi), both round-to-nearest-even (v_cvt_pk_bf16_f32)
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const float p0 = s[2 * c + (j >> 2)][j & 3], p1 = s[2 * c + (j >> 2)][(j & 3) + 1];
        const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){p0, p1}, bf16x2_t));
        const float r0 = p0 - __uint_as_float(hi << 16), r1 = p1 - __uint_as_float(hi & 0xffff0000u);
        phi.u[j / 2] = hi;
        plo.u[j / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){r0, r1}, bf16x2_t));
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint16_t* vr = &vs_[(16 * db + (lane & 15)) * VROW + 32 * c + 4 * grp];
        Frag8 a;
        const uint2 lo4 = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi4 = *reinterpret_cast<const uint2*>(vr + 16);
        a.u[0] = lo4.x;
        a.u[1] = lo4.y;
        a.u[2] = hi4.x;
        a.u[3] = hi4.y;
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, phi.v, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, plo.v, o[db], 0, 0, 0);
      }
    }
  }

  if (!qvalid) return;
  // lane holds O^T[16db + 4grp + i][qi]: four consecutive elements of the output row per db
  uint16_t* orow = out + ((int64_t)b * T + qi) * ldo + (int64_t)h * D;
  const float inv_l = 1.0f / l_run;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    uint2 v;
    v.x = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){o[db][0] * inv_l, o[db][1] * inv_l}, bf16x2_t));
    v.y = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){o[db][2] * inv_l, o[db][3] * inv_l}, bf16x2_t));
    *reinterpret_cast<uint2*>(orow + 16 * db + 4 * grp) = v;
  }
}

template <int D, int G>
hipError_t launch_prefill_g(const uint16_t* q, int64_t ldq, const float* rc, const float* rs, const uint16_t* kc,
                            const uint16_t* vc, int64_t max_len, int b, int hkv, int t, int64_t start, float scale,
                            uint16_t* out, int64_t ldo, hipStream_t s) {
  hipLaunchKernelGGL((gqa_prefill_kernel<D, G>), dim3((t + 15) / 16, hkv, b), dim3(64 * G), 0, s, q, ldq, rc, rs, kc,
                     vc, max_len, hkv, t, start, scale, out, ldo);
  return hipGetLastError();
}

template <int D>
hipError_t launch_prefill_d(int g, const uint16_t* q, int64_t ldq, const uint16_t* kn, int64_t ldk, const uint16_t* vn,
                            int64_t ldv, const float* rc, const float* rs, uint16_t* kc, uint16_t* vc, int64_t max_len,
                            int b, int hkv, int t, int64_t start, float scale, uint16_t* out, int64_t ldo,
                            hipStream_t s) {
  // 16-byte path when the key / value rows allow it (q|k|v column slices of one projection output do)
  const bool vec = (uintptr_t)kn % 16 == 0 && (uintptr_t)vn % 16 == 0 && ldk % 8 == 0 && ldv % 8 == 0;
  hipLaunchKernelGGL((gqa_append_kernel<D>), dim3(t, b), dim3(256), 0, s, kn, ldk, vn, ldv, rc, rs, kc, vc, max_len,
                     hkv, t, start, vec);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
#define WFB_PF_G(GG) \
  case GG: return launch_prefill_g<D, GG>(q, ldq, rc, rs, kc, vc, max_len, b, hkv, t, start, scale, out, ldo, s)
  switch (g) {
    WFB_PF_G(1);
    WFB_PF_G(2);
    WFB_PF_G(3);
    WFB_PF_G(4);
    WFB_PF_G(5);
    WFB_PF_G(6);
    WFB_PF_G(7);
    WFB_PF_G(8);
    default: return hipErrorInvalidValue;
  }
#undef WFB_PF_G
}

}  // namespace

hipError_t launch_gqa_prefill(int d, int g, const void* q, int64_t ldq, const void* kn, int64_t ldk, const void* vn,
                              int64_t ldv, const float* rc, const float* rs, void* kc, void* vc, int64_t max_len, int b,
                              int hkv, int t, int64_t start, float scale, void* out, int64_t ldo, hipStream_t s) {
  auto u16 = [](const void* p) { return reinterpret_cast<const uint16_t*>(p); };
  auto w16 = [](void* p) { return reinterpret_cast<uint16_t*>(p); };
  if (d == 64)
    return launch_prefill_d<64>(g, u16(q), ldq, u16(kn), ldk, u16(vn), ldv, rc, rs, w16(kc), w16(vc), max_len, b, hkv,
                                t, start, scale, w16(out), ldo, s);
  if (d == 128)
    return launch_prefill_d<128>(g, u16(q), ldq, u16(kn), ldk, u16(vn), ldv, rc, rs, w16(kc), w16(vc), max_len, b, hkv,
                                 t, start, scale, w16(out), ldo, s);
  return hipErrorInvalidValue;
}

}  // namespace wfb
