// Shared device helpers and internal launcher declarations of libwfbitnet (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/wfbitnet.h"

namespace wfb {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---- scalar conversions -------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t v) {
  return (float)__builtin_bit_cast(_Float16, v);
}

// fp32 -> bf16 with round-to-nearest-even (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (DT == WFB_F32) {
    return reinterpret_cast<const float*>(p)[i];
  } else if constexpr (DT == WFB_BF16) {
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  } else {
    return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  }
}

// Load 8 consecutive elements starting at element index i (16-byte aligned for 16-bit types,
// 32-byte for fp32) and widen them to fp32.
template <int DT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float (&v)[8]) {
  if constexpr (DT == WFB_F32) {
    const float4* q = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
    float4 a = q[0], b = q[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + i);
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (DT == WFB_BF16) {
        v[2 * e] = __uint_as_float(w[e] << 16);
        v[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
      } else {
        v[2 * e] = f16_bits_to_f32((uint16_t)(w[e] & 0xffffu));
        v[2 * e + 1] = f16_bits_to_f32((uint16_t)(w[e] >> 16));
      }
    }
  }
}

// ---- lane-group reductions ------------------------------------------------------------------

// The value of lane (lane ^ O) -- what __shfl_xor(v, O, 64) returns -- by VALU lane moves instead of the
// LDS permute (whose latency sits on every reduction's critical path): gfx950's v_permlane32_swap /
// v_permlane16_swap for O = 32 / 16, DPP row_ror:8, row_shl:4 / row_shr:4 and quad permutes below; all
// 64 lanes must be active.  Checked against __shfl_xor for every lane and offset on MI355X.
template <int O>
__device__ __forceinline__ int xor_lanes(int v) {
  const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  if constexpr (O == 32) {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // p[0]: halves swapped up, p[1]: down
    return lane < 32 ? (int)p[1] : (int)p[0];
  } else if constexpr (O == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? (int)p[0] : (int)p[1];
  } else if constexpr (O == 8) {
    return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (O == 4) {
    const int up = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0xF, false);  // row_shl:4: lane + 4
    const int dn = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4: lane - 4
    return (lane & 4) ? dn : up;
  } else if constexpr (O == 2) {
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
  } else {
    static_assert(O == 1, "O is a power of two below 64");
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
  }
}
template <int O>
__device__ __forceinline__ float xor_lanes_f32(float v) {
  return __int_as_float(xor_lanes<O>(__float_as_int(v)));
}

// Sum over aligned groups of L consecutive lanes (L = 2..64, a power of two); every lane of a group
// ends with the group total.  DPP quad_perm / row_half_mirror / row_mirror below 32 lanes.
template <int L>
__device__ __forceinline__ int group_sum(int v) {
  if constexpr (L >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
  if constexpr (L >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
  if constexpr (L >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  if constexpr (L >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false); // row_mirror
  if constexpr (L >= 32) v += xor_lanes<16>(v);
  if constexpr (L >= 64) v += xor_lanes<32>(v);
  return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int L>
__device__ __forceinline__ float group_sum_f32(float v) {
  if constexpr (L >= 2) v += dpp_f32<0xB1>(v);
  if constexpr (L >= 4) v += dpp_f32<0x4E>(v);
  if constexpr (L >= 8) v += dpp_f32<0x141>(v);
  if constexpr (L >= 16) v += dpp_f32<0x140>(v);
  if constexpr (L >= 32) v += xor_lanes_f32<16>(v);
  if constexpr (L >= 64) v += xor_lanes_f32<32>(v);
  return v;
}

// Round half to even, then saturate to int8 (the vector path of the reference quantiser:
// _mm256_round_ps(NEAREST_INT) + saturating packs).
__device__ __forceinline__ int quant_i8(float v, float inv) {
  float r = __builtin_rintf(__fmul_rn(v, inv));
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  return (int)r;
}

// Four codes quant_i8(v[e], inv), e = 0..3, packed little-endian into one word.  Clamping first and
// rounding after gives the same integer for every finite input (a value clamped to +-127/-128 is already
// integral; one inside rounds as before), and NaN clamps to -128 as in quant_i8.  The rounding adds
// 1.5 * 2^23: below 2^22 in magnitude the sum is rounded to an integer, half to even, and its low byte is
// that integer's two's-complement byte; v_perm_b32 then gathers the four low bytes.
__device__ __forceinline__ uint32_t quant4_i8(const float* v, float inv) {
  uint32_t b[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float c = fminf(fmaxf(__fmul_rn(v[e], inv), -128.0f), 127.0f);
    b[e] = __float_as_uint(__fadd_rn(c, 12582912.0f));
  }
  const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u);  // bytes: b0.0, b1.0, 0, 0
  const uint32_t hi = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);  // bytes: b2.0, b3.0, 0, 0
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);                   // lo.0, lo.1, hi.0, hi.1
}

// ---- raw buffer access (out-of-range reads return 0) --------------------------------------

typedef __amdgpu_buffer_rsrc_t buf_t;
constexpr int kBufDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)
constexpr int kLoadNT = 2;              // non-temporal: streamed once, do not keep in cache

__device__ __forceinline__ buf_t make_buf(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufDword3);
}
template <int AUX = 0>
__device__ __forceinline__ v4i buf_load16(buf_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX);
}

// ---- GEMV / GEMM epilogue -------------------------------------------------------------------

struct Epilogue {
  const float* a_scale;  // [M] or null
  const float* ws_dev;   // [nseg] or null
  float ws;              // used when ws_dev is null
  const void* bias;      // [N] or null
  int bias_dtype;
  void* out;             // [M, N] or null
  int out_dtype;
  int64_t ldo;
  int32_t* acc_out;      // [M, N] or null
  // Output rows (weight rows) split in nseg consecutive segments, each with its own weight scale
  // ws_dev[s]; segment s ends at row seg_end[s] (s < nseg - 1).  nseg = 1: one per-tensor scale.
  int nseg;
  int seg_end[WFB_MAX_SEGMENTS - 1];
  // Greedy-argmax epilogue (GEMV and skinny kernels only): when set, workgroup b writes, for each
  // token m, the largest argmax key of its rows to amax[b * ld + m], ld = amax_ld or, if that is 0, M
  // (see amax_key); the value compared is y rounded to amax_dt (WFB_F32 or WFB_BF16), i.e. the logit as
  // stored.  (A launch over a chunk of the tokens sets amax_ld to the full count and offsets amax.)
  uint64_t* amax;
  int amax_dt;
  int amax_ld;
  // Residual added to every output before it is stored (y = ... + res[m, n]), or null.
  const void* res;
  int res_dtype;
  int64_t ldr;
  // Gated (gate|up) epilogue only: the type the two products are rounded to before the activation.
  int mid_dtype;
};

__device__ __forceinline__ float epi_res(const Epilogue& e, int m, int n) {
  const int64_t off = (int64_t)m * e.ldr + n;
  if (e.res_dtype == WFB_F32) return reinterpret_cast<const float*>(e.res)[off];
  return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(e.res)[off]);
}

// Gated activations (GLU = 1: silu(g) * u, GLU = 2: relu(g)^2 * u).  Every step is one correctly
// rounded fp32 operation (no FMA), so a float32 CPU restatement reproduces the result bit for bit.
// 2^t = 2^n * p(t - n), n = rint(t) with t clamped to [-125, 125] (2^n stays a normal number),
// p the degree-7 Taylor polynomial of 2^f = exp(f ln 2) on |f| <= 1/2 (remainder < 6e-9).
__device__ __forceinline__ float exp2_fixed(float t) {
  t = fminf(fmaxf(t, -125.0f), 125.0f);
  const float n = rintf(t);
  const float f = __fsub_rn(t, n);
  float p = 1.525273380405984e-05f;  // ln(2)^7 / 7!
  p = __fadd_rn(__fmul_rn(p, f), 1.5403530393381606e-04f);
  p = __fadd_rn(__fmul_rn(p, f), 1.3333558146428443e-03f);
  p = __fadd_rn(__fmul_rn(p, f), 9.618129107628477e-03f);
  p = __fadd_rn(__fmul_rn(p, f), 5.550410866482158e-02f);
  p = __fadd_rn(__fmul_rn(p, f), 2.402265069591007e-01f);
  p = __fadd_rn(__fmul_rn(p, f), 6.931471805599453e-01f);
  p = __fadd_rn(__fmul_rn(p, f), 1.0f);
  return __fmul_rn(p, __int_as_float(((int)n + 127) << 23));
}

template <int GLU>
__device__ __forceinline__ float glu(float g, float u) {
  if constexpr (GLU == 1) {
    const float e = exp2_fixed(__fmul_rn(-g, 1.4426950408889634f));  // exp(-g)
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
  } else {
    const float r = fmaxf(g, 0.0f);
    return __fmul_rn(__fmul_rn(r, r), u);
  }
}

// Orderable 64-bit key of (value y, row n): larger y wins, and among equal values the smaller row
// (the first maximum, as std::max_element and torch.argmax pick).  Never 0 for n < 2^32 - 1.
__device__ __forceinline__ uint64_t amax_key(float y, int n) {
  const uint32_t u = __float_as_uint(y);
  const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)n);
}

template <int O>
__device__ __forceinline__ uint64_t xor_lanes_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)xor_lanes<O>((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)xor_lanes<O>((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
template <int O>
__device__ __forceinline__ uint64_t max_xor_u64(uint64_t v) {
  const uint64_t x = xor_lanes_u64<O>(v);
  return x > v ? x : v;
}

// max over aligned groups of L lanes (xor butterfly by lane moves; all 64 lanes active); every lane of a
// group ends with the maximum
template <int L>
__device__ __forceinline__ uint64_t group_max_u64(uint64_t v) {
  if constexpr (L > 1) v = max_xor_u64<1>(v);
  if constexpr (L > 2) v = max_xor_u64<2>(v);
  if constexpr (L > 4) v = max_xor_u64<4>(v);
  if constexpr (L > 8) v = max_xor_u64<8>(v);
  if constexpr (L > 16) v = max_xor_u64<16>(v);
  if constexpr (L > 32) v = max_xor_u64<32>(v);
  return v;
}

// Weight scale of output column n (segment lookup without branches).
__device__ __forceinline__ float epi_wscale(const Epilogue& e, int n) {
  if (!e.ws_dev) return e.ws;
  int s = 0;
#pragma unroll
  for (int j = 0; j < WFB_MAX_SEGMENTS - 1; ++j) s += (j + 1 < e.nseg && n >= e.seg_end[j]) ? 1 : 0;
  return e.ws_dev[s];
}
__device__ __forceinline__ float epi_ascale(const Epilogue& e, int m) { return e.a_scale ? e.a_scale[m] : 1.0f; }
__device__ __forceinline__ float epi_bias(const Epilogue& e, int n) {
  if (!e.bias) return 0.0f;
  if (e.bias_dtype == WFB_F32) return reinterpret_cast<const float*>(e.bias)[n];
  if (e.bias_dtype == WFB_BF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(e.bias)[n]);
  return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(e.bias)[n]);
}

// y = ((float)acc * ws) * as (+ bias): the two products in this order, each rounded to fp32
// (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:846 then SGB/python/sglang/srt/layers/quantization/bitnet.py:241).
// ws, as and bias are loaded by the caller (ahead of the main loop, to keep them off the critical path).
__device__ __forceinline__ float epi_y(const Epilogue& e, float ws, float as, float bias, int32_t acc) {
  float y = __fmul_rn(__fmul_rn((float)acc, ws), as);
  if (e.bias) y = __fadd_rn(y, bias);
  return y;
}

// Store of output (m, n) with the residual value res (used when e.res is set) already loaded.
__device__ __forceinline__ void epi_store_r(const Epilogue& e, float ws, float as, float bias, float res, int m,
                                            int n, int32_t acc) {
  const int64_t off = (int64_t)m * e.ldo + n;
  if (e.acc_out) e.acc_out[off] = acc;
  if (!e.out) return;
  float y = epi_y(e, ws, as, bias, acc);
  if (e.res) y = __fadd_rn(y, res);
  if (e.out_dtype == WFB_F32) reinterpret_cast<float*>(e.out)[off] = y;
  else reinterpret_cast<uint16_t*>(e.out)[off] = f32_to_bf16_rne(y);
}

__device__ __forceinline__ void epi_store(const Epilogue& e, float ws, float as, float bias, int m, int n,
                                          int32_t acc) {
  const int64_t off = (int64_t)m * e.ldo + n;
  if (e.acc_out) e.acc_out[off] = acc;
  if (!e.out) return;
  float y = epi_y(e, ws, as, bias, acc);
  if (e.res) y = __fadd_rn(y, epi_res(e, m, n));
  if (e.out_dtype == WFB_F32) reinterpret_cast<float*>(e.out)[off] = y;
  else reinterpret_cast<uint16_t*>(e.out)[off] = f32_to_bf16_rne(y);
}

// Argmax key of output (m, n) (store included); 0 when (m, n) is out of range.
__device__ __forceinline__ uint64_t epi_store_key_r(const Epilogue& e, float ws, float as, float bias, float res,
                                                    int m, int n, int32_t acc, bool valid) {
  if (!valid) return 0;
  epi_store_r(e, ws, as, bias, res, m, n, acc);
  float y = epi_y(e, ws, as, bias, acc);
  if (e.res) y = __fadd_rn(y, res);
  if (e.amax_dt == WFB_BF16) y = bf16_bits_to_f32(f32_to_bf16_rne(y));
  return amax_key(y, n);
}

__device__ __forceinline__ uint64_t epi_store_key(const Epilogue& e, float ws, float as, float bias, int m, int n,
                                                  int32_t acc, bool valid) {
  if (!valid) return 0;
  epi_store(e, ws, as, bias, m, n, acc);
  float y = epi_y(e, ws, as, bias, acc);
  if (e.res) y = __fadd_rn(y, epi_res(e, m, n));
  if (e.amax_dt == WFB_BF16) y = bf16_bits_to_f32(f32_to_bf16_rne(y));
  return amax_key(y, n);
}

// Epilogue operands of output column n for T tokens tok[j] (weight scale, bias, token scales and
// residuals), loaded at kernel entry so their latency overlaps the weight stream instead of following
// the final reduction (a kernel's first touch of them misses the cache).  Entries of tokens >= M or of
// n >= N are not loaded.
// Residuals res[tok[j], n] of the tokens with ok[j] (0 for the others).  Every load is issued before
// the first wait: entries not wanted load element 0 (in bounds whenever a residual is given) and are
// zeroed afterwards, so no branch encloses a load (a test and a conversion per element made each load
// wait for the previous one).
template <int T>
__device__ __forceinline__ void load_res_col(const Epilogue& e, const int (&tok)[T], const bool (&ok)[T], int n,
                                             float (&res)[T]) {
  if (e.res_dtype == WFB_F32) {
    const float* r = reinterpret_cast<const float*>(e.res);
    float v[T];
#pragma unroll
    for (int j = 0; j < T; ++j) v[j] = r[ok[j] ? (int64_t)tok[j] * e.ldr + n : 0];
#pragma unroll
    for (int j = 0; j < T; ++j) res[j] = ok[j] ? v[j] : 0.0f;
  } else {
    const uint16_t* r = reinterpret_cast<const uint16_t*>(e.res);
    uint16_t v[T];
#pragma unroll
    for (int j = 0; j < T; ++j) v[j] = r[ok[j] ? (int64_t)tok[j] * e.ldr + n : 0];
#pragma unroll
    for (int j = 0; j < T; ++j) res[j] = ok[j] ? bf16_bits_to_f32(v[j]) : 0.0f;
  }
}

template <int T>
struct EpiCol {
  float ws = 0.0f, bias = 0.0f;
  float as[T], res[T];
  __device__ __forceinline__ void load(const Epilogue& e, int n, int N, const int (&tok)[T], int M) {
#pragma unroll
    for (int j = 0; j < T; ++j) as[j] = res[j] = 0.0f;
    if (n >= N) return;
    ws = epi_wscale(e, n);
    bias = epi_bias(e, n);
#pragma unroll
    for (int j = 0; j < T; ++j)
      if (tok[j] < M) as[j] = epi_ascale(e, tok[j]);
    if (e.res) {
      bool ok[T];
#pragma unroll
      for (int j = 0; j < T; ++j) ok[j] = tok[j] < M;
      load_res_col<T>(e, tok, ok, n, res);
    }
  }
  // load() with the bias and the residuals kept as the bits loaded, converted by finish() at the
  // epilogue: a conversion right after a load inside a dtype branch makes the wave wait for every load
  // in flight at that point (the weight stream included, in the GEMV's storing wave)
  uint32_t braw = 0, rraw[T], okm = 0;
  __device__ __forceinline__ void load_raw(const Epilogue& e, int n, int N, const int (&tok)[T], int M) {
#pragma unroll
    for (int j = 0; j < T; ++j) as[j] = res[j] = 0.0f, rraw[j] = 0;
    if (n >= N) return;
    ws = epi_wscale(e, n);
    if (e.bias) {
      if (e.bias_dtype == WFB_F32) braw = reinterpret_cast<const uint32_t*>(e.bias)[n];
      else braw = reinterpret_cast<const uint16_t*>(e.bias)[n];
    }
#pragma unroll
    for (int j = 0; j < T; ++j)
      if (tok[j] < M) as[j] = epi_ascale(e, tok[j]);
    if (e.res) {
      // every load issued before the first use; entries not wanted load element 0 (in bounds whenever a
      // residual is given) and are zeroed by finish()
#pragma unroll
      for (int j = 0; j < T; ++j) {
        const int64_t off = tok[j] < M ? (int64_t)tok[j] * e.ldr + n : 0;
        if (e.res_dtype == WFB_F32) rraw[j] = reinterpret_cast<const uint32_t*>(e.res)[off];
        else rraw[j] = reinterpret_cast<const uint16_t*>(e.res)[off];
        okm |= tok[j] < M ? 1u << j : 0u;
      }
    }
  }
  __device__ __forceinline__ void finish(const Epilogue& e) {
    if (e.bias)
      bias = e.bias_dtype == WFB_F32    ? __uint_as_float(braw)
             : e.bias_dtype == WFB_BF16 ? bf16_bits_to_f32((uint16_t)braw)
                                        : f16_bits_to_f32((uint16_t)braw);
#pragma unroll
    for (int j = 0; j < T; ++j) {
      const float v = e.res_dtype == WFB_F32 ? __uint_as_float(rraw[j]) : bf16_bits_to_f32((uint16_t)rraw[j]);
      res[j] = (okm >> j) & 1u ? v : 0.0f;
    }
  }
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Four consecutive outputs of one token row: y[m, n..n+3] from int32 accumulators v[0..3].
// Same arithmetic as epi_store; bf16 conversion by v_cvt_pk_bf16_f32 (round to nearest even).
// vec: the 4 outputs are in range and their address is 4-element aligned (one wide store).
__device__ __forceinline__ void epi_store4(const Epilogue& e, float ws, float as, int m, int n, const int32_t (&v)[4],
                                           bool vec, int N) {
  const int64_t off = (int64_t)m * e.ldo + n;
  if (e.acc_out) {
    if (vec) {
      *reinterpret_cast<v4i*>(e.acc_out + off) = v4i{v[0], v[1], v[2], v[3]};
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (n + j < N) e.acc_out[off + j] = v[j];
    }
  }
  if (!e.out) return;
  float y[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    y[j] = __fmul_rn(__fmul_rn((float)v[j], ws), as);
    if (e.bias && n + j < N) y[j] = __fadd_rn(y[j], epi_bias(e, n + j));
    if (e.res && n + j < N) y[j] = __fadd_rn(y[j], epi_res(e, m, n + j));
  }
  if (e.out_dtype == WFB_F32) {
    float* o = reinterpret_cast<float*>(e.out) + off;
    if (vec) {
      *reinterpret_cast<float4*>(o) = make_float4(y[0], y[1], y[2], y[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (n + j < N) o[j] = y[j];
    }
  } else {
    uint16_t* o = reinterpret_cast<uint16_t*>(e.out) + off;
    if (vec) {
      const bf16x2_t lo = __builtin_convertvector((f32x2_t){y[0], y[1]}, bf16x2_t);
      const bf16x2_t hi = __builtin_convertvector((f32x2_t){y[2], y[3]}, bf16x2_t);
      *reinterpret_cast<uint2*>(o) = make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (n + j < N) o[j] = f32_to_bf16_rne(y[j]);
    }
  }
}

// ---- internal launchers (return hipError_t of the launch) --------------------------------

hipError_t launch_weight_absmean(const void* w, int dt, int64_t numel, float* scale, double* ws, hipStream_t s);
hipError_t launch_pack_i2s(const void* w, int dt, int64_t n, int64_t k, int64_t ldw, const float* scale,
                           uint8_t* qw, hipStream_t s);
hipError_t launch_unpack_i2s(const uint8_t* qw, int64_t n, int64_t k, int8_t* out, hipStream_t s);
hipError_t launch_quant_rows(const void* x, int dt, int64_t ldx, const void* gamma, int gdt, bool norm,
                             float eps, int64_t m, int64_t h, int8_t* q, int64_t k_pad, int64_t ldq,
                             float* a_scale, hipStream_t s);
hipError_t launch_glu_quant_rows(const void* gate, const void* up, int dt, int64_t ldx, int act, const void* gamma,
                                 int gdt, float eps, int64_t m, int64_t h, int8_t* q, int64_t k_pad, int64_t ldq,
                                 float* a_scale, hipStream_t s);
hipError_t launch_quant_tensor(const void* x, int dt, int64_t numel, int8_t* q, float* a_scale, hipStream_t s);
hipError_t launch_gemv_i2s(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda,
                           const Epilogue& e, hipStream_t s);
// Scratch of wfb_gqa_decode_attention_noalloc: 8 Mi floats (32 MiB) per GPU.
constexpr int64_t kAttnScratchFloats = int64_t(8) << 20;
static_assert(kAttnScratchFloats == WFB_ATTN_SCRATCH_FLOATS, "scratch size stated in the header");
// floats of split partials launch_gqa_decode uses for these sizes (0: one split, no workspace pass)
int64_t gqa_decode_workspace_floats(int64_t max_len, int g, int64_t batch, int64_t hkv, int d);
// device address of the scratch array on the stream's GPU (looked up on the first call per device)
hipError_t gqa_decode_scratch(hipStream_t stream, float** ptr);
hipError_t launch_gqa_decode(int dt, int d, int g, const void* q, int64_t ldq, const void* kn, int64_t ldk,
                             const void* vn, int64_t ldv, const float* rc, const float* rs, void* kc, void* vc,
                             int64_t max_len, const int64_t* pos, int b, int hkv, float scale, void* out, int64_t ldo,
                             float* part, hipStream_t s);
hipError_t launch_gqa_prefill(int d, int g, const void* q, int64_t ldq, const void* kn, int64_t ldk, const void* vn,
                              int64_t ldv, const float* rc, const float* rs, void* kc, void* vc, int64_t max_len, int b,
                              int hkv, int t, int64_t start, float scale, void* out, int64_t ldo, hipStream_t s);
hipError_t launch_convert_hf_offline(const uint8_t* src, int64_t nb, int64_t n, int64_t k, int64_t k_pad,
                                     const void* ws_dev, int ws_dt, float ws_host, int mode, uint8_t* qw,
                                     float* scale_out, int64_t* parts, hipStream_t s);
hipError_t launch_argmax_finalize(const uint64_t* parts, int64_t n_parts, int64_t m, int64_t* tokens, hipStream_t s);
hipError_t launch_lm_head_argmax(const void* x, int xdt, int64_t ldx, const void* gamma, int gdt, float eps,
                                 const void* w, int wdt, int64_t ldw, int64_t m, int64_t n, int64_t h, float* logits,
                                 int64_t ldo, uint64_t* parts, hipStream_t s);
// Activation rows that the batched-decode kernel normalises and quantises itself (its RMSNorm prologue):
// x [M, H] (x_dtype WFB_F32 / WFB_BF16, row stride ldx elements, rows 16-byte aligned), gamma [H]
// (gdt WFB_F32 / WFB_BF16, 16-byte aligned) or null, H % 8 == 0, H <= K <= 4096.  x == null: the
// activations are int8 codes A with per-token scales ep.a_scale, as for wfb_linear_i2s.
struct NormSrc {
  const void* x;
  int xdt;
  int64_t ldx;
  const void* gamma;
  int gdt;
  float eps;
  int h;
};
// One token (m == 1) whose RMSNorm/SubLN + quantisation runs in the decode GEMV's prologue (codes in
// LDS, the quantiser's 256-thread order): 4096 < H <= K <= 16384, rows 16-byte aligned; ep.a_scale unused.
// hipErrorNotSupported for other sizes.
hipError_t launch_gemv_i2s_norm(const uint8_t* W, int n, int k, int m, const Epilogue& e, const NormSrc& ns,
                                hipStream_t s);
// One token, norm prologue + gate|up + act(gate) * up into fp32 out (e.out, e.ldo, e.mid_dtype, two
// weight-scale segments), K <= 4096, n % 64 == 0; act WFB_ACT_SILU or WFB_ACT_RELU2.
hipError_t launch_gemv_i2s_norm_glu(const uint8_t* W, int n, int k, const Epilogue& e, const NormSrc& ns, int act,
                                    hipStream_t s);
// M <= 32 tokens (16 with the norm prologue) with both operands staged in LDS (skinny_lds.h); act 0 (plain) or a WFB_ACT_* gated
// gate|up product; returns hipErrorNotSupported when the shape does not fit its LDS (the caller then
// takes the register-operand kernels).  Needs N*K/4 and (M-1)*lda + K below 2^31.
hipError_t launch_skinny_lds_mr4(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                 const Epilogue& e, int act, int nt_pref, const NormSrc& ns, hipStream_t s);
hipError_t launch_skinny_lds_mr8(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                 const Epilogue& e, int act, int nt_pref, const NormSrc& ns, hipStream_t s);
hipError_t launch_skinny_lds_mr16(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                  const Epilogue& e, int act, int nt_pref, const NormSrc& ns, hipStream_t s);
// 17..32 tokens as two 16-token tiles (33..64 as two token blocks of such workgroups, one grid row each),
// 33..64 as four (no norm prologue; the four-tile form plain only)
hipError_t launch_skinny_lds_mr32(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                  const Epilogue& e, int act, int nt_pref, const NormSrc& ns, hipStream_t s);
hipError_t launch_skinny_lds_mr64(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                  const Epilogue& e, int act, int nt_pref, const NormSrc& ns, hipStream_t s);
inline hipError_t launch_skinny_lds(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda,
                                    const Epilogue& e, int act, hipStream_t s, const NormSrc& ns = NormSrc{}) {
  const int C = k / 64;
  // 16-row tiles per workgroup, from sweeps on MI355X (rows n counts gate + up rows when gated):
  //  * n >= 24576 (28672 gate|up, 128256 LM head): 4 for M <= 4, whose staging lets two such
  //    workgroups share a CU, else 8 (one workgroup per CU either way, so fewer, larger ones);
  //  * n >= 8192: 4; gated 2 up to M = 8 (13824 gate|up: 432 workgroups, all resident);
  //  * shorter outputs: 1 (2 when gated, one gate and one up tile).
  int nt_pref = n >= 24576 ? (m <= 4 ? 4 : 8) : n >= 8192 ? (act && m <= 8 ? 2 : 4) : act ? 2 : 1;
  // with the norm prologue every workgroup repeats the M x H normalisation, so the grid is kept to one
  // round of at most 256 workgroups (one per CU)
  if (ns.x) {
    const int tiles = (n + 15) / 16;
    nt_pref = tiles <= 256 ? 1 : tiles <= 512 ? 2 : tiles <= 1024 ? 4 : 8;
    if (act && nt_pref < 2) nt_pref = 2;
  }
  if (m < 1) return hipErrorInvalidValue;
  if (m <= 4) return launch_skinny_lds_mr4(W, n, C, A, m, lda, e, act, nt_pref, ns, s);
  if (m <= 8) return launch_skinny_lds_mr8(W, n, C, A, m, lda, e, act, nt_pref, ns, s);
  if (m <= 16) return launch_skinny_lds_mr16(W, n, C, A, m, lda, e, act, nt_pref, ns, s);
  // 17..32 tokens: two token tiles per weight fragment where the staging of 32 activation rows still
  // leaves room for a full grid -- rows up to 2560 on outputs up to 32768 rows (gate|up rows when
  // gated), rows up to 4096 on outputs of one round (4096 rows).  Measured on MI355X against the
  // split-K and 32-row tile kernels at M = 17 / 24 / 32: 13824 x 2560 12.7 -> 7.3-7.7 us, 2560 x 2560
  // 5.1-6.4 -> 4.4, gated 13824 x 2560 8.9-11.8 -> 8.1-9.0, 4096 x 4096 6.3-8.0 -> 5.5-5.8; with 4096-long
  // rows on taller outputs (6144 x 4096: 7.4 -> 9.4 at M = 17, 28672 x 4096: 17.4 -> 29.8) and rows
  // held in registers (2560 x 6912) it is slower or even, and those keep the other kernels.
  if (m <= 32 && !ns.x && ((k <= 2560 && n <= 32768) || (k <= 7168 && n <= 4096)))
    return launch_skinny_lds_mr32(W, n, C, A, m, lda, e, act, nt_pref, ns, s);
  // 33..64 tokens: four token tiles, one row tile per workgroup, activations staged one step at a time
  // (rows up to 2560) or held in registers (up to 4096) -- ahead only on narrow outputs (M = 64:
  // 2560 x 2560 10.1 -> 6.4 us, 3200 x 2560 10.2 -> 6.5, 4096 x 4096 13.5 -> 12.5; 13824 x 2560 12.9 ->
  // 23.2 and 6144 x 4096 15.7 -> 23.3 keep the 32-row tile kernel)
  if (m > 32 && m <= 64 && !ns.x && k <= 4096 && n <= 4096) {
    // rows of 4096 (the four-tile form holds their activations in registers): the two-tile form over two
    // token blocks of one launch instead, measured on MI355X (4096 x 4096: M = 40 10.2 -> 9.4 us, M = 64
    // 11.8 -> 10.0; on 2560-long rows it is slower, 6.2 -> 7.7 us at 2560 x 2560)
    if (k == 4096 && !e.amax) {
      const hipError_t st = launch_skinny_lds_mr32(W, n, C, A, m, lda, e, act, 1, ns, s);
      if (st != hipErrorNotSupported) return st;
    }
    return launch_skinny_lds_mr64(W, n, C, A, m, lda, e, act, 1, ns, s);
  }
  return hipErrorNotSupported;
}
// Rows from which a greedy head of more than 16 tokens runs in chunks of 16 (the persistent form's rows).
constexpr int kHeadChunkMinRows = 32768;
// 3 <= M <= 64 through the split-K skinny kernel (16, 32 or 64 rows per workgroup); needs
// N*K/4 and (M-1)*lda + K below 2^31
hipError_t launch_gemm_i2s_skinny(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda,
                                  const Epilogue& e, hipStream_t s);
hipError_t launch_gemm_i2s(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda,
                           const Epilogue& e, hipStream_t s);
// gate|up linear with the gated activation in its epilogue (M <= 64; n = 2 * half, half % 32 == 0;
// fp32 output [M, half] at e.out / e.ldo)
hipError_t launch_gemm_i2s_glu(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda, int act,
                               const Epilogue& e, hipStream_t s);

}  // namespace wfb
