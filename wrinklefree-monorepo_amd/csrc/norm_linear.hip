// RMSNorm/SubLN + per-token int8 quantisation fused into the prologue of the batched-decode BitLinear
// (M <= 16 tokens, H <= 4096): y = rmsnorm(x) * gamma -> int8 codes + per-token scales -> ternary
// linear (optionally multi-segment, optionally + residual).  Bit-identical to wfb_rmsnorm_quant_i8
// followed by wfb_linear_i2s(_segmented / _residual) on the same inputs; one launch instead of two.
//
// Replaces, for decode, the pair SubLN.forward / RMSNorm.forward -> BitLinear.activation_quant ->
// BitLinear.forward (packages/training/src/wrinklefree/models/subln.py:42-59, 64-97,
// packages/training/src/wrinklefree/models/bitlinear.py:66-113) that the reference's fused QKV / MLP ops
// run per token (SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:150-231, 289-375).
//
// Work mapping.  A workgroup owns NT tiles of 16 output rows and splits K over its S waves exactly as
// the skinny batched-decode kernel does (v_mfma_i32_16x16x64_i8, fields masked in place into x1/x4/x16
// accumulators, partial tiles summed through LDS).  Differences:
//  * every wave first issues the weight loads of all its K-steps (up to PF of them), so their HBM
//    latency overlaps the prologue;
//  * prologue: wave w normalises and quantises token rows w, w + S, ... in the one summation order the
//    per-token quantiser uses for rows up to 4096 elements (lane l adds elements (l + 64 j) * 8 + e, j
//    ascending, e = 0..7, then a fixed xor butterfly), writes the codes to LDS (row stride K + 16
//    bytes, zero beyond H) and the token scale next to them;
//  * the activation fragments come from LDS instead of global memory (16 token rows 16 bytes apart
//    in bank space: conflict-free).
// The workgroup recomputes the quantisation of all M rows: M * H * (2 + 2) bytes of cache-resident
// reads per workgroup, against a separate launch per projection.  Measured on MI355X (cold weights): 6-23%
// faster than the two launches while the grid fits one workgroup per CU (q|k|v and o at the Llama-3-8B,
// BitNet-2B and SmolLM2 shapes); slower for wider outputs (gate|up of Llama-3-8B and BitNet-2B), where
// the registers of the prologue leave one workgroup per CU and the grid needs two rounds.
#include "quant_rows.h"

namespace wfb {

namespace {

constexpr int kNormLinMaxH = 4096;  // rows of the wave summation order

// 8 consecutive elements in their storage type: one 16-byte load (bf16) or two (fp32); zero-initialised
// when not loaded.
template <int DT>
struct Raw8 {
  v4i r[DT == WFB_F32 ? 2 : 1] = {};
};

template <int DT>
__device__ __forceinline__ Raw8<DT> load_raw8(const void* p, int e0) {
  Raw8<DT> v;
  const v4i* q = reinterpret_cast<const v4i*>(reinterpret_cast<const char*>(p) + (int64_t)e0 * (DT == WFB_F32 ? 4 : 2));
  v.r[0] = q[0];
  if constexpr (DT == WFB_F32) v.r[1] = q[1];
  return v;
}

// widen to fp32 exactly as load8 does
template <int DT>
__device__ __forceinline__ void widen8(const Raw8<DT>& v, float (&f)[kVec]) {
  if constexpr (DT == WFB_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = __int_as_float(v.r[0][e]);
      f[4 + e] = __int_as_float(v.r[1][e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t u = (uint32_t)v.r[0][e];
      f[2 * e] = __uint_as_float(u << 16);
      f[2 * e + 1] = __uint_as_float(u & 0xffff0000u);
    }
  }
}

template <int XT, int GT, int S, int NT, int PF>
__global__ __launch_bounds__(64 * S) void norm_linear_kernel(const void* __restrict__ x, int64_t ldx,
                                                             const void* __restrict__ gamma, float eps, int H,
                                                             const uint8_t* __restrict__ W, int M, int N, int C,
                                                             Epilogue ep) {
  static_assert(NT <= S, "one wave per row tile in the epilogue");
  extern __shared__ __attribute__((aligned(16))) int8_t aq[];  // [M][K + 16] codes
  __shared__ int red[S][NT][4][64];
  __shared__ float sas[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int K = C * 64, AST = K + 16;
  const uint32_t row_bytes = (uint32_t)C * 16;
  const uint32_t w_end = (uint32_t)N * row_bytes;
  const buf_t wb = make_buf(W, w_end);
  const int T = (C + 3) >> 2;
  const int tok0 = 4 * g;
  const bool tok_ok = nl < M;
  const int8_t* arow = aq + nl * AST;

  {
    const int n0 = blockIdx.x * 16 * NT;
    uint32_t woff[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) woff[nt] = (uint32_t)(n0 + nt * 16 + nl) * row_bytes + 16 * g;

    // 1. weights of this wave's first PF K-steps (t = w, w + S, ...)
    v4i wpre[PF][NT];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int t = w + p * S;
      const bool ok = t < T && 4 * t + g < C;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wpre[p][nt] = buf_load16(wb, ok ? woff[nt] + 64u * t : w_end);
    }
    // epilogue operands of the column this lane stores (waves w < NT); token scales from the prologue
    EpiCol<4> col;
    const int ncol = n0 + w * 16 + nl;
    if (w < NT) {
      int toks[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) toks[j] = tok0 + j;
      col.load(ep, ncol, N, toks, 0);  // M = 0: no token scales from memory
      if (ep.res) {
        bool ok[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ok[j] = tok0 + j < M && ncol < N;
        load_res_col<4>(ep, toks, ok, ncol, col.res);
      }
    }

    // 2. prologue: norm + quant of the M token rows into LDS.  The loaded rows and gamma stay in
    // registers in their storage type and are widened where used; y = (x * rs) * gamma is formed twice
    // (for the maximum, then for the codes) with the same operations, so both passes see the same values.
    for (int r = w; r < M; r += S) {
      const void* xr = reinterpret_cast<const char*>(x) + (int64_t)r * ldx * (XT == WFB_F32 ? 4 : 2);
      Raw8<XT> xv[8];
      Raw8<GT> gv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e0 = (lane + 64 * j) * kVec;
        xv[j] = e0 < H ? load_raw8<XT>(xr, e0) : Raw8<XT>{};
        gv[j] = (e0 < H && gamma) ? load_raw8<GT>(gamma, e0) : Raw8<GT>{};
      }
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float v[kVec];
        widen8<XT>(xv[j], v);
#pragma unroll
        for (int e = 0; e < kVec; ++e) ss = __fadd_rn(ss, __fmul_rn(v[e], v[e]));
      }
      ss = wave_sum_fixed(ss);
      const float rs = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(ss, (float)H), eps)));
      auto scaled = [&](int j, float rsc, float (&y)[kVec]) {
        float v[kVec], gm[kVec];
        widen8<XT>(xv[j], v);
        if (gamma && (lane + 64 * j) * kVec < H) {
          widen8<GT>(gv[j], gm);
        } else {
#pragma unroll
          for (int e = 0; e < kVec; ++e) gm[e] = 1.0f;
        }
#pragma unroll
        for (int e = 0; e < kVec; ++e) y[e] = __fmul_rn(__fmul_rn(v[e], rsc), gm[e]);
      };
      float mx = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float y[kVec];
        scaled(j, rs, y);
#pragma unroll
        for (int e = 0; e < kVec; ++e) mx = fmaxf(mx, fabsf(y[e]));
      }
      mx = wave_max(mx);
      if (mx < 1e-6f) mx = 1.0f;
      const float inv = __fdiv_rn(127.0f, mx);
      if (lane == 0) sas[r] = __fdiv_rn(mx, 127.0f);
      int8_t* qr = aq + r * AST;
      // the same rs, hidden from the optimiser so the products are recomputed rather than kept live
      float rs2 = rs;
      asm volatile("" : "+v"(rs2));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e0 = (lane + 64 * j) * kVec;
        if (e0 < K) {  // codes up to H, zeros up to K
          uint32_t lo = 0, hi = 0;
          if (e0 < H) {
            float y[kVec];
            scaled(j, rs2, y);
#pragma unroll
            for (int e = 0; e < 4; ++e) lo |= (uint32_t)(quant_i8(y[e], inv) & 0xff) << (8 * e);
#pragma unroll
            for (int e = 0; e < 4; ++e) hi |= (uint32_t)(quant_i8(y[4 + e], inv) & 0xff) << (8 * e);
          }
          *reinterpret_cast<uint2*>(qr + e0) = make_uint2(lo, hi);
        }
      }
    }
    __syncthreads();

    // 3. the batched-decode GEMV on the LDS activations
    v4i acc1[NT], acc4[NT], acc16[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc1[nt] = acc4[nt] = acc16[nt] = v4i{0, 0, 0, 0};
    int sa = 0;
    auto step = [&](int t, const v4i (&wv)[NT]) {
      const int c = 4 * t + g;
      const bool ok = c < C && tok_ok;
      const int ab0 = 128 * (c >> 1) + 16 * (c & 1);
      v4i av[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) av[f] = ok ? *reinterpret_cast<const v4i*>(arow + ab0 + 32 * f) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        v4i b0, b1, b2, b3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = wv[nt][e];
          b0[e] = (d >> 2) & 0x30303030;
          b1[e] = d & 0x30303030;
          b2[e] = d & 0x0C0C0C0C;
          b3[e] = d & 0x03030303;
        }
        acc16[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[0], b0, acc16[nt], 0, 0, 0);
        acc16[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[1], b1, acc16[nt], 0, 0, 0);
        acc4[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[2], b2, acc4[nt], 0, 0, 0);
        acc1[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[3], b3, acc1[nt], 0, 0, 0);
      }
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int e = 0; e < 4; ++e) sa = __builtin_amdgcn_sdot4(av[f][e], 0x01010101, sa, false);
    };
#pragma unroll
    for (int p = 0; p < PF; ++p)
      if (w + p * S < T) step(w + p * S, wpre[p]);
    for (int t = w + PF * S; t < T; t += S) {
      v4i wv[NT];
      const bool ok = 4 * t + g < C;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wv[nt] = buf_load16(wb, ok ? woff[nt] + 64u * t : w_end);
      step(t, wv);
    }

    // 4. partial tiles through LDS (C layout: lane (nl, g) holds tokens 4g + j of weight row nl)
    {
      int sm = sa;
      sm += __shfl_xor(sm, 16, 64);
      sm += __shfl_xor(sm, 32, 64);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int sj = __shfl(sm, 4 * g + j, 64);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          red[w][nt][j][lane] = acc1[nt][j] + (acc4[nt][j] >> 2) + (acc16[nt][j] >> 4) - sj;
      }
    }
    __syncthreads();
    if (w < NT && ncol < N) {
      const int nt = w;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = tok0 + j;
        if (tok >= M) continue;
        int tot = red[0][nt][j][lane];
#pragma unroll
        for (int k = 1; k < S; ++k) tot += red[k][nt][j][lane];
        epi_store_r(ep, col.ws, sas[tok], col.bias, col.res[j], tok, ncol, tot);
      }
    }
  }
}

template <int XT, int GT, int S, int NT>
hipError_t launch_nl(const void* x, int64_t ldx, const void* gamma, float eps, int h, const uint8_t* W, int m, int n,
                     int C, const Epilogue& e, hipStream_t s) {
  const size_t lds = (size_t)m * (C * 64 + 16);
  const int ntiles = (n + 16 * NT - 1) / (16 * NT);
  hipLaunchKernelGGL((norm_linear_kernel<XT, GT, S, NT, 16 / S>), dim3(ntiles), dim3(64 * S), lds, s, x, ldx, gamma, eps,
                     h, W, m, n, C, e);
  return hipGetLastError();
}

template <int XT, int GT>
hipError_t launch_nl_shape(const void* x, int64_t ldx, const void* gamma, float eps, int h, const uint8_t* W, int m,
                           int n, int C, const Epilogue& e, hipStream_t s) {
  // the batched-decode kernel's launch shapes (16-token tiles): 4 row tiles x 4 waves for N >= 24576,
  // 2 x 8 for N >= 6144 with K <= 8192, else one row tile x 8 waves (4 for short K)
  const int T = (C + 3) / 4;
  if (n >= 24576) return launch_nl<XT, GT, 4, 4>(x, ldx, gamma, eps, h, W, m, n, C, e, s);
  if (n >= 6144 && C <= 128) return launch_nl<XT, GT, 8, 2>(x, ldx, gamma, eps, h, W, m, n, C, e, s);
  if (T >= 8) return launch_nl<XT, GT, 8, 1>(x, ldx, gamma, eps, h, W, m, n, C, e, s);
  return launch_nl<XT, GT, 4, 1>(x, ldx, gamma, eps, h, W, m, n, C, e, s);
}

}  // namespace

int norm_linear_max_h() { return kNormLinMaxH; }

hipError_t launch_norm_linear(const void* x, int xdt, int64_t ldx, const void* gamma, int gdt, float eps, int h,
                              const uint8_t* W, int m, int n, int k, const Epilogue& e, hipStream_t s) {
  const int C = k / 64;
#define WFB_NL(XT, GT) return launch_nl_shape<XT, GT>(x, ldx, gamma, eps, h, W, m, n, C, e, s)
  if (xdt == WFB_BF16) {
    if (gdt == WFB_F32) WFB_NL(WFB_BF16, WFB_F32);
    WFB_NL(WFB_BF16, WFB_BF16);
  }
  if (gdt == WFB_F32) WFB_NL(WFB_F32, WFB_F32);
  WFB_NL(WFB_F32, WFB_BF16);
#undef WFB_NL
}

}  // namespace wfb
