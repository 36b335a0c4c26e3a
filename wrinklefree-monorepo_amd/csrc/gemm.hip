// int8-MFMA GEMM for the I2_S ternary BitLinear: Y[M, N] = A[M, K] (int8) x W[N, K]^T (ternary).
//
// Replaces bitnet_gemm_i2_i8 / bitnet_gemm_cpu (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:814-874,
// SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:370-406), which runs M*N independent I2_S dots.
//
// MFMA v_mfma_i32_16x16x64_i8 (gfx950).  Each lane of a wave supplies 16 bytes of A (one token row,
// one k-group) and 16 bytes of B (one weight row, the same k-group); the instruction pairs A and B
// bytes of the same (k-group, byte) slot, so any consistent assignment of k to slots is valid.
// Slot assignment used here: lane group g = lane / 16 at K-step t takes weight chunk c = 4t + g
// (16 packed bytes = 64 weights of the lane's row).  One 128-bit load gives the B operands of four
// MFMAs, one per 2-bit field f: field f of chunk c covers k = 128*(c/2) + 32f + 16*(c%2) + 0..15, so
// the matching A operand is the 16 contiguous activation bytes at that k.
// Codes {0,1,2} are turned into signed int8 {-1,0,+1} with one v_perm_b32 byte lookup per dword.
#include "wfb_common.h"

namespace wfb {

namespace {

// byte-wise code -> weight: 0 -> 0xFF (-1), 1 -> 0x00, 2 -> 0x01
__device__ __forceinline__ int codes_to_i8(uint32_t x) { return (int)__builtin_amdgcn_perm(0u, 0x000100FFu, x); }

template <int MT, int WPB>
__global__ __launch_bounds__(64 * WPB) void gemm_i2s_mfma16_kernel(const uint8_t* __restrict__ W,
                                                                   const int8_t* __restrict__ A, int64_t lda,
                                                                   int M, int N, int C, Epilogue ep) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * WPB + wave) * 16;
  if (n0 >= N) return;
  const int m0 = blockIdx.y * 16 * MT;
  const int nl = lane & 15, g = lane >> 4;
  const int n = n0 + nl;
  const int64_t row_bytes = (int64_t)C * 16;
  const uint8_t* wr = W + (int64_t)(n < N ? n : N - 1) * row_bytes;
  const int8_t* ar[MT];
  bool tok_ok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int tok = m0 + mt * 16 + nl;
    tok_ok[mt] = tok < M;
    ar[mt] = A + (int64_t)(tok < M ? tok : M - 1) * lda;
  }

  v4i acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};

  const int T = (C + 3) >> 2;
  for (int t = 0; t < T; ++t) {
    const int c = 4 * t + g;
    const bool c_ok = c < C;
    const v4i wv = c_ok ? *reinterpret_cast<const v4i*>(wr + 16 * c) : v4i{0, 0, 0, 0};
    v4i b[4];
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int e = 0; e < 4; ++e) b[f][e] = codes_to_i8(((uint32_t)wv[e] >> (6 - 2 * f)) & 0x03030303u);
    const int aoff = 128 * (c >> 1) + 16 * (c & 1);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const v4i av = (c_ok && tok_ok[mt]) ? *reinterpret_cast<const v4i*>(ar[mt] + aoff + 32 * f) : v4i{0, 0, 0, 0};
        acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[f], acc[mt], 0, 0, 0);
      }
    }
  }

  // C layout of a 16x16 MFMA tile: lane holds rows 4*(lane/16) + j (tokens), column lane % 16 (weight row).
  const float ws = epi_wscale(ep);
  if (n < N) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = m0 + mt * 16 + 4 * g + j;
        if (tok < M) epi_store(ep, ws, epi_ascale(ep, tok), epi_bias(ep, n), tok, n, acc[mt][j]);
      }
  }
}

// Skinny GEMM for M <= 16 tokens (decode batches): one 16-row weight tile per workgroup, K split
// over the S waves of the workgroup (SPW K-steps of 256 weights each), partial tiles summed in LDS.
// Fields enter the MFMA masked but not shifted -- bits 1:0 (x1), 3:2 (x4), 5:4 and 7:6>>2 (x16) --
// into three accumulators, so a packed dword costs 4 AND + 1 shift; the code offset (+1) is removed
// with sum(a) per token: acc = acc1 + acc4/4 + acc16/16 - sum(a).
template <int SPW, int S>
__global__ __launch_bounds__(64 * S) void gemv_mfma16_kernel(const uint8_t* __restrict__ W,
                                                             const int8_t* __restrict__ A, int64_t lda, int M,
                                                             int N, int C, Epilogue ep) {
  __shared__ int red[S][4][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16;
  const int nl = lane & 15, g = lane >> 4;
  const int n = n0 + nl;
  const int64_t row_bytes = (int64_t)C * 16;
  const uint8_t* wr = W + (int64_t)(n < N ? n : N - 1) * row_bytes;
  const bool tok_ok = nl < M;
  const int8_t* ar = A + (int64_t)(tok_ok ? nl : 0) * lda;
  const int t0 = w * SPW;

  // issue every load first
  v4i wv[SPW];
  v4i av[SPW][4];
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    const int c = 4 * (t0 + i) + g;
    const bool ok = c < C;
    wv[i] = ok ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wr + 16 * c)) : v4i{0, 0, 0, 0};
    const int aoff = 128 * (c >> 1) + 16 * (c & 1);
#pragma unroll
    for (int f = 0; f < 4; ++f)
      av[i][f] = (ok && tok_ok) ? *reinterpret_cast<const v4i*>(ar + aoff + 32 * f) : v4i{0, 0, 0, 0};
  }

  v4i acc1 = {0, 0, 0, 0}, acc4 = {0, 0, 0, 0}, acc16 = {0, 0, 0, 0};
  int sa = 0;
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    v4i b0, b1, b2, b3;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = wv[i][e];
      b0[e] = (d >> 2) & 0x30303030;
      b1[e] = d & 0x30303030;
      b2[e] = d & 0x0C0C0C0C;
      b3[e] = d & 0x03030303;
    }
    acc16 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][0], b0, acc16, 0, 0, 0);
    acc16 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][1], b1, acc16, 0, 0, 0);
    acc4 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][2], b2, acc4, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][3], b3, acc1, 0, 0, 0);
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int e = 0; e < 4; ++e) sa = __builtin_amdgcn_sdot4(av[i][f][e], 0x01010101, sa, false);
  }
  // sum(a) of token nl over this wave's K range: add the 4 lane groups
  sa += __shfl_xor(sa, 16, 64);
  sa += __shfl_xor(sa, 32, 64);
  // this lane holds tokens 4g + j of column nl
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int saj = __shfl(sa, 4 * g + j, 64);
    red[w][j][lane] = acc1[j] + (acc4[j] >> 2) + (acc16[j] >> 4) - saj;
  }
  __syncthreads();
  if (w != 0) return;
  const float ws = epi_wscale(ep);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tok = 4 * g + j;
    int tot = red[0][j][lane];
#pragma unroll
    for (int k = 1; k < S; ++k) tot += red[k][j][lane];
    if (tok < M && n < N) epi_store(ep, ws, epi_ascale(ep, tok), epi_bias(ep, n), tok, n, tot);
  }
}

template <int MT>
hipError_t launch_mt(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                     hipStream_t s) {
  constexpr int WPB = 4;
  const int ntiles = (n + 15) / 16;
  dim3 grid((ntiles + WPB - 1) / WPB, (m + 16 * MT - 1) / (16 * MT));
  hipLaunchKernelGGL((gemm_i2s_mfma16_kernel<MT, WPB>), grid, dim3(64 * WPB), 0, s, W, A, lda, m, n, C, e);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_i2s(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                           hipStream_t s) {
  const int C = k / 64;
  if (m <= 16) return launch_mt<1>(W, n, C, A, m, lda, e, s);
  if (m <= 32) return launch_mt<2>(W, n, C, A, m, lda, e, s);
  return launch_mt<4>(W, n, C, A, m, lda, e, s);
}

}  // namespace wfb
