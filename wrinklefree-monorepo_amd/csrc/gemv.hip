// Decode GEMV for the I2_S ternary BitLinear (M <= 2 tokens): VALU sdot4, no MFMA.
//
// Replaces bitnet_vec_dot_i2_i8 / bitnet_gemv_cpu
// (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:325-808, SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:331-367):
//   acc[n] = sum_k code(W[n,k]) * a[k] - sum_k a[k] = sum_k w[n,k] * a[k].
//
// Work mapping (wave64).  A row of K weights is C = K/64 chunks of 16 packed bytes.  L lanes share
// a row ("row group" = 64/L rows per wave pass); lane s of a group owns chunks s, s+L, ..., s+L*(CPL-1).
// One 128-bit load per chunk per row, so each wave instruction reads 64/L rows x 16L contiguous bytes.
// The activations a lane needs for its chunks (4 fields x 16 bytes per chunk) are loaded once into
// registers and reused for every row group the wave visits.
//
// Inner product of one packed dword d (16 weights) with the 4 activation dwords it pairs with uses
// the fields in place instead of shifting each down:
//   bits 1:0 of every byte:  d & 0x03030303          -> code      (acc_a)
//   bits 3:2:                d & 0x0C0C0C0C          -> 4 * code  (acc_b)
//   bits 5:4:                d & 0x30303030          -> 16 * code (acc_c)
//   bits 7:6:                (d >> 2) & 0x30303030   -> 16 * code (acc_c)
// and acc = acc_a + acc_b / 4 + acc_c / 16 (all exact), then minus sum(a) of the lane's chunks.
// Row totals are reduced over the L lanes of a group with DPP (quad_perm, row_half_mirror,
// row_mirror) and, above 16 lanes, xor shuffles.
#include "wfb_common.h"

namespace wfb {

namespace {

template <int L>
__device__ __forceinline__ int group_sum(int v) {
  if constexpr (L >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
  if constexpr (L >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
  if constexpr (L >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  if constexpr (L >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false); // row_mirror
  if constexpr (L >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

template <int M, int L, int CPL>
__global__ __launch_bounds__(64) void gemv_i2s_kernel(const uint8_t* __restrict__ W, const int8_t* __restrict__ A,
                                                      int64_t lda, int N, int C, int n_groups, int rg,
                                                      Epilogue ep) {
  constexpr int RPG = 64 / L;
  const int lane = threadIdx.x;
  const int r_in = lane / L, s = lane % L;
  const int64_t row_bytes = (int64_t)C * 16;

  // Activations for this lane's chunks, all tokens: a[m][i][q] = a_m[128b + 32q + j0 .. +15].
  v4i a[M][CPL][4];
  int suma[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    suma[m] = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = s + L * i;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (c < C) {
          a[m][i][q] = *reinterpret_cast<const v4i*>(A + m * lda + 128 * (c >> 1) + 32 * q + 16 * (c & 1));
        } else {
          a[m][i][q] = v4i{0, 0, 0, 0};
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) suma[m] = __builtin_amdgcn_sdot4(a[m][i][q][t], 0x01010101, suma[m], false);

  const float ws = epi_wscale(ep);
  const int g0 = blockIdx.x * rg;

  v4i cur[CPL], nxt[CPL];
  auto load_group = [&](v4i (&w)[CPL], int g) {
    const int n = g * RPG + r_in;
    const bool row_ok = (g < n_groups) && (n < N);
    const uint8_t* wr = W + (int64_t)n * row_bytes;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = s + L * i;
      if (row_ok && c < C) w[i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wr + 16 * c));
      else w[i] = v4i{0, 0, 0, 0};
    }
  };

  load_group(cur, g0);
  for (int r = 0; r < rg; ++r) {
    const int g = g0 + r;
    if (g >= n_groups) break;
    if (r + 1 < rg) load_group(nxt, g + 1);
    const int n = g * RPG + r_in;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      int acc_a = 0, acc_b = 0, acc_c = 0;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int d = cur[i][t];
          acc_c = __builtin_amdgcn_sdot4((d >> 2) & 0x30303030, a[m][i][0][t], acc_c, false);
          acc_c = __builtin_amdgcn_sdot4(d & 0x30303030, a[m][i][1][t], acc_c, false);
          acc_b = __builtin_amdgcn_sdot4(d & 0x0C0C0C0C, a[m][i][2][t], acc_b, false);
          acc_a = __builtin_amdgcn_sdot4(d & 0x03030303, a[m][i][3][t], acc_a, false);
        }
      }
      int tot = acc_a + (acc_b >> 2) + (acc_c >> 4) - suma[m];
      tot = group_sum<L>(tot);
      if (s == 0 && n < N) epi_store(ep, ws, m, n, tot);
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) cur[i] = nxt[i];
  }
}

template <int M, int L, int CPL>
hipError_t launch_cfg(const uint8_t* W, int n, int C, const int8_t* A, int64_t lda, const Epilogue& e,
                      hipStream_t s) {
  constexpr int RPG = 64 / L;
  const int n_groups = (n + RPG - 1) / RPG;
  // Aim for >= 4 waves per CU on 256 CUs before a wave takes a second row group.
  int rg = n_groups / 2048;
  if (rg < 1) rg = 1;
  if (rg > 8) rg = 8;
  const int blocks = (n_groups + rg - 1) / rg;
  hipLaunchKernelGGL((gemv_i2s_kernel<M, L, CPL>), dim3(blocks), dim3(64), 0, s, W, A, lda, n, C, n_groups, rg, e);
  return hipGetLastError();
}

// Pick (L, CPL) with L * CPL >= C, at most 10 token-chunks of activations per lane (160 VGPRs),
// L as small as possible (more rows share each wave instruction's activation addresses).
template <int M>
hipError_t launch_m(const uint8_t* W, int n, int C, const int8_t* A, int64_t lda, const Epilogue& e, hipStream_t s) {
#define WFB_TRY(LL, CC) \
  if constexpr (M * (CC) <= 10) {                                   \
    if (C <= (LL) * (CC)) return launch_cfg<M, LL, CC>(W, n, C, A, lda, e, s); \
  }
  WFB_TRY(1, 4) WFB_TRY(1, 8)
  WFB_TRY(2, 4) WFB_TRY(2, 5) WFB_TRY(2, 8)
  WFB_TRY(4, 4) WFB_TRY(4, 5) WFB_TRY(4, 7) WFB_TRY(4, 8)
  WFB_TRY(8, 4) WFB_TRY(8, 5) WFB_TRY(8, 7) WFB_TRY(8, 8)
  WFB_TRY(16, 4) WFB_TRY(16, 5) WFB_TRY(16, 7) WFB_TRY(16, 8)
  WFB_TRY(32, 4) WFB_TRY(32, 5) WFB_TRY(32, 7) WFB_TRY(32, 8)
  WFB_TRY(64, 4) WFB_TRY(64, 5) WFB_TRY(64, 7) WFB_TRY(64, 8)
#undef WFB_TRY
  return hipErrorInvalidValue;  // K > 32768: callers route these to the MFMA kernel
}

}  // namespace

hipError_t launch_gemv_i2s(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                           hipStream_t s) {
  const int C = k / 64;
  if (m == 1) return launch_m<1>(W, n, C, A, lda, e, s);
  if (m == 2) return launch_m<2>(W, n, C, A, lda, e, s);
  return hipErrorInvalidValue;
}

}  // namespace wfb
