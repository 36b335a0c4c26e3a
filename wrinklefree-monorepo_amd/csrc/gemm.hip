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

// Prefill GEMM (M > 64): v_mfma_i32_32x32x32_i8, workgroup tile BM x BN, four waves side by side in
// N (wave tile BM x BN/4 = TM x TN sub-tiles of 32 x 32), K advancing one I2_S block (128 weights)
// per step.
//  * Operands: weights are src0 and activations src1, so an accumulator tile is C^T: lane (i, g)
//    register r holds token row i and weight column 8*(r/4) + 4*g + r%4, and the epilogue writes 4
//    consecutive outputs of one token row per store.
//  * Weights go from global memory straight into registers (each wave owns its BN/4 columns): lane
//    (i, g) of a 32-column sub-tile loads the 16 packed bytes of chunk 2*kt + g of its weight row,
//    the src0 operands of 4 MFMAs, one per 2-bit field f, which pair with activation bytes
//    [128*kt + 32f + 16g, +16).  A field enters the MFMA as its raw code {0,1,2} (shift + AND per
//    dword); the +1 offset is removed at the end with each token's sum of activations, accumulated
//    while the activations are staged: acc = sum(code * a) - sum(a).
//  * Activations stream through LDS, double buffered (rows padded to 144 bytes so the 32 rows read
//    by one MFMA operand fall on distinct banks).
//  * Software pipeline: activation loads run three steps ahead and weight loads two steps ahead, in
//    two register sets each (the K loop is unrolled by two so every register index is static); a
//    step's activations are written to LDS one step before they are used; one barrier per step.
//    The MFMA operands of field f + 1 are read from LDS while field f is multiplied.
//  * Tile order: workgroup ids are remapped so that each XCD takes a contiguous range of tiles, and
//    tiles are numbered in groups of kGroupM tile rows (column-major inside a group), so the
//    workgroups resident on one XCD share activation rows and weight columns in its L2.
//  * EPI = 1: bf16 output without bias or accumulator copy (the prefill case), vector stores only;
//    EPI = 0: any output type, bias, accumulator copy.
constexpr int kGroupM = 8;

template <int BM, int BN, int OCC, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC, 8))) void gemm_i2s_tile_kernel(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ A, int64_t lda, int M, int N, int C, int tiles_m,
    int tiles_n, int ntiles, bool vec_out, Epilogue ep) {
  constexpr int WN = 4;
  constexpr int TM = BM / 32, TN = BN / WN / 32;
  constexpr int PITCH = 144;
  constexpr int AS = BM / 32;  // 16-byte activation segments per thread and step (8 threads per row)
  static_assert(TN >= 1 && BN % (32 * WN) == 0 && BM % 32 == 0, "tile shape");
  __shared__ __attribute__((aligned(16))) int8_t lds[2][BM * PITCH];
  __shared__ int rowsum[BM];
  const int tid = threadIdx.x, lane = tid & 63, wn = tid >> 6;
  const int i = lane & 31, g = lane >> 5;

  const int per = gridDim.x / 8;  // the grid is a multiple of 8
  const int t = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (t >= ntiles) return;
  const int gsz = kGroupM * tiles_n;
  const int grp = t / gsz, r = t - grp * gsz;
  const int gm = min(kGroupM, tiles_m - grp * kGroupM);
  const int m0 = (grp * kGroupM + r % gm) * BM, n0 = (r / gm) * BN;

  const int KT = C / 2;
  const uint32_t row_bytes = (uint32_t)C * 16;
  const uint32_t a_end = (uint32_t)((int64_t)(M - 1) * lda + (int64_t)C * 64), b_end = (uint32_t)N * row_bytes;
  const buf_t wb = make_buf(W, b_end);
  const buf_t ab = make_buf(A, a_end);
  // rows past the end of A or W are clamped to the last one (their results are never stored)
  const int arow = tid >> 3, aseg = (tid & 7) * 16;
  uint32_t aoff[AS], boff[TN];
#pragma unroll
  for (int s = 0; s < AS; ++s) aoff[s] = (uint32_t)((int64_t)min(m0 + arow + 32 * s, M - 1) * lda) + aseg;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) boff[tn] = (uint32_t)min(n0 + (wn * TN + tn) * 32 + i, N - 1) * row_bytes + g * 16;

  // Loads past the last step get an offset beyond the buffer: they return zeros without touching
  // memory, so every load in the loop is unconditional (a fixed count of loads in flight).
  v4i areg[2][AS], breg[2][TN];
  int sa[AS];
#pragma unroll
  for (int s = 0; s < AS; ++s) sa[s] = 0;
  auto load_a = [&](int p, int kt) {
#pragma unroll
    for (int s = 0; s < AS; ++s) areg[p][s] = buf_load16(ab, kt < KT ? aoff[s] + 128 * kt : a_end);
  };
  auto load_b = [&](int p, int kt) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) breg[p][tn] = buf_load16(wb, kt < KT ? boff[tn] + 32 * kt : b_end);
  };
  auto stage_a = [&](int p) {
#pragma unroll
    for (int s = 0; s < AS; ++s) {
#pragma unroll
      for (int e = 0; e < 4; ++e) sa[s] = __builtin_amdgcn_sdot4(areg[p][s][e], 0x01010101, sa[s], false);
      *reinterpret_cast<v4i*>(&lds[p][(arow + 32 * s) * PITCH + aseg]) = areg[p][s];
    }
  };

  v16i acc[TN][TM];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[tn][tm][q] = 0;

  auto compute = [&](int p) {
    const int8_t* la = &lds[p][i * PITCH + 16 * g];
    v4i af[2][TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) af[0][tm] = *reinterpret_cast<const v4i*>(la + tm * 32 * PITCH);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      if (f < 3) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
          af[(f + 1) & 1][tm] = *reinterpret_cast<const v4i*>(la + tm * 32 * PITCH + 32 * (f + 1));
      }
      __builtin_amdgcn_sched_barrier(0);
      v4i bf[TN];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int e = 0; e < 4; ++e) bf[tn][e] = (int)(((uint32_t)breg[p][tn][e] >> (6 - 2 * f)) & 0x03030303u);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tn][tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[tn], af[f & 1][tm], acc[tn][tm], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // A(j) lives in areg[j & 1] and lds[j & 1], B(j) in breg[j & 1].  Step kt: stage A(kt + 1), load
  // A(kt + 3), multiply step kt, load B(kt + 2), barrier.
  load_a(0, 0);
  load_b(0, 0);
  load_a(1, 1);
  load_b(1, 1);
  stage_a(0);
  load_a(0, 2);
  __syncthreads();
  const int KT2 = KT & ~1;
  for (int kb = 0; kb < KT2; kb += 2) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int kt = kb + p;
      if (kt + 1 < KT) stage_a(p ^ 1);
      load_a(p ^ 1, kt + 3);
      __builtin_amdgcn_sched_barrier(0);
      compute(p);
      load_b(p, kt + 2);
      __syncthreads();
    }
  }
  if (KT & 1) compute(0);  // last step (even index), staged in lds[0] by the previous step

  // the 8 threads of a row (consecutive lanes) hold partial sums of its 16-byte segments
#pragma unroll
  for (int s = 0; s < AS; ++s) {
    int v = sa[s];
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
    v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    if ((tid & 7) == 0) rowsum[arow + 32 * s] = v;
  }
  __syncthreads();

  const float ws = epi_wscale(ep);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int ml = tm * 32 + i;
    const int m = m0 + ml;
    if (m >= M) continue;
    const float as = epi_ascale(ep, m);
    const int rs = rowsum[ml];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + (wn * TN + tn) * 32 + 8 * q + 4 * g;
        if (n >= N) continue;
        const int32_t v[4] = {acc[tn][tm][4 * q] - rs, acc[tn][tm][4 * q + 1] - rs, acc[tn][tm][4 * q + 2] - rs,
                              acc[tn][tm][4 * q + 3] - rs};
        if constexpr (EPI == 1) {
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = __fmul_rn(__fmul_rn((float)v[e], ws), as);
          uint16_t* o = reinterpret_cast<uint16_t*>(ep.out) + (int64_t)m * ep.ldo + n;
          if (n + 3 < N) {
            const bf16x2_t lo = __builtin_convertvector((f32x2_t){y[0], y[1]}, bf16x2_t);
            const bf16x2_t hi = __builtin_convertvector((f32x2_t){y[2], y[3]}, bf16x2_t);
            *reinterpret_cast<uint2*>(o) =
                make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < N) o[e] = f32_to_bf16_rne(y[e]);
          }
        } else {
          epi_store4(ep, ws, as, m, n, v, vec_out && n + 3 < N, N);
        }
      }
  }
}

template <int BM, int BN, int OCC>
hipError_t launch_tile(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                       hipStream_t s) {
  const int tiles_n = (n + BN - 1) / BN, tiles_m = (m + BM - 1) / BM;
  const int nwg = tiles_n * tiles_m;
  const int grid = ((nwg + 7) / 8) * 8;
  const bool vec_out = e.ldo % 4 == 0 && (uintptr_t)e.out % 16 == 0 && (uintptr_t)e.acc_out % 16 == 0;
  const bool bf16_only = e.out && e.out_dtype == WFB_BF16 && !e.bias && !e.acc_out && vec_out;
  if (bf16_only)
    hipLaunchKernelGGL((gemm_i2s_tile_kernel<BM, BN, OCC, 1>), dim3(grid), dim3(256), 0, s, W, A, lda, m, n, C,
                       tiles_m, tiles_n, nwg, vec_out, e);
  else
    hipLaunchKernelGGL((gemm_i2s_tile_kernel<BM, BN, OCC, 0>), dim3(grid), dim3(256), 0, s, W, A, lda, m, n, C,
                       tiles_m, tiles_n, nwg, vec_out, e);
  return hipGetLastError();
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
  if (m <= 64) return launch_mt<4>(W, n, C, A, m, lda, e, s);
  return launch_tile<64, 256, 3>(W, n, C, A, m, lda, e, s);
}

}  // namespace wfb
