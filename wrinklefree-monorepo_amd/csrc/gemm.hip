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

// Prefill GEMM (large M): v_mfma_i32_32x32x32_i8, workgroup tile BM x BN computed by 4 waves in a
// WM x WN grid (wave tile TM x TN sub-tiles of 32 x 32), K advancing one I2_S block (128 weights) per
// step.
//  * A (int8 activations) streams through LDS, double buffered; rows are padded to 144 bytes so the
//    32 lanes reading one MFMA fragment (16 B each, row stride 144) hit distinct banks.
//  * W goes from global memory straight into registers: lane (j, g) of a 32-row weight sub-tile
//    loads the 16 packed bytes of chunk 2*kt + g of row j, which are the B operands of 4 MFMAs, one
//    per 2-bit field f; field f pairs with activation bytes [128*kt + 32f + 16g, +16) of each row.
//  * Codes become signed int8 with one v_perm_b32 byte lookup per dword.
//  * Workgroup ids are remapped so that the 8 XCDs each take a contiguous range of tiles (tiles in
//    one range share activation rows in that XCD's L2).
template <int BM, int BN, int WM, int WN, int KB = 1, int OCC = 1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC, 8))) void gemm_i2s_mfma32_kernel(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ A, int64_t lda, int M, int N, int C, int tiles_n,
    int ntiles, Epilogue ep) {
  static_assert(WM * WN == 4, "4 waves");
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  constexpr int PITCH = 128 * KB + 16;
  constexpr int AS = BM * KB / 32;  // 16-byte A segments per thread per K-step
  __shared__ __attribute__((aligned(16))) int8_t lds[2][BM * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int i = lane & 31, g = lane >> 5;

  // XCD-aware tile order: hardware hands consecutive workgroup ids to the 8 XCDs in turn.
  const int per = gridDim.x / 8;  // the grid is a multiple of 8
  const int b = blockIdx.x;
  const int t = (b % 8) * per + b / 8;
  if (t >= ntiles) return;  // padding workgroups (whole workgroup leaves before any barrier)
  const int m0 = (t / tiles_n) * BM, n0 = (t % tiles_n) * BN;

  const int KT = C / (2 * KB);  // K-steps of 128*KB weights (callers guarantee C % (2*KB) == 0)
  const uint32_t row_bytes = (uint32_t)C * 16;
  const buf_t wb = make_buf(W, (uint32_t)N * row_bytes);
  const buf_t ab = make_buf(A, (uint32_t)((int64_t)(M - 1) * lda + (int64_t)C * 64));

  // A staging: thread covers rows arow + (256/(8*KB))*s, 16-byte segment aseg of the step's 128*KB bytes
  constexpr int RPS = 256 / (8 * KB);  // rows covered per pass of the 256 threads
  v4i areg[AS];
  v4i breg[TN][KB];
  const int arow = tid / (8 * KB), aseg = (tid % (8 * KB)) * 16;
  auto load_a = [&](int kt) {
#pragma unroll
    for (int s = 0; s < AS; ++s)
      areg[s] = buf_load16(ab, (uint32_t)((int64_t)(m0 + arow + RPS * s) * lda) + 128 * KB * kt + aseg);
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int s = 0; s < AS; ++s) *reinterpret_cast<v4i*>(&lds[buf][(arow + RPS * s) * PITCH + aseg]) = areg[s];
  };
  auto load_b = [&](int kt) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = n0 + (wn * TN + tn) * 32 + i;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) breg[tn][kb] = buf_load16(wb, (uint32_t)n * row_bytes + (2 * (KB * kt + kb) + g) * 16);
    }
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[tm][tn][r] = 0;

  load_a(0);
  load_b(0);
  store_a(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    v4i bcur[TN][KB];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) bcur[tn][kb] = breg[tn][kb];
    if (kt + 1 < KT) {
      load_a(kt + 1);
      load_b(kt + 1);
    }
    const int8_t* la = &lds[cur][(wm * TM * 32 + i) * PITCH + 16 * g];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        v4i bf[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int e = 0; e < 4; ++e) bf[tn][e] = codes_to_i8(((uint32_t)bcur[tn][kb][e] >> (6 - 2 * f)) & 0x03030303u);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
          const v4i a = *reinterpret_cast<const v4i*>(la + tm * 32 * PITCH + 128 * kb + 32 * f);
#pragma unroll
          for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bf[tn], acc[tm][tn], 0, 0, 0);
        }
      }
    if (kt + 1 < KT) store_a(cur ^ 1);
    __syncthreads();
  }

  // 32x32 accumulator layout: lane (i, g), register r -> row 8*(r/4) + 4*g + r%4, column i.
  const float ws = epi_wscale(ep);
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int n = n0 + (wn * TN + tn) * 32 + i;
    if (n >= N) continue;
    const float bias = epi_bias(ep, n);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + (wm * TM + tm) * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m < M) epi_store(ep, ws, epi_ascale(ep, m), bias, m, n, acc[tm][tn][r]);
      }
  }
}

template <int BM, int BN, int WM, int WN, int KB = 1, int OCC = 1>
hipError_t launch_tile(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                       hipStream_t s) {
  const int tiles_n = (n + BN - 1) / BN, tiles_m = (m + BM - 1) / BM;
  const int nwg = tiles_n * tiles_m;
  const int grid = ((nwg + 7) / 8) * 8;
  hipLaunchKernelGGL((gemm_i2s_mfma32_kernel<BM, BN, WM, WN, KB, OCC>), dim3(grid), dim3(256), 0, s, W, A, lda, m,
                     n, C, tiles_n, nwg, e);
  return hipGetLastError();
}

// Prefill GEMM, pipelined: workgroup tile BM x BN, WM x WN waves (wave tile TM x TN sub-tiles of 32x32,
// v_mfma_i32_32x32x32_i8), K advancing one I2_S block (128 weights) per step.
//  * Both operands are staged through LDS, double buffered: A (int8, 128 B per row and step, rows
//    padded to 144 B) and W (packed, 32 B per row and step, rows padded to 48 B); both pitches keep
//    the 8 lanes of a 128-bit LDS read phase on distinct banks.
//  * Global loads run two steps ahead through two register stage sets (the K loop is unrolled by two
//    so every register index is static); a step's data is written to LDS one iteration after it was
//    requested, and one barrier per step orders the buffers.
//  * Lane (j, g) of a 32-row weight sub-tile reads the 16 packed bytes of chunk 2*kt + g of its row:
//    the B operands of 4 MFMAs, one per 2-bit field f, which pair with activation bytes
//    [32f + 16g, +16) of the step.  Codes become signed int8 with one v_perm_b32 per dword.
//  * Workgroup ids are remapped so that each XCD takes a contiguous range of tiles.
template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_i2s_pipe_kernel(const uint8_t* __restrict__ W,
                                                                     const int8_t* __restrict__ A, int64_t lda,
                                                                     int M, int N, int C, int tiles_n, int ntiles,
                                                                     Epilogue ep) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  constexpr int AP = 144, BP = 48;             // LDS row pitches
  constexpr int AS = BM * 8 / NT;              // 16-byte A segments per thread per step
  constexpr int BS = BN * 2 / NT;              // 16-byte W segments per thread per step
  static_assert(AS >= 1 && BS >= 1 && BM * 8 % NT == 0 && BN * 2 % NT == 0, "tile / thread mismatch");
  __shared__ __attribute__((aligned(16))) int8_t la[2][BM * AP];
  __shared__ __attribute__((aligned(16))) uint8_t lb[2][BN * BP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int i = lane & 31, g = lane >> 5;

  const int per = gridDim.x / 8;  // the grid is a multiple of 8
  const int t = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (t >= ntiles) return;
  const int m0 = (t / tiles_n) * BM, n0 = (t % tiles_n) * BN;

  const int KT = C / 2;
  const uint32_t row_bytes = (uint32_t)C * 16;
  const buf_t wb = make_buf(W, (uint32_t)N * row_bytes);
  const buf_t ab = make_buf(A, (uint32_t)((int64_t)(M - 1) * lda + (int64_t)C * 64));

  // per-thread global source / LDS destination of its segments
  const int arow = tid >> 3, aseg = (tid & 7) * 16;
  const int brow = tid >> 1, bseg = (tid & 1) * 16;
  uint32_t aoff[AS], boff[BS];
#pragma unroll
  for (int s = 0; s < AS; ++s) aoff[s] = (uint32_t)((int64_t)(m0 + arow + s * (NT / 8)) * lda) + aseg;
#pragma unroll
  for (int s = 0; s < BS; ++s) boff[s] = (uint32_t)(n0 + brow + s * (NT / 2)) * row_bytes + bseg;

  v4i ra0[AS], rb0[BS], ra1[AS], rb1[BS];
  auto gload = [&](v4i (&ra)[AS], v4i (&rb)[BS], int kt) {
#pragma unroll
    for (int s = 0; s < AS; ++s) ra[s] = buf_load16(ab, aoff[s] + 128 * kt);
#pragma unroll
    for (int s = 0; s < BS; ++s) rb[s] = buf_load16(wb, boff[s] + 32 * kt);
  };
  auto lstore = [&](const v4i (&ra)[AS], const v4i (&rb)[BS], int buf) {
#pragma unroll
    for (int s = 0; s < AS; ++s) *reinterpret_cast<v4i*>(&la[buf][(arow + s * (NT / 8)) * AP + aseg]) = ra[s];
#pragma unroll
    for (int s = 0; s < BS; ++s) *reinterpret_cast<v4i*>(&lb[buf][(brow + s * (NT / 2)) * BP + bseg]) = rb[s];
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[tm][tn][r] = 0;

  auto compute = [&](int buf) {
    const int8_t* pa = &la[buf][(wm * TM * 32 + i) * AP + 16 * g];
    const uint8_t* pb = &lb[buf][(wn * TN * 32 + i) * BP + 16 * g];
    v4i bp[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) bp[tn] = *reinterpret_cast<const v4i*>(pb + tn * 32 * BP);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      v4i bf[TN];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int e = 0; e < 4; ++e) bf[tn][e] = codes_to_i8(((uint32_t)bp[tn][e] >> (6 - 2 * f)) & 0x03030303u);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        const v4i a = *reinterpret_cast<const v4i*>(pa + tm * 32 * AP + 32 * f);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bf[tn], acc[tm][tn], 0, 0, 0);
      }
    }
  };

  // prologue: steps 0 and 1 in flight, step 0 in LDS
  gload(ra0, rb0, 0);
  if (KT > 1) gload(ra1, rb1, 1);
  lstore(ra0, rb0, 0);
  __syncthreads();
  for (int kt = 0; kt < KT; kt += 2) {
    // even step kt: compute buffer 0; registers 0 take step kt+2; registers 1 (step kt+1) -> buffer 1
    if (kt + 2 < KT) gload(ra0, rb0, kt + 2);
    compute(0);
    if (kt + 1 < KT) lstore(ra1, rb1, 1);
    __syncthreads();
    if (kt + 1 >= KT) break;
    // odd step kt+1: compute buffer 1; registers 1 take step kt+3; registers 0 (step kt+2) -> buffer 0
    if (kt + 3 < KT) gload(ra1, rb1, kt + 3);
    compute(1);
    if (kt + 2 < KT) lstore(ra0, rb0, 0);
    __syncthreads();
  }

  // 32x32 accumulator layout: lane (i, g), register r -> row 8*(r/4) + 4*g + r%4, column i.
  const float ws = epi_wscale(ep);
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int n = n0 + (wn * TN + tn) * 32 + i;
    if (n >= N) continue;
    const float bias = epi_bias(ep, n);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + (wm * TM + tm) * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m < M) epi_store(ep, ws, epi_ascale(ep, m), bias, m, n, acc[tm][tn][r]);
      }
  }
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_pipe(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                       hipStream_t s) {
  const int tiles_n = (n + BN - 1) / BN, tiles_m = (m + BM - 1) / BM;
  const int nwg = tiles_n * tiles_m;
  const int grid = ((nwg + 7) / 8) * 8;
  hipLaunchKernelGGL((gemm_i2s_pipe_kernel<BM, BN, WM, WN>), dim3(grid), dim3(64 * WM * WN), 0, s, W, A, lda, m,
                     n, C, tiles_n, nwg, e);
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
  return launch_tile<64, 256, 1, 4, 1, 3>(W, n, C, A, m, lda, e, s);
}

}  // namespace wfb
