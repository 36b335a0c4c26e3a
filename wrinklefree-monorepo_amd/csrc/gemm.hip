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
#include <algorithm>

#include "wfb_common.h"

namespace wfb {

namespace {

// byte-wise code -> weight: 0 -> 0xFF (-1), 1 -> 0x00, 2 -> 0x01
__device__ __forceinline__ int codes_to_i8(uint32_t x) { return (int)__builtin_amdgcn_perm(0u, 0x000100FFu, x); }

// Wave-per-16-rows batched kernel (whole K per wave, tokens split over grid.y): kept for the M <= 64
// shapes where the split-K skinny kernel below re-reads too many activation rows (large N at M > 8) or
// where offsets exceed 32 bits.
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
  const float ws = epi_wscale(ep, n);
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

// Batched decode (3 <= M <= 64 tokens): v_mfma_i32_16x16x64_i8 over MT tiles of 16 tokens.  A
// workgroup owns NT tiles of 16 weight rows and splits K over its S waves: wave w takes the
// 256-weight K-steps w, w + S, w + 2S, ..., so the waves of a workgroup read adjacent 64-byte chunks
// of the same rows.  Lane (nl, g) loads 16 packed bytes of row n0 + 16*nt + nl, chunk 4t + g (64
// weights; field f covers k = 128*(c/2) + 32f + 16*(c%2) + 0..15), the B operands of four MFMAs; the
// activation fragments of a step are loaded once and shared by the NT row tiles.  Fields enter masked
// but not shifted -- bits 1:0 (x1), 3:2 (x4), 5:4 and (7:6 >> 2) (x16) -- into three accumulators (5
// VALU per packed dword); the code offset is removed with each token's sum(a): acc = acc1 + acc4/4 +
// acc16/16 - sum(a).  Partial 16 x 16 tiles of the S waves are summed through LDS; wave nt < NT
// finishes row tile nt.  Loads go through raw buffer descriptors: rows past N or M and chunks past K
// read as zeros.
// Gated mode (GLUE = 1: SiLU, 2: relu^2): W is gate|up (N = 2 * half rows, two segments of scales); a
// workgroup takes gate row tiles 0 .. NT/2 - 1 and the up row tiles of the same rows, and wave nt <
// NT/2 stores x[m, n] = act(gate) * up for its 16 columns: both products rescaled as a plain linear
// would store them (rounded to ep.mid_dtype), then the fixed-operation gated activation, stored fp32.
template <int MT, int S, int NT, int GLUE = 0>
__global__ __launch_bounds__(64 * S) void gemm_i2s_skinny_kernel(const uint8_t* __restrict__ W,
                                                                 const int8_t* __restrict__ A, int64_t lda,
                                                                 int M, int N, int C, Epilogue ep) {
  static_assert(NT <= S, "one wave per row tile in the epilogue");
  static_assert(GLUE == 0 || NT % 2 == 0, "gated mode pairs gate and up tiles");
  __shared__ int red[S][NT][MT][4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int half = N / 2;
  const int n0 = GLUE ? blockIdx.x * 16 * (NT / 2) : blockIdx.x * 16 * NT;
  const int nl = lane & 15, g = lane >> 4;
  const uint32_t row_bytes = (uint32_t)C * 16;
  const uint32_t w_end = (uint32_t)N * row_bytes, a_end = (uint32_t)((int64_t)(M - 1) * lda + (int64_t)C * 64);
  const buf_t wb = make_buf(W, w_end);
  const buf_t ab = make_buf(A, a_end);
  uint32_t woff[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r0 = !GLUE ? n0 + nt * 16 : nt < NT / 2 ? n0 + nt * 16 : half + n0 + (nt - NT / 2) * 16;
    woff[nt] = (uint32_t)(r0 + nl) * row_bytes + 16 * g;
  }
  uint32_t aoff[MT];
  bool tok_ok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    tok_ok[mt] = mt * 16 + nl < M;
    aoff[mt] = (uint32_t)((int64_t)(mt * 16 + nl) * lda);
  }

  // Epilogue operands of the column this lane stores (waves w < NT; tokens 16 mt + 4 g + j), loaded
  // here, ahead of the weight stream -- measured on MI355X: 5-10% faster at M = 8..64 on 4096-row
  // outputs -- except with four row tiles (N >= 24576), where loading them after the final barrier is
  // 3% faster (fewer registers).
  constexpr bool PRE = NT < 4 && GLUE == 0;
  int toks[4 * MT];
#pragma unroll
  for (int j = 0; j < 4 * MT; ++j) toks[j] = (j / 4) * 16 + 4 * g + (j % 4);
  EpiCol<4 * MT> col;
  if (PRE && w < NT) col.load(ep, n0 + w * 16 + nl, N, toks, M);

  v4i acc1[NT][MT], acc4[NT][MT], acc16[NT][MT];
  int sa[MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc1[nt][mt] = acc4[nt][mt] = acc16[nt][mt] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = 0;
  const int T = (C + 3) >> 2;
  // operands of step t: the weight chunk of each row tile and the activation fragments (steps past T read
  // zeros from out-of-range offsets)
  auto load_step = [&](int t, v4i (&wv)[NT], v4i (&av)[MT][4]) {
    const int c = 4 * t + g;
    const bool ok = t < T && c < C;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wv[nt] = buf_load16(wb, ok ? woff[nt] + 64u * t : w_end);
    const uint32_t ab0 = 128u * (c >> 1) + 16u * (c & 1);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int f = 0; f < 4; ++f) av[mt][f] = buf_load16(ab, (ok && tok_ok[mt]) ? aoff[mt] + ab0 + 32 * f : a_end);
  };
  auto compute_step = [&](const v4i (&wv)[NT], const v4i (&av)[MT][4]) {
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
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc16[nt][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt][0], b0, acc16[nt][mt], 0, 0, 0);
        acc16[nt][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt][1], b1, acc16[nt][mt], 0, 0, 0);
        acc4[nt][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt][2], b2, acc4[nt][mt], 0, 0, 0);
        acc1[nt][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt][3], b3, acc1[nt][mt], 0, 0, 0);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int e = 0; e < 4; ++e) sa[mt] = __builtin_amdgcn_sdot4(av[mt][f][e], 0x01010101, sa[mt], false);
  };
  // (a form with two operand sets, the next step's loads issued before this step's MFMAs, measured no
  // faster at M = 17..32 on MI355X: the activation fragments' cache traffic, not the round trip, bounds it)
  for (int t = w; t < T; t += S) {
    v4i wv[NT], av[MT][4];
    load_step(t, wv, av);
    compute_step(wv, av);
  }
  // C layout of a 16x16 tile: lane (nl, g) holds tokens 4g + j (j < 4) of weight row nl.  sum(a) of
  // token nl over this wave's K range: add the 4 lane groups, then fetch token 4g + j's from lane 4g + j.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    int s = sa[mt];
    s += xor_lanes<16>(s);
    s += xor_lanes<32>(s);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int sj = __shfl(s, 4 * g + j, 64);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        red[w][nt][mt][j][lane] = acc1[nt][mt][j] + (acc4[nt][mt][j] >> 2) + (acc16[nt][mt][j] >> 4) - sj;
    }
  }
  __syncthreads();
  if constexpr (GLUE != 0) {
    if (w >= NT / 2) return;
    const int n = n0 + w * 16 + nl;  // output column = gate row; its up row is half + n
    if (n >= half) return;
    const float wsg = epi_wscale(ep, n), wsu = epi_wscale(ep, half + n);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = mt * 16 + 4 * g + j;
        if (tok >= M) continue;
        int tg = red[0][w][mt][j][lane], tu = red[0][w + NT / 2][mt][j][lane];
#pragma unroll
        for (int k = 1; k < S; ++k) {
          tg += red[k][w][mt][j][lane];
          tu += red[k][w + NT / 2][mt][j][lane];
        }
        const float as = epi_ascale(ep, tok);
        float yg = __fmul_rn(__fmul_rn((float)tg, wsg), as), yu = __fmul_rn(__fmul_rn((float)tu, wsu), as);
        if (ep.mid_dtype == WFB_BF16) {
          yg = bf16_bits_to_f32(f32_to_bf16_rne(yg));
          yu = bf16_bits_to_f32(f32_to_bf16_rne(yu));
        }
        reinterpret_cast<float*>(ep.out)[(int64_t)tok * ep.ldo + n] = glu<GLUE>(yg, yu);
      }
    return;
  }
  if (w >= NT) return;
  const int nt = w;
  const int n = n0 + nt * 16 + nl;
  // token scales of the late (non-PRE) epilogue, all loaded before the first is used: an index clamped
  // into range instead of a branch around each load
  float asl[4 * MT];
  if constexpr (!PRE) {
#pragma unroll
    for (int j = 0; j < 4 * MT; ++j) {
      const int tok = (j / 4) * 16 + 4 * g + (j % 4);
      asl[j] = ep.a_scale ? ep.a_scale[tok < M ? tok : 0] : 1.0f;
    }
  }
  if (ep.amax) {  // argmax epilogue: max over the 16 rows (lanes 16g .. 16g + 15) of each token
    const float ws = PRE ? col.ws : n < N ? epi_wscale(ep, n) : 0.0f;
    const float bias = PRE ? col.bias : n < N ? epi_bias(ep, n) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = mt * 16 + 4 * g + j;
        int tot = red[0][nt][mt][j][lane];
#pragma unroll
        for (int k = 1; k < S; ++k) tot += red[k][nt][mt][j][lane];
        const bool valid = tok < M && n < N;
        uint64_t key;
        if constexpr (PRE)
          key = epi_store_key_r(ep, ws, col.as[4 * mt + j], bias, col.res[4 * mt + j], tok, n, tot, valid);
        else
          key = epi_store_key(ep, ws, valid ? asl[4 * mt + j] : 0.0f, bias, tok, n, tot, valid);
        key = group_max_u64<16>(key);
        const int slot = blockIdx.x * NT + nt;  // one slot per 16 rows
        if (nl == 0 && tok < M && slot < (N + 15) / 16) ep.amax[(int64_t)slot * (ep.amax_ld ? ep.amax_ld : M) + tok] = key;
      }
    return;
  }
  if (n >= N) return;
  const float ws = PRE ? col.ws : epi_wscale(ep, n);
  const float bias = PRE ? col.bias : epi_bias(ep, n);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tok = mt * 16 + 4 * g + j;
      int tot = red[0][nt][mt][j][lane];
#pragma unroll
      for (int k = 1; k < S; ++k) tot += red[k][nt][mt][j][lane];
      if (tok < M) {
        if constexpr (PRE) epi_store_r(ep, ws, col.as[4 * mt + j], bias, col.res[4 * mt + j], tok, n, tot);
        else epi_store(ep, ws, asl[4 * mt + j], bias, tok, n, tot);
      }
    }
}

// Launch shape from sweeps on MI355X over the Llama-3-8B / BitNet-2B decode shapes (M = 1..16):
// enough workgroups for 256 CUs first, then more rows per workgroup (fewer, longer waves and shared
// activation loads): 4 row tiles x 4 waves for N >= 24576, 2 row tiles x 8 waves for N >= 6144 with
// K <= 8192, else one row tile x 8 waves (4 for short K).  NT > 1 only at MT <= 2 (LDS).
template <int MT>
hipError_t launch_skinny(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                         hipStream_t s) {
  const int T = (C + 3) / 4;
  if constexpr (MT == 1) {
    if (n >= 24576) {
      hipLaunchKernelGGL((gemm_i2s_skinny_kernel<MT, 4, 4>), dim3((n + 63) / 64), dim3(256), 0, s, W, A, lda, m, n, C,
                         e);
      return hipGetLastError();
    }
  }
  if constexpr (MT <= 2) {
    if (n >= 6144 && C <= 128) {
      hipLaunchKernelGGL((gemm_i2s_skinny_kernel<MT, 8, 2>), dim3((n + 31) / 32), dim3(512), 0, s, W, A, lda, m, n, C,
                         e);
      return hipGetLastError();
    }
  }
  if (T >= 8) {
    hipLaunchKernelGGL((gemm_i2s_skinny_kernel<MT, 8, 1>), dim3((n + 15) / 16), dim3(512), 0, s, W, A, lda, m, n, C, e);
  } else {
    hipLaunchKernelGGL((gemm_i2s_skinny_kernel<MT, 4, 1>), dim3((n + 15) / 16), dim3(256), 0, s, W, A, lda, m, n, C, e);
  }
  return hipGetLastError();
}

// Prefill GEMM (M > 64): v_mfma_i32_32x32x32_i8.  Workgroup tile BM x 256 (BM = 32 TM), four waves
// side by side in N, each owning 64 weight columns (wave tile BM x 64 = TM x 2 MFMA tiles).  K advances
// in stages of KB I2_S blocks (128 KB weights).
//  * Operand roles: weights are src0 and activations src1, so an accumulator tile is C^T: lane (i, g)
//    register r holds token row i and weight column 8*(r/4) + 4*g + r%4.
//  * k-slot pairing: lane (i, g) feeds the 16 packed bytes of half g of an I2_S block of its weight
//    row -- field f of them covers k = 128*b + 32f + 16g + 0..15 -- so the activation operand of
//    the same lane is the 16 contiguous bytes at that k.  A field enters the MFMA as its raw code
//    {0,1,2} (shift + AND per dword); the +1 offset is removed at the end with each token's sum of
//    activations: acc = sum(code * a) - sum(a).
//  * Both operands go from global memory straight into LDS (buffer_load_dwordx4 ... lds, 16 bytes per
//    lane at LDS base + 16 * lane), double buffered per stage.  Each load instruction covers whole
//    128-byte lines (activations: 8 or 4 rows) or 16-32 rows x 32-64 bytes (weights), against 32 rows
//    per instruction when weights are loaded into registers in MFMA layout.  The global source of
//    each lane is chosen so the LDS rows come out XOR-swizzled in 16-byte chunks, which makes the
//    MFMA-operand reads conflict-free.
//  * Per stage: one vmcnt(0) + barrier, the next stage's loads issued, then the stage multiplied.
//    All operand fragments of the stage are read up front (double-buffered MFMA tiles per field for
//    TM = 4); the unpack of field f + 1 is interleaved with the MFMAs of field f.
//  * sum(a): each wave sums a quarter of the tile rows from the staged activations.
//  * Tile order: XCD-aware (each XCD takes a contiguous range of tiles) and grouped by kGroupM tile
//    rows, so the workgroups resident on one XCD share activation rows and weight columns in its L2.
//  * EPI = 1 (bf16 output, no bias, no accumulator copy): the tile is converted in registers, staged
//    through LDS and written with 16-byte stores that fill whole output lines.  EPI = 2 (fp32 or bf16
//    output with an optional residual, aligned rows): fp32 outputs staged through LDS, the residual
//    added after a coalesced 16-byte load, whole-line stores.  EPI = 0: any output type, bias,
//    accumulator copy, stored from registers.
//  * KSPL = 2..4: groups of four waves split the tile's K stages, their int32 partials added in LDS.
//  * GL (gated gate|up, with KSPL = 2): 64 gate rows and their 64 up rows per tile; the fp32 output is
//    act(gate) * up, the up products handed to the gate waves through LDS.
constexpr int kGroupM = 8;

typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void lds_load16(buf_t r, void* lds_base, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds_base, 16, voff, 0, 0, 0);
}

template <int TM, int KB, int OCC, int EPI, int TN, int KSPL = 1, int GL = 0>
__global__ __launch_bounds__(256 * KSPL) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm_i2s_tile_kernel(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ A, int64_t lda, int M, int N, int K, int tiles_m,
    int tiles_n, int ntiles, bool vec_out, Epilogue ep) {
  // TN 32-column MFMA tiles per wave: 256-column tiles, or 128 where 256 leave most of the chip idle
  constexpr int BM = 32 * TM, BN = 128 * TN;
  constexpr int AROW = 128 * KB;  // bytes of an activation row per stage
  constexpr int CH = 8 * KB;      // 16-byte chunks per activation row
  constexpr int BROW = 32 * KB;   // bytes of a weight row per stage
  constexpr int ASZ = BM * AROW, BSZ = BN * BROW;
  constexpr int AI = ASZ / 4096, BI = BSZ / 4096;  // 1 KB load instructions per wave and stage
  constexpr int ARPI = 64 / CH;                    // activation rows per load instruction
  constexpr int BLPR = BROW / 16;                  // lanes per weight row in a load instruction
  constexpr int X = 4 * KB;                        // (block, field) MFMA steps per stage
  constexpr int LPR = 256 / BM, SCH = CH / LPR;    // sum(a): lanes per row, chunks per lane
  static_assert(AI >= 1 && BI >= 1 && ASZ >= 8192 && BSZ >= 8192 && SCH >= 1 && SCH <= X && LPR <= 8, "tile shape");
  // KSPL > 1: KSPL groups of four waves split the stages of K (group kh takes stages kh*KSH ..), each with
  // its own operand buffers and sum(a); their integer tile partials are added in LDS at the end (exact, in
  // any order) and group 0 runs the epilogue -- more waves on one tile where few tiles leave CUs idle.
  static_assert(KSPL >= 1 && KSPL <= 4, "one to four K groups");
  // GL (1 SiLU, 2 relu^2): W is gate|up (N = 2 * half); a tile's 128 weight rows are 64 gate rows n0 .. and
  // their up rows half + n0 .., loaded and multiplied by waves 0-1 and 2-3 (one wave's load instructions
  // cover the 32 rows it multiplies), and the epilogue stores act(gate) * up fp32 for 64 output columns
  static_assert(GL == 0 || (TN == 1 && EPI == 0 && BI * (64 / BLPR) == 32), "gated tiles: 128 rows, 32 loaded per wave");
  __shared__ __attribute__((aligned(16))) int8_t lds_a0s[KSPL][ASZ];
  __shared__ __attribute__((aligned(16))) int8_t lds_a1s[KSPL][ASZ];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b0s[KSPL][BSZ];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b1s[KSPL][BSZ];
  __shared__ int rowsum_s[KSPL][BM];
  const int tid = threadIdx.x, l = tid & 63, wq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = KSPL > 1 ? wq >> 2 : 0, wn = KSPL > 1 ? wq & 3 : wq;  // K group, wave within it
  int8_t* const lds_a0 = lds_a0s[kh];
  int8_t* const lds_a1 = lds_a1s[kh];
  uint8_t* const lds_b0 = lds_b0s[kh];
  uint8_t* const lds_b1 = lds_b1s[kh];
  int* const rowsum = rowsum_s[kh];
  const int i = l & 31, g = l >> 5;

  const int per = gridDim.x / 8;  // the grid is a multiple of 8
  const int t = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (t >= ntiles) return;
  const int gsz = kGroupM * tiles_n;
  const int grp = t / gsz, rr = t - grp * gsz;
  const int gm = min(kGroupM, tiles_m - grp * kGroupM);
  const int m0 = (grp * kGroupM + rr % gm) * BM, n0 = (rr / gm) * (GL ? BN / 2 : BN);
  const int half = N / 2;  // (gated mode)

  // The buffer descriptors start at the tile's first activation row and first weight row (64-bit
  // pointer arithmetic), so the 32-bit offsets inside them stay below (BM - 1) * lda + K and
  // 256 * K / 4 whatever M, N and the row stride (the host checks (BM - 1) * lda + K < 2^31).
  const int KS = (K + AROW - 1) / AROW;
  const uint32_t row_bytes = (uint32_t)K / 4;
  const int mrows = min(BM, M - m0), nrows = GL ? min(BN / 2, half - n0) : min(BN, N - n0);
  const uint32_t a_end = (uint32_t)((int64_t)(mrows - 1) * lda + K), b_end = (uint32_t)nrows * row_bytes;
  const buf_t ab = make_buf(A + (int64_t)m0 * lda, a_end);
  const int wrow0 = GL && wn >= 2 ? half + n0 : n0;  // first weight row this wave loads from (gated: up rows)
  const buf_t wb = make_buf(W + (int64_t)wrow0 * row_bytes, b_end);

  // LDS position p of activation row r holds chunk p ^ aswz(r); position q of weight row R holds
  // 16-byte piece q ^ bswz(R).  (16 consecutive rows then fall on 16 distinct 16-byte bank groups.)
  auto aswz = [](int r) { return KB == 2 ? (r & 15) : ((r >> 1) & 7); };
  auto bswz = [](int R) { return KB == 2 ? ((R >> 2) & 3) : ((R >> 3) & 1); };

  // Load descriptors: wave wn issues instructions AI*wn.. and BI*wn.. of each stage.  Rows past the
  // end of A or W are clamped to the last one (their results are never stored); bytes past K get an
  // offset beyond the buffer and load as zeros without touching memory.  Offsets are tile-relative.
  uint32_t a_row[AI], a_col[AI], b_row[BI], b_col[BI];
#pragma unroll
  for (int jj = 0; jj < AI; ++jj) {
    const int r = ARPI * (AI * wn + jj) + l / CH;
    a_row[jj] = (uint32_t)((int64_t)min(r, mrows - 1) * lda);
    a_col[jj] = 16 * ((l % CH) ^ aswz(r));
  }
#pragma unroll
  for (int jj = 0; jj < BI; ++jj) {
    const int R = (64 / BLPR) * (BI * wn + jj) + l / BLPR;
    const int Rl = GL && wn >= 2 ? R - BN / 2 : R;  // row within the block this wave loads from
    b_row[jj] = (uint32_t)min(Rl, nrows - 1) * row_bytes;
    b_col[jj] = 16 * ((l % BLPR) ^ bswz(R));
  }
  auto issue = [&](int kt, int8_t* la, uint8_t* lb) {
#pragma unroll
    for (int jj = 0; jj < AI; ++jj) {
      const uint32_t ka = (uint32_t)AROW * kt + a_col[jj];
      lds_load16(ab, la + (AI * wn + jj) * 1024, ka < (uint32_t)K ? a_row[jj] + ka : a_end);
    }
#pragma unroll
    for (int jj = 0; jj < BI; ++jj) {
      const uint32_t kb = (uint32_t)BROW * kt + b_col[jj];
      lds_load16(wb, lb + (BI * wn + jj) * 1024, kb < row_bytes ? b_row[jj] + kb : b_end);
    }
  };

  // per-lane LDS offsets of the MFMA operands and of the sum(a) chunks (the same every stage)
  uint32_t aoffs[X], boffs[KB][TN], soffs[SCH];
#pragma unroll
  for (int x = 0; x < X; ++x) aoffs[x] = i * AROW + (((8 * (x >> 2) + 2 * (x & 3) + g) ^ aswz(i)) * 16);
#pragma unroll
  for (int u = 0; u < KB; ++u)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int R = (wn * TN + tn) * 32 + i;
      boffs[u][tn] = R * BROW + (((2 * u + g) ^ bswz(R)) * 16);
    }
  // Wave wn sums rows [wn BM/4, (wn + 1) BM/4); lane part l % LPR of a row reads its SCH chunk positions
  // starting at a row-dependent rotation, so 16 consecutive lanes hit 16 distinct 16-byte bank groups
  // (without it, rows 256 B apart read the same group: a 4-way conflict).  The sum does not depend on
  // the order in which a row's chunks are read.
  const int srow = wn * (BM / 4) + l / LPR;
#pragma unroll
  for (int j = 0; j < SCH; ++j) soffs[j] = srow * AROW + ((l % LPR) * SCH + ((j + srow + (srow >> 2)) % SCH)) * 16;
  int ssum = 0;

  v16i acc[TN][TM];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[tn][tm][q] = 0;

  auto compute = [&](const int8_t* la, const uint8_t* lb) {
    constexpr int AF = TM >= 4 ? 2 : X;  // A fragments held: all of the stage, or a two-step ring
    v4i af[AF][TM], bw[KB][TN], bf[2][TN], sv[SCH];
    auto read_a = [&](v4i(&dst)[TM], int x) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) dst[tm] = *reinterpret_cast<const v4i*>(la + aoffs[x] + tm * 32 * AROW);
    };
#pragma unroll
    for (int u = 0; u < KB; ++u)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) bw[u][tn] = *reinterpret_cast<const v4i*>(lb + boffs[u][tn]);
#pragma unroll
    for (int x = 0; x < (AF == X ? X : 1); ++x) read_a(af[x], x);
#pragma unroll
    for (int j = 0; j < SCH; ++j) sv[j] = *reinterpret_cast<const v4i*>(la + soffs[j]);
    __builtin_amdgcn_sched_barrier(0);
    auto unpack = [&](v4i(&dst)[TN], const v4i(&src)[TN], int f) {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[tn][e] = (int)(((uint32_t)src[tn][e] >> (6 - 2 * f)) & 0x03030303u);
    };
    unpack(bf[0], bw[0], 0);
#pragma unroll
    for (int x = 0; x < X; ++x) {
      if (AF != X && x + 1 < X) read_a(af[(x + 1) % AF], x + 1);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tn][tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[x & 1][tn], af[x % AF][tm], acc[tn][tm], 0, 0, 0);
      if (x + 1 < X) unpack(bf[(x + 1) & 1], bw[(x + 1) >> 2], (x + 1) & 3);
      if (x < SCH) {
#pragma unroll
        for (int e = 0; e < 4; ++e) ssum = __builtin_amdgcn_sdot4(sv[x][e], 0x01010101, ssum, false);
      }
      // interleave: one MFMA, then a share of the unpack / sum VALU work (and the next A reads)
#pragma unroll
      for (int k = 0; k < TM * TN; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        if (AF != X && k < TM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
  };

  if constexpr (KSPL == 1) {
    issue(0, lds_a0, lds_b0);
    for (int kb = 0; kb < KS; kb += 2) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of stage kb are in LDS
      __syncthreads();                      // everyone's; and everyone is done with stage kb - 1
      if (kb + 1 < KS) issue(kb + 1, lds_a1, lds_b1);
      compute(lds_a0, lds_b0);
      if (kb + 1 < KS) {
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        if (kb + 2 < KS) issue(kb + 2, lds_a0, lds_b0);
        compute(lds_a1, lds_b1);
      }
    }
  } else {
    // group kh: stages k0s .. k0s + ksn - 1; both groups step through KSH stages so that every wave of the
    // workgroup meets the same barriers (the shorter group skips its missing last stage's loads and work)
    const int KSH = (KS + KSPL - 1) / KSPL, k0s = kh * KSH, ksn = min(KS - k0s, KSH);
    if (ksn > 0) issue(k0s, lds_a0, lds_b0);
    for (int kb = 0; kb < KSH; kb += 2) {
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
      if (kb + 1 < ksn) issue(k0s + kb + 1, lds_a1, lds_b1);
      if (kb < ksn) compute(lds_a0, lds_b0);
      if (kb + 1 < KSH) {
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        if (kb + 2 < ksn) issue(k0s + kb + 2, lds_a0, lds_b0);
        if (kb + 1 < ksn) compute(lds_a1, lds_b1);
      }
    }
  }

  // sum(a) per row: the LPR lanes of a row (consecutive) hold partial sums of its chunks
  if constexpr (LPR >= 2) ssum += __builtin_amdgcn_update_dpp(0, ssum, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
  if constexpr (LPR >= 4) ssum += __builtin_amdgcn_update_dpp(0, ssum, 0x4E, 0xF, 0xF, false);  // 2,3,0,1
  if constexpr (LPR >= 8) ssum += __shfl_xor(ssum, 4);
  if ((l % LPR) == 0) rowsum[srow] = ssum;
  __syncthreads();  // also: every wave is done reading the operand buffers
  if constexpr (KSPL == 2) {
    // group 1's partial tiles into group 0's accumulators, wave wn through group 1's buffer number wn (free
    // now); sum(a) of a row is the sum of the two groups' row sums (rsum)
    static_assert(64 * TM * TN * 16 * 4 <= (ASZ < BSZ ? ASZ : BSZ), "a wave's partial tiles fit one buffer");
    int* xr = reinterpret_cast<int*>(wn == 0 ? (void*)lds_a0s[1] : wn == 1 ? (void*)lds_a1s[1]
                                     : wn == 2 ? (void*)lds_b0s[1] : (void*)lds_b1s[1]);
    if (kh == 1) {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int q = 0; q < 16; ++q) xr[((tn * TM + tm) * 16 + q) * 64 + l] = acc[tn][tm][q];
    }
    __syncthreads();
    if (kh == 1) return;  // (no barrier follows)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[tn][tm][q] += xr[((tn * TM + tm) * 16 + q) * 64 + l];
  } else if constexpr (KSPL > 2) {
    // the same with groups 1 .. KSPL - 1, each through its own buffers, added into group 0 in order
    static_assert(64 * TM * TN * 16 * 4 <= (ASZ < BSZ ? ASZ : BSZ), "a wave's partial tiles fit one buffer");
    auto xbuf = [&](int gk) {
      return reinterpret_cast<int*>(wn == 0 ? (void*)lds_a0s[gk] : wn == 1 ? (void*)lds_a1s[gk]
                                    : wn == 2 ? (void*)lds_b0s[gk] : (void*)lds_b1s[gk]);
    };
    if (kh >= 1) {
      int* xr = xbuf(kh);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int q = 0; q < 16; ++q) xr[((tn * TM + tm) * 16 + q) * 64 + l] = acc[tn][tm][q];
    }
    __syncthreads();
    if (kh >= 1) return;  // (no barrier follows)
#pragma unroll
    for (int gk = 1; gk < KSPL; ++gk) {
      const int* xr = xbuf(gk);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int q = 0; q < 16; ++q) acc[tn][tm][q] += xr[((tn * TM + tm) * 16 + q) * 64 + l];
    }
  }
  auto rsum = [&](int r) {
    if constexpr (KSPL <= 2) {
      return KSPL > 1 ? rowsum_s[0][r] + rowsum_s[KSPL - 1][r] : rowsum_s[0][r];
    } else {
      int v = rowsum_s[0][r];
#pragma unroll
      for (int gk = 1; gk < KSPL; ++gk) v += rowsum_s[gk][r];
      return v;
    }
  };

  if constexpr (GL != 0) {
    // up waves 2, 3 hand their rescaled products (rounded to ep.mid_dtype, as a plain linear stores them)
    // to gate waves 0, 1 through LDS; the gate waves store act(gate) * up (fp32) -- the skinny kernels'
    // gated epilogue, element for element
    static_assert(64 * TM * 16 * 4 <= ASZ, "a wave's products fit one activation buffer");
    float* xf = reinterpret_cast<float*>((wn & 1) ? lds_a1 : lds_a0);
    const int c0 = 32 * (wn & 1);  // the wave pair's 32 of the tile's 64 output columns
    auto mid = [&](float y) { return ep.mid_dtype == WFB_BF16 ? bf16_bits_to_f32(f32_to_bf16_rne(y)) : y; };
    if (wn >= 2) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        const int rs = rsum(tm * 32 + i);
        const float as = epi_ascale(ep, min(m0 + tm * 32 + i, M - 1));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float wsu = epi_wscale(ep, half + n0 + c0 + 8 * q + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            xf[((tm * 4 + q) * 4 + e) * 64 + l] = mid(__fmul_rn(__fmul_rn((float)(acc[0][tm][4 * q + e] - rs), wsu), as));
        }
      }
    }
    __syncthreads();  // (the waves of this K group only: the other one has ended)
    if (wn >= 2) return;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int m = m0 + tm * 32 + i;
      if (m >= M) continue;
      const int rs = rsum(tm * 32 + i);
      const float as = epi_ascale(ep, m);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + c0 + 8 * q + 4 * g;
        if (n >= half) continue;
        const float wsg = epi_wscale(ep, n);
        float o4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float yg = mid(__fmul_rn(__fmul_rn((float)(acc[0][tm][4 * q + e] - rs), wsg), as));
          o4[e] = glu<GL>(yg, xf[((tm * 4 + q) * 4 + e) * 64 + l]);
        }
        float* o = reinterpret_cast<float*>(ep.out) + (int64_t)m * ep.ldo + n;
        if (vec_out && n + 3 < half) {
          *reinterpret_cast<float4*>(o) = make_float4(o4[0], o4[1], o4[2], o4[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < half) o[e] = o4[e];
        }
      }
    }
    return;
  }

  // weight scale per 4-column output group (segments are multiples of 8 rows, so a group has one)
  float wsg[TN][4];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int q = 0; q < 4; ++q) wsg[tn][q] = epi_wscale(ep, n0 + (wn * TN + tn) * 32 + 8 * q + 4 * g);
  if constexpr (EPI == 1) {
    // per 32-row MFMA tile: convert in registers, stage 32 rows x 32 TN bf16 (64 TN-byte rows, 16-byte
    // chunks XOR-swizzled by row) in this wave's own LDS buffer, store whole rows (8 rows x 128 B or
    // 16 rows x 64 B per instruction)
    constexpr int CPR = 4 * TN, RPI = 64 / CPR;  // 16-byte chunks per staged row, rows per instruction
    uint8_t* st = wn == 0 ? reinterpret_cast<uint8_t*>(lds_a0)
                : wn == 1 ? reinterpret_cast<uint8_t*>(lds_a1)
                : wn == 2 ? lds_b0 : lds_b1;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int rs = rsum(tm * 32 + i);
      const float as = epi_ascale(ep, min(m0 + tm * 32 + i, M - 1));
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = __fmul_rn(__fmul_rn((float)(acc[tn][tm][4 * q + e] - rs), wsg[tn][q]), as);
          const bf16x2_t lo = __builtin_convertvector((f32x2_t){y[0], y[1]}, bf16x2_t);
          const bf16x2_t hi = __builtin_convertvector((f32x2_t){y[2], y[3]}, bf16x2_t);
          const int c = tn * 4 + q;
          *reinterpret_cast<uint2*>(st + i * 16 * CPR + ((c ^ (i & (CPR - 1))) * 16) + 8 * g) =
              make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
        }
#pragma unroll
      for (int j = 0; j < 32 / RPI; ++j) {
        const int r = RPI * j + l / CPR, c = l % CPR;
        const v4i v = *reinterpret_cast<const v4i*>(st + r * 16 * CPR + ((c ^ (r & (CPR - 1))) * 16));
        const int m = m0 + tm * 32 + r, n = n0 + wn * 32 * TN + c * 8;
        if (m < M) {
          uint16_t* o = reinterpret_cast<uint16_t*>(ep.out) + (int64_t)m * ep.ldo + n;
          if (n + 7 < N) {
            *reinterpret_cast<v4i*>(o) = v;
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (n + e < N) o[e] = (uint16_t)((uint32_t)v[e / 2] >> (16 * (e & 1)));
          }
        }
      }
    }
  } else if constexpr (EPI == 2) {
    // per 32-row MFMA tile: stage the fp32 outputs (32 rows x 32 TN columns, 128 TN-byte rows, 16-byte
    // chunks XOR-swizzled by row) in this wave's own LDS buffer; each lane then takes 8 consecutive
    // outputs of a row, adds the residual read with one coalesced load (fp32 add, as epi_store), and
    // stores them in the output type with one or two 16-byte stores -- whole lines, like EPI = 1
    constexpr int CPR = 8 * TN, LPR8 = CPR / 2, RPI = 64 / LPR8;  // chunks per row, lanes per row, rows
    float* st = wn == 0 ? reinterpret_cast<float*>(lds_a0)
              : wn == 1 ? reinterpret_cast<float*>(lds_a1)
              : wn == 2 ? reinterpret_cast<float*>(lds_b0) : reinterpret_cast<float*>(lds_b1);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int rs = rsum(tm * 32 + i);
      const float as = epi_ascale(ep, min(m0 + tm * 32 + i, M - 1));
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float4 y;
          y.x = __fmul_rn(__fmul_rn((float)(acc[tn][tm][4 * q + 0] - rs), wsg[tn][q]), as);
          y.y = __fmul_rn(__fmul_rn((float)(acc[tn][tm][4 * q + 1] - rs), wsg[tn][q]), as);
          y.z = __fmul_rn(__fmul_rn((float)(acc[tn][tm][4 * q + 2] - rs), wsg[tn][q]), as);
          y.w = __fmul_rn(__fmul_rn((float)(acc[tn][tm][4 * q + 3] - rs), wsg[tn][q]), as);
          const int c = tn * 8 + 2 * q + g;  // 16-byte chunk of the row: columns 4c .. 4c + 3
          *reinterpret_cast<float4*>(st + i * 4 * CPR + ((c ^ (i & (CPR - 1))) * 4)) = y;
        }
#pragma unroll
      for (int j = 0; j < 32 / RPI; ++j) {
        const int r = RPI * j + l / LPR8, c8 = l % LPR8;
        const float4 ya = *reinterpret_cast<const float4*>(st + r * 4 * CPR + (((2 * c8) ^ (r & (CPR - 1))) * 4));
        const float4 yb = *reinterpret_cast<const float4*>(st + r * 4 * CPR + (((2 * c8 + 1) ^ (r & (CPR - 1))) * 4));
        float y[8] = {ya.x, ya.y, ya.z, ya.w, yb.x, yb.y, yb.z, yb.w};
        const int m = m0 + tm * 32 + r, n = n0 + wn * 32 * TN + c8 * 8;
        if (m >= M) continue;
        const bool full = n + 7 < N;
        if (ep.res) {
          float rv[8];
          if (full) {
            if (ep.res_dtype == WFB_BF16) load8<WFB_BF16>(ep.res, (int64_t)m * ep.ldr + n, rv);
            else load8<WFB_F32>(ep.res, (int64_t)m * ep.ldr + n, rv);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) rv[e] = n + e < N ? epi_res(ep, m, n + e) : 0.0f;
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] = __fadd_rn(y[e], rv[e]);
        }
        if (ep.out_dtype == WFB_BF16) {
          uint16_t* o = reinterpret_cast<uint16_t*>(ep.out) + (int64_t)m * ep.ldo + n;
          if (full) {
            uint32_t w4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
              w4[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){y[2 * e], y[2 * e + 1]}, bf16x2_t));
            *reinterpret_cast<uint4*>(o) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (n + e < N) o[e] = f32_to_bf16_rne(y[e]);
          }
        } else {
          float* o = reinterpret_cast<float*>(ep.out) + (int64_t)m * ep.ldo + n;
          if (full) {
            *reinterpret_cast<float4*>(o) = make_float4(y[0], y[1], y[2], y[3]);
            *reinterpret_cast<float4*>(o + 4) = make_float4(y[4], y[5], y[6], y[7]);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (n + e < N) o[e] = y[e];
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int m = m0 + tm * 32 + i;
      if (m >= M) continue;
      const float as = epi_ascale(ep, m);
      const int rs = rsum(tm * 32 + i);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + (wn * TN + tn) * 32 + 8 * q + 4 * g;
          if (n >= N) continue;
          const int32_t v[4] = {acc[tn][tm][4 * q] - rs, acc[tn][tm][4 * q + 1] - rs, acc[tn][tm][4 * q + 2] - rs,
                                acc[tn][tm][4 * q + 3] - rs};
          epi_store4(ep, wsg[tn][q], as, m, n, v, vec_out && n + 3 < N, N);
        }
    }
  }
}

template <int TM, int KB, int OCC, int TN = 2, int KSPL = 1>
hipError_t launch_tile(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                       hipStream_t s) {
  const int tiles_n = (n + 128 * TN - 1) / (128 * TN), tiles_m = (m + 32 * TM - 1) / (32 * TM);
  const int nwg = tiles_n * tiles_m;
  const int grid = ((nwg + 7) / 8) * 8;
  const bool vec_out = e.ldo % 4 == 0 && (uintptr_t)e.out % 16 == 0 && (uintptr_t)e.acc_out % 16 == 0;
  const bool bf16_only = e.out && e.out_dtype == WFB_BF16 && !e.bias && !e.acc_out && !e.res && e.ldo % 8 == 0 &&
                         (uintptr_t)e.out % 16 == 0;
  // staged fp32 epilogue: fp32 or bf16 out with an optional residual, 16-byte aligned rows
  const int osz = e.out_dtype == WFB_F32 ? 4 : 2, rsz = e.res_dtype == WFB_F32 ? 4 : 2;
  const bool staged = e.out && !e.bias && !e.acc_out && (e.ldo * osz) % 16 == 0 && (uintptr_t)e.out % 16 == 0 &&
                      (!e.res || ((e.ldr * rsz) % 16 == 0 && (uintptr_t)e.res % 16 == 0));
  if (bf16_only)
    hipLaunchKernelGGL((gemm_i2s_tile_kernel<TM, KB, OCC, 1, TN, KSPL>), dim3(grid), dim3(256 * KSPL), 0, s, W, A, lda, m, n, k,
                       tiles_m, tiles_n, nwg, vec_out, e);
  else if (staged)
    hipLaunchKernelGGL((gemm_i2s_tile_kernel<TM, KB, OCC, 2, TN, KSPL>), dim3(grid), dim3(256 * KSPL), 0, s, W, A, lda, m, n, k,
                       tiles_m, tiles_n, nwg, vec_out, e);
  else
    hipLaunchKernelGGL((gemm_i2s_tile_kernel<TM, KB, OCC, 0, TN, KSPL>), dim3(grid), dim3(256 * KSPL), 0, s, W, A, lda, m, n, k,
                       tiles_m, tiles_n, nwg, vec_out, e);
  return hipGetLastError();
}

// Gated gate|up (N = 2 * half rows) as 32 x 64-output tiles of the K-split tile kernel: out [m, half] fp32 =
// act(gate) * up.
template <int GL>
hipError_t launch_tile_glu(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                           hipStream_t s) {
  const int half = n / 2;
  const int tiles_n = (half + 63) / 64, tiles_m = (m + 31) / 32;
  const int nwg = tiles_n * tiles_m;
  const int grid = ((nwg + 7) / 8) * 8;
  const bool vec_out = e.ldo % 4 == 0 && (uintptr_t)e.out % 16 == 0;
  hipLaunchKernelGGL((gemm_i2s_tile_kernel<1, 2, 4, 0, 1, 2, GL>), dim3(grid), dim3(512), 0, s, W, A, lda, m, n, k,
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

// 33..64 tokens as two launches of the staged kernel over token rows 0..31 and 32..M-1 (per-lane or
// whole-line epilogues and the gated product, act != 0; not the greedy-argmax keys, which are laid out by
// the launch's M).  Returns hipErrorNotSupported, before launching anything, where the staged kernel does
// not take 32 tokens of this shape.
static hipError_t launch_token_halves(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda,
                                      const Epilogue& e, int act, hipStream_t s) {
  const hipError_t st = launch_skinny_lds(W, n, k, A, 32, lda, e, act, s);
  if (st != hipSuccess) return st;
  Epilogue e2 = e;
  if (e2.a_scale) e2.a_scale += 32;
  // the gated product is stored fp32
  if (e2.out) e2.out = static_cast<char*>(e2.out) + 32 * e2.ldo * (act || e2.out_dtype == WFB_F32 ? 4 : 2);
  if (e2.acc_out) e2.acc_out += 32 * e2.ldo;
  if (e2.res) e2.res = static_cast<const char*>(e2.res) + 32 * e2.ldr * (e2.res_dtype == WFB_F32 ? 4 : 2);
  const hipError_t st2 = launch_skinny_lds(W, n, k, A + 32 * lda, m - 32, lda, e2, act, s);
  return st2 == hipErrorNotSupported ? hipErrorInvalidValue : st2;  // the second half must not fall back
}

template <int MT, int GLUE>
hipError_t launch_skinny_glu(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                             hipStream_t s) {
  const int half = n / 2;
  if (MT == 1 && n >= 24576)
    hipLaunchKernelGGL((gemm_i2s_skinny_kernel<MT, 4, 4, GLUE>), dim3((half + 31) / 32), dim3(256), 0, s, W, A, lda, m,
                       n, C, e);
  else
    hipLaunchKernelGGL((gemm_i2s_skinny_kernel<MT, 8, 2, GLUE>), dim3((half + 15) / 16), dim3(512), 0, s, W, A, lda, m,
                       n, C, e);
  return hipGetLastError();
}

hipError_t launch_gemm_i2s_skinny(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda,
                                  const Epilogue& e, hipStream_t s) {
  const int C = k / 64;
  if (m <= 64) {
    const hipError_t st = launch_skinny_lds(W, n, k, A, m, lda, e, 0, s);
    if (st != hipErrorNotSupported) return st;
  }
  if (m <= 16) return launch_skinny<1>(W, n, C, A, m, lda, e, s);
  if (m <= 32) return launch_skinny<2>(W, n, C, A, m, lda, e, s);
  if (m <= 64) return launch_skinny<4>(W, n, C, A, m, lda, e, s);
  return hipErrorInvalidValue;
}

hipError_t launch_gemm_i2s_glu(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda, int act,
                               const Epilogue& e, hipStream_t s) {
  const int C = k / 64;
  // 33..64 tokens, and 17..32 on long rows of a wide gate|up: the K-split tile kernel with the gated
  // epilogue, 32 tokens x 64 outputs per tile (interleaved medians on MI355X against the staged kernel
  // below, SiLU, bf16 products: gated 28672 x 4096 at M = 64 43.8 -> 19.0 us, M = 33 28.6 -> 19.6, M = 24
  // 24.4 -> 14.6; 13824 x 2560 at M = 64 15.8 -> 10.9, M = 33 13.3 -> 12.4; 3072 x 4096 at M = 64 13.2 ->
  // 12.1; slower at M <= 32 on 13824 x 2560 (8.2 -> 10.7, half the CUs without a tile) and 3072 x 4096,
  // and at M <= 16)
  const bool small_offsets = (int64_t)n * (k / 4) <= INT32_MAX && (int64_t)(m - 1) * lda + k <= INT32_MAX;
  if (m > 64 || n % 2 != 0 || !small_offsets) return hipErrorInvalidValue;  // (the C ABI checks these first)
  if (m > 32 || (m > 16 && k >= 4096 && n >= 8192))
    return act == WFB_ACT_SILU ? launch_tile_glu<WFB_ACT_SILU>(W, n, k, A, m, lda, e, s)
                               : launch_tile_glu<WFB_ACT_RELU2>(W, n, k, A, m, lda, e, s);
  const hipError_t st = launch_skinny_lds(W, n, k, A, m, lda, e, act, s);
  if (st != hipErrorNotSupported) return st;
#define WFB_GLU(MT)                                                                              \
  return act == WFB_ACT_SILU ? launch_skinny_glu<MT, WFB_ACT_SILU>(W, n, C, A, m, lda, e, s) \
                             : launch_skinny_glu<MT, WFB_ACT_RELU2>(W, n, C, A, m, lda, e, s)
  if (m <= 16) WFB_GLU(1);
  WFB_GLU(2);
#undef WFB_GLU
}

hipError_t launch_gemm_i2s(const uint8_t* W, int n, int k, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                           hipStream_t s) {
  const int C = k / 64;
  // Split-K skinny kernel while its per-workgroup re-read of all M activation rows stays cheap against
  // the weight stream (measured on MI355X over the Llama-3-8B / BitNet-2B decode shapes: always for
  // M <= 8, for larger M while N * (16-token tiles) <= 32768); it addresses through 32-bit offsets.
  const int mt = (m + 15) / 16;
  // 32-row tiles of 256 columns that leave CUs idle (fewer than 256): 128-column tiles, four waves of 32
  // columns, measured on MI355X (13824 x 2560 at M = 64: 12.9 -> 9.6 us; M = 128: 2560 x 2560 10.3 ->
  // 7.7, 4096 x 14336 45.2 -> 35.5; 2560 x 6912 at M = 512 24.3 -> 22.3), and two groups of four waves
  // splitting K on each tile, two workgroups per CU (interleaved medians: 13824 x 2560 at M = 64 8.1 ->
  // 7.2 us, 6144 x 4096 at M = 64 10.1 -> 8.5, 2560 x 6912 at M = 256 15.7 -> 12.3, at M = 512 20.1 ->
  // 18.9; 28672 x 4096 at M = 64 unchanged)
  const bool few_tiles = (int64_t)((n + 255) / 256) * ((m + 31) / 32) < 256;
  const bool small_offsets = (int64_t)n * (k / 4) <= INT32_MAX && (int64_t)(m - 1) * lda + k <= INT32_MAX;
  // 17 <= M <= 64 on wide outputs: the 32-row tile kernel (one or two tile rows, its time nearly flat
  // in M), measured on MI355X against the skinny and whole-K kernels over M = 9..64 and the BitNet-2B /
  // Llama-3-8B shapes: faster from N * ceil(M/16) >= 18432 with K <= 8192 (M = 64: 28672 x 4096
  // 67.1 -> 15.0 us, 13824 x 2560 26.1 -> 10.0, 6144 x 4096 25.8 -> 13.3; M = 24: 13824 x 2560 10.5 -> 9.8),
  // the split-K kernels below that and for longer rows (M = 64, 4096 x 14336: 33.5 vs 37.2 us).
  // 33..64 tokens on rows of 4096 or more and 4096 or more outputs: the tile kernel with its K split
  // (interleaved medians on MI355X: 4096 x 4096 at M = 40..64 9.5-10.4 -> 8.4 us, 4096 x 14336 24.7-31.5
  // -> 21.5; 6144 x 4096 and 28672 x 4096 within 1%; at 17..32 tokens, and on 2560-long or 2560-row
  // shapes, the kernels below stay ahead)
  // (rows of 8192 or more: four groups of four waves splitting K, 4096 x 14336 at M = 64 22.2 -> 18.2 us)
  if (m > 32 && m <= 64 && small_offsets && !e.amax && k >= 4096 && n >= 4096)
    return k >= 8192 ? launch_tile<1, 2, 4, 1, 4>(W, n, k, A, m, lda, e, s)
                     : launch_tile<1, 2, 4, 1, 2>(W, n, k, A, m, lda, e, s);
  // operands staged in LDS (skinny_lds.h) where its LDS holds them (17..32 tokens: where measured faster)
  if (m <= 64 && small_offsets) {
    const hipError_t st = launch_skinny_lds(W, n, k, A, m, lda, e, 0, s);
    if (st != hipErrorNotSupported) return st;
  }
  // 33..64 tokens on rows from 4096 to 7168 of narrow outputs (the four-tile form stages neither them nor
  // their registers): two launches of the two-tile form, measured on MI355X against the split-K kernel
  // (2560 x 6912: M = 64 18.8 -> 12.7 us, M = 33 13.5 -> 10.4)
  if (m > 32 && m <= 64 && small_offsets && !e.amax && k > 4096 && k <= 7168 && n <= 4096) {
    // from 49 tokens one launch with two token blocks of workgroups (2560 x 6912 at M = 64: 12.4 -> 11.2 us;
    // at M = 33..48 the two launches stay ahead, 10.3-11.0 against 11.0-11.1)
    if (m > 48) {
      const hipError_t st = launch_skinny_lds_mr32(W, n, C, A, m, lda, e, 0, 1, NormSrc{}, s);
      if (st != hipErrorNotSupported) return st;
    }
    const hipError_t st = launch_token_halves(W, n, k, A, m, lda, e, 0, s);
    if (st != hipErrorNotSupported) return st;
  }
  if (m > 16 && m <= 64 && small_offsets && (int64_t)n * mt >= 18432 && k <= 8192)
    return few_tiles ? launch_tile<1, 2, 4, 1, 2>(W, n, k, A, m, lda, e, s) : launch_tile<1, 2, 3>(W, n, k, A, m, lda, e, s);
  if (m <= 64 && small_offsets && (m <= 8 || (int64_t)n * (mt == 3 ? 4 : mt) <= 32768)) {
    if (m <= 16) return launch_skinny<1>(W, n, C, A, m, lda, e, s);
    if (m <= 32) return launch_skinny<2>(W, n, C, A, m, lda, e, s);
    return launch_skinny<4>(W, n, C, A, m, lda, e, s);
  }
  if (m <= 16) return launch_mt<1>(W, n, C, A, m, lda, e, s);
  if (m <= 32) return launch_mt<2>(W, n, C, A, m, lda, e, s);
  if (m <= 64) return launch_mt<4>(W, n, C, A, m, lda, e, s);
  // Tile height by the number of 256-column tiles (512 workgroup slots at two per CU), from a sweep on
  // MI355X over M = 1024..8192 and the BitNet-2B / Llama-3-8B shapes: 128-row tiles (half the weight
  // unpack per MFMA) from 320 of them (M = 2048, N = 6144: 58.8 vs 66.5 us), 64-row tiles below that
  // (M = 1024, N = 4096, K = 14336: 69.1 vs 107.5 us), 32-row tiles when even 64-row ones leave most
  // of the chip idle (M = 512, N = 2560, K = 6912: 21.7 vs 30.8 us).
  const int64_t tn = (n + 255) / 256, t128 = tn * ((m + 127) / 128), t64 = tn * ((m + 63) / 64);
  if (t128 >= 320) return launch_tile<4, 1, 2>(W, n, k, A, m, lda, e, s);
  // 64-row tiles: 256 columns, or 128 columns at three workgroups per CU where those fill the last round of
  // workgroup slots better (2560 x 6912 at M = 2048: 320 tiles on 512 slots, or 640 on 768: 47.3 -> 42.5 us;
  // 13824 x 2560 at M = 512 keeps 256 columns, 23.1 against 27.3 us; interleaved medians on MI355X)
  auto fill = [](int64_t t, int64_t slots) { return (double)t / (double)(((t + slots - 1) / slots) * slots); };
  if (t64 >= 160) {
    const int64_t t64n = ((n + 127) / 128) * ((m + 63) / 64);
    if (fill(t64n, 768) > fill(t64, 512) + 0.1) return launch_tile<2, 2, 3, 1>(W, n, k, A, m, lda, e, s);
    return launch_tile<2, 2, 2>(W, n, k, A, m, lda, e, s);
  }
  // 160..256 tiles of 32 x 256: three groups of four waves splitting K on each, one workgroup per CU
  // (interleaved medians on MI355X against the two-group 32 x 128 and the one-group 32 x 256 forms: 2560 x
  // 6912 at M = 512 20.5 -> 17.7 us, 4096 x 14336 at M = 512 49.6 -> 37.4, 2560 x 2560 at M = 512 9.9 ->
  // 9.5); fewer tiles on rows of 6912 or more: 32 x 128 tiles with four groups (2560 x 6912 at M = 256 12.9
  // -> 11.6)
  const int64_t t256 = tn * ((m + 31) / 32);
  if (t256 >= 160 && t256 <= 256) return launch_tile<1, 2, 3, 2, 3>(W, n, k, A, m, lda, e, s);
  if (few_tiles && k >= 6912) return launch_tile<1, 2, 4, 1, 4>(W, n, k, A, m, lda, e, s);
  return few_tiles ? launch_tile<1, 2, 4, 1, 2>(W, n, k, A, m, lda, e, s) : launch_tile<1, 2, 3>(W, n, k, A, m, lda, e, s);
}

}  // namespace wfb
