// Batched-decode linear for M <= 64 tokens with both operands staged in LDS (included by the five
// skinny_mr*.hip files, one per staged token-row count, so they compile in parallel).
//
// Replaces, like the other I2_S GEMM paths, bitnet_gemm_i2_i8 / bitnet_gemm_cpu
// (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:814-874, SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:370-406).
//
// v_mfma_i32_16x16x64_i8, one 16-token tile (two for 17..32 tokens, MR = 32, four for 33..64, MR = 64:
// each weight fragment read from LDS and unpacked once feeds every tile's MFMAs).  A workgroup owns NT tiles of 16 weight rows and all of K;
// its S waves split K into step pairs of 512 weights (128 packed bytes per row), wave w taking pairs
// w, w + S, ... (TP of them).  Measured on MI355X, what sets the time of this kernel is how its loads
// cover cache lines, so both operands are brought in whole lines by 16-byte LDS-DMA loads
// (buffer_load ... lds: lane l's 16 bytes land at LDS base + 16 l):
//  * weights: one instruction = 8 rows x 128 bytes (lanes 8r .. 8r+7 read row r's pair); the 16-row tile
//    of a pair takes two.  In LDS, 16-byte slot s of row r holds global chunk s ^ f(r),
//    f(r) = (r & 7) ^ (r >> 3), so the MFMA-layout reads of 16 rows fall on 16 distinct bank groups.
//    (Loading the MFMA layout directly -- 16 rows x 64 bytes per instruction, the other half line from
//    another wave -- measured 0.6 us slower for 8.8 MB of weights.)
//  * activations: per 256-weight step, MR token rows x 256 bytes, 4 rows per instruction; slot q of
//    token row t holds chunk q ^ (t & 15).
// MFMA operands: lane (nl, g) reads weight row nl, chunk 4 step + g (16 bytes = 64 weights; field f
// covers k = 128 (c / 2) + 32 f + 16 (c % 2) + 0..15 of chunk c) and the 16 activation bytes of token nl
// at the same k.  Fields enter masked but unshifted -- bits 1:0 (x1), 3:2 (x4), 5:4 and 7:6 >> 2 (x16) --
// into three accumulators; the code offset is removed with each token's sum(a).  Partial tiles of the S
// waves meet in LDS.
// Epilogues: plain outputs go through LDS (y = (acc * ws) * as + bias in fp32 per element, then each
// thread takes 4 consecutive outputs of a token row, adds the residual and stores them: whole-line
// stores, 0.3-0.5 us faster than per-lane ones at M = 8-16); accumulator copies, the greedy-argmax
// keys and the gated gate|up product are written from the MFMA layout.
// Gated mode (GLUE = 1 SiLU, 2 relu^2): W is gate|up (N = 2 * half); tiles 0 .. NT/2 - 1 are gate rows
// n0 + 16 j, the others the up rows half + n0 + 16 j; x = act(gate) * up is stored fp32 at [tok, n],
// both products rounded to ep.mid_dtype first (what a plain linear would store).
// Norm prologue (XT = storage type of x, K <= 4096): instead of loading int8 codes, every workgroup
// normalises and quantises the M float rows itself -- wave w takes rows w, w + S, ..., in the one-wave
// summation order of the per-token quantiser (lane l adds the squares of elements (l + 64 j) * 8 + e,
// j then e ascending, then a fixed xor butterfly), so the codes and scales are bit-identical to
// wfb_rmsnorm_quant_i8's -- and writes the codes into the activation staging in its swizzled layout
// (zeros from H to the staging's end).  A wave's first row and gamma are loaded before its weight
// DMA, so their latency overlaps the weight stream; the token scales reach the epilogue through the
// free half of the waves' weight staging, next to the partial tiles.
// Replaces, for decode, SubLN/RMSNorm -> activation_quant -> BitLinear
// (packages/training/src/wrinklefree/models/subln.py:42-59, 64-97,
// packages/training/src/wrinklefree/models/bitlinear.py:66-113) as the reference's fused layer ops run
// them per token (SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:150-231, 289-375).
#pragma once

#include "wfb_common.h"

namespace wfb {
namespace skinny_lds {

typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void dma16(buf_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, 0, 0, 0);
}

// The per-wave partial tiles of the K reduction overwrite the wave's own weight staging, and the staged
// output tile the activation staging, so the LDS is the two operand stagings only.
// With more than two token tiles per step pair (MT > 2 TP) the partial tiles get their own buffer.
constexpr size_t red_bytes(int S, int NT, int TP, int MT) { return MT > 2 * TP ? (size_t)S * MT * NT * 1024 : 0; }
// Activation staging of the codes path, in steps per wave: every step of the wave's pairs, or -- with
// several token tiles -- one slot restaged per pair (two tiles, several pairs) or per step (four tiles).
constexpr int act_steps(int TP, int MR) { return MR > 32 ? 1 : MR > 16 && TP > 1 ? 2 : 2 * TP; }
constexpr size_t lds_bytes(int S, int NT, int TP, int MR) {
  return (size_t)S * TP * NT * 2048 + (size_t)S * act_steps(TP, MR) * MR * 256 + red_bytes(S, NT, TP, (MR + 15) / 16);
}
// with the activations in registers (kAreg): the weight staging and the staged output tile
constexpr size_t lds_bytes_areg(int S, int NT, int TP, int MT) {
  return (size_t)S * TP * NT * 2048 + 16 * MT * 16 * NT * 4 + 64 + red_bytes(S, NT, TP, MT);
}

// ---- norm prologue helpers ---------------------------------------------------------------------------
// Storage-type tags of the prologue's x and gamma (kNone: no prologue / no gamma).  Distinct from the
// WFB_* dtype codes, where WFB_F32 is 0.
constexpr int kNone = 0, kBf16 = 1, kF32 = 2;
// Codes path with the activation fragments loaded straight into registers in MFMA layout instead of the
// LDS staging: for shapes whose M x K activation bytes do not fit the LDS beside the weights (the
// Llama-3-8B down projection, K = 14336, at M > 4).
constexpr int kAreg = 3;
inline int src_tag(int wfb_dtype) { return wfb_dtype == WFB_F32 ? kF32 : kBf16; }

// 8 consecutive elements of a row (storage tag DT), as raw 16-byte words (fp32: two), zero when not loaded
template <int DT>
struct Raw8 {
  v4i r[DT == kF32 ? 2 : 1] = {};
};
template <int DT>
__device__ __forceinline__ Raw8<DT> load_raw8(const void* p, int e0) {
  Raw8<DT> v;
  const v4i* q = reinterpret_cast<const v4i*>(reinterpret_cast<const char*>(p) + (int64_t)e0 * (DT == kF32 ? 4 : 2));
  v.r[0] = q[0];
  if constexpr (DT == kF32) v.r[1] = q[1];
  return v;
}
template <int DT>
__device__ __forceinline__ void widen8(const Raw8<DT>& v, float (&f)[8]) {
  if constexpr (DT == kF32) {
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
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, xor_lanes_f32<32>(v));
  v = fmaxf(v, xor_lanes_f32<16>(v));
  v = fmaxf(v, xor_lanes_f32<8>(v));
  v = fmaxf(v, xor_lanes_f32<4>(v));
  v = fmaxf(v, xor_lanes_f32<2>(v));
  return fmaxf(v, xor_lanes_f32<1>(v));
}
// the quantiser's fixed xor-butterfly order (partners 32, 16, 8, 4, 2, 1)
__device__ __forceinline__ float wave_sum_fixed_f32(float v) {
  v = __fadd_rn(v, xor_lanes_f32<32>(v));
  v = __fadd_rn(v, xor_lanes_f32<16>(v));
  v = __fadd_rn(v, xor_lanes_f32<8>(v));
  v = __fadd_rn(v, xor_lanes_f32<4>(v));
  v = __fadd_rn(v, xor_lanes_f32<2>(v));
  return __fadd_rn(v, xor_lanes_f32<1>(v));
}

// The M rows of x through the norm and the quantiser into the activation staging.  XT: x's storage tag;
// GT: gamma's (kNone: no gamma).  between() issues the weight DMA after the first row's loads.  Codes go
// to put() for k < H, zeros for H <= k < lim.  Returns the token scales of the wave's rows w, w + S, ...
// in sc[].
template <int S, int MR, int XT, int GT, class Put, class Between>
__device__ __forceinline__ void norm_prologue(const NormSrc& ns, int M, int w, int lane, int lim, Put put,
                                              Between between, float (&sc)[(MR + S - 1) / S]) {
  constexpr int RPW = (MR + S - 1) / S;
  const int H = ns.h;
  constexpr int GS = GT == kF32 ? kF32 : kBf16;
  Raw8<GS> gv[8];
  Raw8<XT> xv[8];
  auto load_row = [&](int r) {
    const void* xr = reinterpret_cast<const char*>(ns.x) + (int64_t)r * ns.ldx * (XT == kF32 ? 4 : 2);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e0 = (lane + 64 * j) * 8;
      xv[j] = e0 < H ? load_raw8<XT>(xr, e0) : Raw8<XT>{};
    }
  };
  if (w < M) load_row(w);
  if constexpr (GT != kNone) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e0 = (lane + 64 * j) * 8;
      gv[j] = e0 < H ? load_raw8<GS>(ns.gamma, e0) : Raw8<GS>{};
    }
  }
  between();
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = w + S * i;
    sc[i] = 1.0f;
    if (r >= M) break;
    if (i > 0) load_row(r);
    // x widened once; y = (x * rs) * gamma then replaces it
    float y[8][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) widen8<XT>(xv[j], y[j]);
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __fadd_rn(ss, __fmul_rn(y[j][e], y[j][e]));
    ss = wave_sum_fixed_f32(ss);
    const float rs = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(ss, (float)H), ns.eps)));
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float gm[8];
      if constexpr (GT != kNone) {
        widen8<GS>(gv[j], gm);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) gm[e] = 1.0f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y[j][e] = __fmul_rn(__fmul_rn(y[j][e], rs), gm[e]);
        mx = fmaxf(mx, fabsf(y[j][e]));
      }
    }
    mx = wave_max_f32(mx);
    if (mx < 1e-6f) mx = 1.0f;
    const float inv = __fdiv_rn(127.0f, mx);
    sc[i] = __fdiv_rn(mx, 127.0f);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e0 = (lane + 64 * j) * 8;
      if (e0 < lim) {  // codes up to H, zeros to the end of the staging
        uint32_t lo = 0, hi = 0;
        if (e0 < H) {
          lo = quant4_i8(&y[j][0], inv);
          hi = quant4_i8(&y[j][4], inv);
        }
        put(r, e0, lo, hi);
      }
    }
  }
}

template <int S, int NT, int TP, int MR, int GLUE, bool STAGED, int XT>
__global__ __launch_bounds__(64 * S) void kernel(const uint8_t* __restrict__ W, const int8_t* __restrict__ A,
                                                 int64_t lda, int M, int N, int C, Epilogue ep, NormSrc ns) {
  static_assert((GLUE ? NT / 2 : NT) <= S, "one wave per output row tile in the epilogue");
  static_assert(GLUE == 0 || NT % 2 == 0, "gated mode pairs gate and up tiles");
  static_assert(MR == 4 || MR == 8 || MR == 16 || MR == 32 || MR == 64, "staged token rows");
  constexpr bool NORM = XT == kF32 || XT == kBf16;  // codes formed in the prologue, token scales with them
  // 16-token tiles: MR = 32 / 64 run two / four, each weight fragment feeding all of them
  constexpr int MT = MR > 16 ? MR / 16 : 1;
  static_assert(MT == 1 || !NORM, "the norm prologue serves up to 16 tokens");
  constexpr bool RED_OWN = MT > 2 * TP;  // partial tiles beyond the wave's weight staging: own buffer
  // several token tiles (codes path): the activations of one step pair (two tiles, several pairs) or one
  // step (four tiles) at a time, each wave restaging its slot for its next unit (the weights of all its
  // pairs are staged up front); otherwise every step of the wave's pairs at once
  constexpr int STA = XT == kNone && MT > 2 ? 1 : 2;              // steps per slot
  constexpr bool RS = XT == kNone && MT > 1 && (TP > 1 || STA == 1);
  constexpr int TPA = RS ? 1 : TP;                                 // slots per wave
  static_assert(XT == kAreg || TPA * STA == act_steps(TP, MR), "staging size as the launch counts it");
  __shared__ __attribute__((aligned(16))) int8_t wl[S][TP][NT][2048];
  __shared__ __attribute__((aligned(16))) int8_t al[XT == kAreg ? 1 : S][XT == kAreg ? 1 : TPA][STA][XT == kAreg ? 16 : MR * 256];
  // staged output tile of the register-activation mode (the others use the activation staging)
  __shared__ __attribute__((aligned(16))) float ysb[XT == kAreg && STAGED ? 16 * MT * 16 * NT : 1];
  __shared__ __attribute__((aligned(16))) int redo[RED_OWN ? S : 1][RED_OWN ? MT * NT * 256 : 1];
  // partial tile (token tile mt, row tile nt, token slot j, lane) of wave w, in wave w's own weight
  // staging (free once the wave has read it: its LDS reads and writes execute in order) when it fits there
  auto red = [&](int wv, int mt, int nt, int j, int l) -> int& {
    int* base = RED_OWN ? &redo[wv][0] : reinterpret_cast<int*>(&wl[wv][0][0][0]);
    return base[((mt * NT + nt) * 4 + j) * 64 + l];
  };
  // norm prologue: scale of token tok, written by its wave (tok % S) after that wave's partial tiles
  constexpr int RPW = (MR + S - 1) / S;
  auto tok_scale = [&](int tok) -> float& {
    return reinterpret_cast<float*>(&wl[tok % S][0][0][0] + NT * 1024)[tok / S];
  };
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int half = N / 2;
  const int n0 = GLUE ? blockIdx.x * 16 * (NT / 2) : blockIdx.x * 16 * NT;
  if constexpr (MR == 32 && !NORM) {
    // launch over more than MR tokens: workgroups (x, y) take token rows MR y .. MR y + MR - 1 (the host
    // leaves the greedy-argmax keys out of this form)
    if (gridDim.y > 1) {
      const int t0 = MR * (int)blockIdx.y;
      A += (int64_t)t0 * lda;
      M = min(MR, M - t0);
      if (ep.a_scale) ep.a_scale += t0;
      if (ep.out) ep.out = static_cast<char*>(ep.out) + (int64_t)t0 * ep.ldo * (GLUE || ep.out_dtype == WFB_F32 ? 4 : 2);
      if (ep.acc_out) ep.acc_out += (int64_t)t0 * ep.ldo;
      if (ep.res) ep.res = static_cast<const char*>(ep.res) + (int64_t)t0 * ep.ldr * (ep.res_dtype == WFB_F32 ? 4 : 2);
    }
  }
  const uint32_t row_bytes = (uint32_t)C * 16;
  const uint32_t w_end = (uint32_t)N * row_bytes, a_end = (uint32_t)((int64_t)(M - 1) * lda + (int64_t)C * 64);
  const buf_t wb = make_buf(W, w_end);
  const buf_t ab = make_buf(A, a_end);
  const int T = (C + 3) >> 2, T2 = (C + 7) >> 3;
  auto tile_row = [&](int nt) {
    return !GLUE ? n0 + 16 * nt : nt < NT / 2 ? n0 + 16 * nt : half + n0 + 16 * (nt - NT / 2);
  };

  // ---- operands into LDS (every load of the wave in flight before the first wait) --------------------
  auto dma_weights = [&]() {
#pragma unroll
    for (int u = 0; u < TP; ++u) {
      const int p = w + S * u;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int r = lane >> 3;
          const int chunk = 8 * p + ((lane & 7) ^ (r ^ h));
          const int row = tile_row(nt) + 8 * h + r;
          const bool ok = p < T2 && chunk < C;
          dma16(wb, wl[w][u][nt] + 1024 * h, ok ? (uint32_t)row * row_bytes + 16u * chunk : w_end);
        }
    }
  };
  // staging slot of step st of the wave's pair u
  auto aslot = [&](int u, int st) -> int8_t* { return al[w][TPA == 1 ? 0 : u][STA == 1 ? 0 : st]; };
  // activations of steps st0 .. st1 - 1 of the wave's step pair u (MR token rows x 256 bytes per step,
  // 4 rows per instruction) into their slots
  auto dma_act = [&](int u, int st0, int st1) {
    const int p = w + S * u;
#pragma unroll
    for (int st = st0; st < st1; ++st)
#pragma unroll
      for (int i = 0; i < MR / 4; ++i) {
        const int t = 2 * p + st;
        const int tok = 4 * i + (lane >> 4);
        const int q = (lane & 15) ^ (tok & 15);
        const uint32_t kb = 256u * t + 16u * q;
        const bool ok = p < T2 && t < T && tok < M && kb < (uint32_t)(64 * C);
        dma16(ab, aslot(u, st) + 1024 * i, ok ? (uint32_t)((int64_t)tok * lda) + kb : a_end);
      }
  };
  // epilogue operands of the column this lane owns in the MFMA layout (row n, tokens 16 mt + 4g + j at
  // slot 4 mt + j)
  constexpr int JT = 4 * MT;
  int toks[JT];
#pragma unroll
  for (int jj = 0; jj < JT; ++jj) toks[jj] = 16 * (jj >> 2) + 4 * g + (jj & 3);
  EpiCol<JT> col;
  // staged epilogue: thread i of the workgroup finishes 4 consecutive outputs (token i / (RW / 4), rows
  // n0 + 4 (i % (RW / 4)) ..) for i = threadIdx.x, + 64 S, ...; its residual values are requested here,
  // with the other epilogue operands, instead of after the final barrier (where each was a round trip of
  // its own at the end of the kernel).  Whole 4-element groups of aligned residuals only, as raw words
  // through a buffer range (groups past the tile read zeros, no branches); the others load late.
  constexpr int RW = 16 * NT;
  constexpr int RI = STAGED ? (16 * MT * (RW / 4) + 64 * S - 1) / (64 * S) : 1;  // items per thread
  v4i rraw[RI];
  const bool rpre = STAGED && ep.res && ep.ldr % 4 == 0 &&
                    (uintptr_t)ep.res % (ep.res_dtype == WFB_F32 ? 16 : 8) == 0 &&
                    ((int64_t)(M - 1) * ep.ldr + N) * 4 < ((int64_t)1 << 32);  // uniform; range within 32 bits
  auto res_loads = [&]() {
    if constexpr (STAGED) {
      if (!rpre) return;
      const uint32_t esz = ep.res_dtype == WFB_F32 ? 4u : 2u;
      const uint32_t rbytes = (uint32_t)((int64_t)(M - 1) * ep.ldr + N) * esz;
      const buf_t rb = make_buf(ep.res, rbytes);
#pragma unroll
      for (int r = 0; r < RI; ++r) {
        const int i = threadIdx.x + 64 * S * r;
        const int tok = i / (RW / 4), n = n0 + 4 * (i % (RW / 4));
        const uint32_t off = tok < M && n + 3 < N ? (uint32_t)((int64_t)tok * ep.ldr + n) * esz : rbytes;
        if (esz == 4) {
          rraw[r] = buf_load16(rb, off);
        } else {
          const u32x2 h2 = __builtin_amdgcn_raw_buffer_load_b64(rb, off, 0, 0);
          rraw[r] = v4i{(int)h2[0], (int)h2[1], 0, 0};
        }
      }
    }
  };
  // gated epilogue operands (the gate and up rows' weight scales, and the token scales of the codes path),
  // requested with the others at entry rather than after the final barrier
  float gws[2] = {0.0f, 0.0f}, gas[GLUE != 0 && !NORM ? JT : 1];
  auto glu_loads = [&]() {
    if constexpr (GLUE != 0) {
      if (w < NT / 2) {
        const int n = n0 + 16 * w + nl;
        const int nc = n < half ? n : half - 1;  // (a column past the outputs stores nothing)
        gws[0] = epi_wscale(ep, nc);
        gws[1] = epi_wscale(ep, half + nc);
        if constexpr (!NORM) {
#pragma unroll
          for (int jj = 0; jj < JT; ++jj) gas[jj] = toks[jj] < M ? epi_ascale(ep, toks[jj]) : 0.0f;
        }
      }
    }
  };
  auto col_loads = [&]() {
    if (!GLUE && w < NT) {
      Epilogue e1 = ep;
      if (STAGED) e1.res = nullptr;  // the staged path adds the residual with whole-line loads
      col.load(e1, tile_row(w) + nl, N, toks, M);
    }
    glu_loads();
    res_loads();
  };
  float my_scale[RPW];
  // register-activation mode: lane (nl, g)'s 16 activation bytes of token tile mt, step pair u, step st,
  // field f -- step bytes 128 (g / 2) + 16 (g % 2) + 32 f of token 16 mt + nl (zeros past M and past K)
  v4i avr[XT == kAreg ? MT : 1][XT == kAreg ? TP : 1][2][4];
  if constexpr (XT == kAreg) {
    dma_weights();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int u = 0; u < TP; ++u)
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int f = 0; f < 4; ++f) {
            const int p = w + S * u;
            const int t = 2 * p + st;
            const int tr = 16 * mt + nl;
            const int qg = 8 * (g >> 1) + (g & 1) + 2 * f;
            const uint32_t kb = 256u * t + 16u * qg;
            const bool ok = p < T2 && t < T && tr < M && kb < (uint32_t)(64 * C);
            avr[mt][u][st][f] = buf_load16(ab, ok ? (uint32_t)((int64_t)tr * lda) + kb : a_end);
          }
    col_loads();
  } else if constexpr (XT == kNone) {
    dma_weights();
#pragma unroll
    for (int u = 0; u < TPA; ++u) dma_act(u, 0, STA);
    col_loads();
  } else {
    // 8 codes of token row r at k = e0 .. e0 + 7 into the staging: step t = e0 / 256 of pair t / 2, which
    // wave (t / 2) % S stages as its pair (t / 2) / S; 16-byte slot q of the step at q ^ (r & 15)
    auto put = [&](int r, int e0, uint32_t lo, uint32_t hi) {
      const int t = e0 >> 8, p = t >> 1, b = e0 & 255;
      int8_t* dst = al[p % S][p / S][t & 1] + 256 * r + 16 * ((b >> 4) ^ (r & 15)) + (b & 15);
      *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
    };
    auto between = [&]() { dma_weights(); };
    // the epilogue operands first: issued after the weight DMA (they load in waves w < NT only), the
    // prologue's wait for its row and gamma also covered DMA loads in those waves (loads complete in
    // issue order), and the prologue's barrier passed that wait on to every wave
    col_loads();
    // the whole staging: waves whose pairs lie past K read zeros (their sum(a) stays 0), as after the DMA
    constexpr int lim = 512 * S * TP;
    static_assert(lim <= 64 * 8 * 8, "the prologue's lanes cover 4096 elements");
    if (ns.gamma == nullptr)
      norm_prologue<S, MR, XT, kNone>(ns, M, w, lane, lim, put, between, my_scale);
    else if (ns.gdt == WFB_F32)
      norm_prologue<S, MR, XT, kF32>(ns, M, w, lane, lim, put, between, my_scale);
    else
      norm_prologue<S, MR, XT, kBf16>(ns, M, w, lane, lim, put, between, my_scale);
    __syncthreads();  // every wave's codes are in the staging
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's LDS-DMA loads have landed

  // ---- MFMA over the wave's step pairs -----------------------------------------------------------
  v4i acc1[MT][NT], acc4[MT][NT], acc16[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc1[mt][nt] = acc4[mt][nt] = acc16[mt][nt] = v4i{0, 0, 0, 0};
  int sa[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = 0;
  const int hh = nl >> 3, rr = nl & 7;
#pragma unroll
  for (int u = 0; u < TP; ++u) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      if constexpr (RS) {
        if ((u > 0 || st > 0) && st % STA == 0) {
          // the slot's previous unit has been read (its fragments are in registers) before it is refilled
          __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
          dma_act(u, st, st + STA);
          __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        }
      }
      v4i av[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (XT == kAreg) {
#pragma unroll
          for (int f = 0; f < 4; ++f) av[mt][f] = avr[mt][u][st][f];
        } else {
          // token row 16 mt + nl (its slots swizzled by nl); rows >= M hold zeros or unused codes
          const int tr = 16 * mt + nl;
          const int8_t* arow = aslot(u, st) + 256 * (tr < MR ? tr : MR - 1);
#pragma unroll
          for (int f = 0; f < 4; ++f) {
            const int qg = 8 * (g >> 1) + (g & 1) + 2 * f;  // step bytes 128 (g / 2) + 16 (g % 2) + 32 f
            av[mt][f] = *reinterpret_cast<const v4i*>(arow + 16 * (qg ^ nl));
          }
        }
      }
      const int slot = (4 * st + g) ^ (rr ^ hh);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const v4i wv = *reinterpret_cast<const v4i*>(wl[w][u][nt] + 1024 * hh + 128 * rr + 16 * slot);
        v4i b0, b1, b2, b3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = wv[e];
          b0[e] = (d >> 2) & 0x30303030;
          b1[e] = d & 0x30303030;
          b2[e] = d & 0x0C0C0C0C;
          b3[e] = d & 0x03030303;
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc16[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt][0], b0, acc16[mt][nt], 0, 0, 0);
          acc16[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt][1], b1, acc16[mt][nt], 0, 0, 0);
          acc4[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt][2], b2, acc4[mt][nt], 0, 0, 0);
          acc1[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt][3], b3, acc1[mt][nt], 0, 0, 0);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
          for (int e = 0; e < 4; ++e) sa[mt] = __builtin_amdgcn_sdot4(av[mt][f][e], 0x01010101, sa[mt], false);
    }
  }
  // C layout of a 16x16 tile: lane (nl, g) holds tokens 4g + j of weight row nl.  sum(a) of token nl over
  // this wave's K range: add the 4 lane groups, then fetch token 4g + j's from lane 4g + j.
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
        red(w, mt, nt, j, lane) = acc1[mt][nt][j] + (acc4[mt][nt][j] >> 2) + (acc16[mt][nt][j] >> 4) - sj;
    }
  }
  if constexpr (NORM) {
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < RPW; ++i)
        if (w + S * i < M) tok_scale(w + S * i) = my_scale[i];
    }
  }
  __syncthreads();
  if constexpr (NORM) {  // token scales from the prologue (ep.a_scale is not used)
#pragma unroll
    for (int jj = 0; jj < JT; ++jj) col.as[jj] = toks[jj] < M ? tok_scale(toks[jj]) : 0.0f;
  }

  // ---- epilogues -----------------------------------------------------------------------------------
  if constexpr (GLUE != 0) {
    if (w >= NT / 2) return;
    const int n = n0 + 16 * w + nl;  // output column = gate row; its up row is half + n
    if (n >= half) return;
    const float wsg = gws[0], wsu = gws[1];
#pragma unroll
    for (int jj = 0; jj < JT; ++jj) {
      const int tok = toks[jj], mt = jj >> 2, j = jj & 3;
      if (tok >= M) continue;
      int tg = red(0, mt, w, j, lane), tu = red(0, mt, w + NT / 2, j, lane);
#pragma unroll
      for (int k = 1; k < S; ++k) {
        tg += red(k, mt, w, j, lane);
        tu += red(k, mt, w + NT / 2, j, lane);
      }
      float as;
      if constexpr (NORM) as = col.as[jj];
      else as = gas[jj];
      float yg = __fmul_rn(__fmul_rn((float)tg, wsg), as), yu = __fmul_rn(__fmul_rn((float)tu, wsu), as);
      if (ep.mid_dtype == WFB_BF16) {
        yg = bf16_bits_to_f32(f32_to_bf16_rne(yg));
        yu = bf16_bits_to_f32(f32_to_bf16_rne(yu));
      }
      reinterpret_cast<float*>(ep.out)[(int64_t)tok * ep.ldo + n] = glu<GLUE>(yg, yu);
    }
    return;
  } else if constexpr (!STAGED) {
    if (w >= NT) return;
    const int nt = w;
    const int n = n0 + 16 * nt + nl;
    if (ep.amax) {  // greedy-argmax keys: the maximum over the 16 rows of each token, one slot per 16 rows
#pragma unroll
      for (int jj = 0; jj < JT; ++jj) {
        const int tok = toks[jj], mt = jj >> 2, j = jj & 3;
        int tot = red(0, mt, nt, j, lane);
#pragma unroll
        for (int k = 1; k < S; ++k) tot += red(k, mt, nt, j, lane);
        const bool valid = tok < M && n < N;
        uint64_t key = epi_store_key_r(ep, col.ws, col.as[jj], col.bias, col.res[jj], tok, n, tot, valid);
        key = group_max_u64<16>(key);
        const int slot = blockIdx.x * NT + nt;
        if (nl == 0 && tok < M && slot < (N + 15) / 16) ep.amax[(int64_t)slot * (ep.amax_ld ? ep.amax_ld : M) + tok] = key;
      }
      return;
    }
    if (n >= N) return;
#pragma unroll
    for (int jj = 0; jj < JT; ++jj) {
      const int tok = toks[jj], mt = jj >> 2, j = jj & 3;
      int tot = red(0, mt, nt, j, lane);
#pragma unroll
      for (int k = 1; k < S; ++k) tot += red(k, mt, nt, j, lane);
      if (tok < M) epi_store_r(ep, col.ws, col.as[jj], col.bias, col.res[jj], tok, n, tot);
    }
  } else {
    // y (fp32, before the residual) of the [M tokens x 16 NT rows] tile into LDS (the activation staging),
    // rows rotated by 4 per token to spread the banks
    float* ys = XT == kAreg ? ysb : reinterpret_cast<float*>(&al[0][0][0][0]);  // free after the barrier above
    static_assert(XT == kAreg || sizeof(al) >= 16 * MT * RW * 4, "staging space");
    if (w < NT) {
      const int c = 16 * w + nl;
#pragma unroll
      for (int jj = 0; jj < JT; ++jj) {
        const int tok = toks[jj], mt = jj >> 2, j = jj & 3;
        int tot = red(0, mt, w, j, lane);
#pragma unroll
        for (int k = 1; k < S; ++k) tot += red(k, mt, w, j, lane);
        ys[tok * RW + ((c + 4 * tok) & (RW - 1))] = epi_y(ep, col.ws, col.as[jj], col.bias, tot);
      }
    }
    __syncthreads();
    const bool out_vec = ep.ldo % 4 == 0 && (uintptr_t)ep.out % (ep.out_dtype == WFB_F32 ? 16 : 8) == 0;
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      const int i = threadIdx.x + 64 * S * r;
      const int tok = i / (RW / 4), q = i % (RW / 4);
      const int n = n0 + 4 * q;
      if (tok >= M || n >= N) continue;
      const bool full = n + 3 < N;
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = ys[tok * RW + ((4 * q + e + 4 * tok) & (RW - 1))];
      if (ep.res) {
        float rv[4];
        if (rpre && full) {  // requested at kernel entry
          if (ep.res_dtype == WFB_F32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) rv[e] = __int_as_float(rraw[r][e]);
          } else {
            const uint32_t x0 = (uint32_t)rraw[r][0], x1 = (uint32_t)rraw[r][1];
            rv[0] = __uint_as_float(x0 << 16); rv[1] = __uint_as_float(x0 & 0xffff0000u);
            rv[2] = __uint_as_float(x1 << 16); rv[3] = __uint_as_float(x1 & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) rv[e] = n + e < N ? epi_res(ep, tok, n + e) : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = __fadd_rn(y[e], rv[e]);
      }
      const int64_t off = (int64_t)tok * ep.ldo + n;
      if (ep.out_dtype == WFB_F32) {
        float* o = reinterpret_cast<float*>(ep.out) + off;
        if (full && out_vec) *reinterpret_cast<float4*>(o) = make_float4(y[0], y[1], y[2], y[3]);
        else
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) o[e] = y[e];
      } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(ep.out) + off;
        if (full && out_vec) {
          const bf16x2_t lo = __builtin_convertvector((f32x2_t){y[0], y[1]}, bf16x2_t);
          const bf16x2_t hi = __builtin_convertvector((f32x2_t){y[2], y[3]}, bf16x2_t);
          *reinterpret_cast<uint2*>(o) = make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) o[e] = f32_to_bf16_rne(y[e]);
        }
      }
    }
  }
}

// Persistent form for outputs of many row tiles (the LM head: 128256 rows = 4008 tiles of 32), codes
// path, one weight scale, no bias or residual, per-lane epilogues (greedy-argmax keys, accumulator copies,
// per-lane stores).  One workgroup per CU loops over tiles t = blockIdx.x, + gridDim.x, ...  The
// activation fragments and token scales are loaded once into registers (they are the same for every
// tile), so the LDS holds only weights: a ring of DEPTH tile buffers, DEPTH - 1 tiles' weight DMA in
// flight while one tile is multiplied, reduced and stored -- about 128 KB per CU at K = 4096, what the M = 1
// GEMV keeps in flight to stream at ~6.4 TB/s.  TP = 1 (K <= 4096).  Same operand layouts and arithmetic
// as the one-shot kernel.
// Waits: a tile's DMA is waited for with vmcnt(DMA instructions issued after it).  Loads complete in issue
// order, so that count is exact for them; stores may complete before earlier loads on this part, so the
// epilogue's stores are left out of the count (counting them let a wait pass with the tile's DMA still
// in flight) -- a store still outstanding can only make the wait longer.
// Every LDS access of the loop is inline asm (with its own lgkmcnt wait): the compiler, which cannot tell
// the ring slots from the other LDS, otherwise waits for every outstanding LDS DMA (vmcnt(0)) before each
// LDS read, which drains the ring on every tile (measured: 35.0 -> 26.5 us for the Llama-3-8B head at M = 8).
template <int OPS>
__device__ __forceinline__ void wait_tiles_after(int later) {
  // vmcnt(n) with expcnt / lgkmcnt at their maxima (gfx9: vmcnt bits 3:0 and 15:14)
#define WFB_VMCNT(nn) __builtin_amdgcn_s_waitcnt(((nn) & 15) | (((nn) >> 4) << 14) | (7 << 4) | (15 << 8))
  switch (later) {
    case 0: WFB_VMCNT(0); break;
    case 1: WFB_VMCNT(OPS); break;
    case 2: WFB_VMCNT(2 * OPS); break;
    case 3: WFB_VMCNT(3 * OPS); break;
    case 4: WFB_VMCNT(4 * OPS); break;
    case 5: WFB_VMCNT(5 * OPS); break;
    case 6: WFB_VMCNT(6 * OPS); break;
    default: WFB_VMCNT(7 * OPS); break;
  }
#undef WFB_VMCNT
}

// LDS offset of a pointer into __shared__ memory (the low 32 bits of its flat address)
__device__ __forceinline__ uint32_t lds_off(const void* p) { return (uint32_t)(uintptr_t)p; }

// Sum of the S int32 partial tiles 2048 bytes apart from LDS offset a (one wait; integer sums, so the
// order is immaterial).
template <int S>
__device__ __forceinline__ int lds_sum_parts(uint32_t a) {
  int t[8];
  if constexpr (S == 8) {
    asm volatile(
        "ds_read_b32 %0, %8\n\tds_read_b32 %1, %8 offset:2048\n\tds_read_b32 %2, %8 offset:4096\n\t"
        "ds_read_b32 %3, %8 offset:6144\n\tds_read_b32 %4, %8 offset:8192\n\tds_read_b32 %5, %8 offset:10240\n\t"
        "ds_read_b32 %6, %8 offset:12288\n\tds_read_b32 %7, %8 offset:14336\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7])
        : "v"(a)
        : "memory");
    return t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];
  } else if constexpr (S == 5) {
    asm volatile(
        "ds_read_b32 %0, %5\n\tds_read_b32 %1, %5 offset:2048\n\tds_read_b32 %2, %5 offset:4096\n\t"
        "ds_read_b32 %3, %5 offset:6144\n\tds_read_b32 %4, %5 offset:8192\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4])
        : "v"(a)
        : "memory");
    return t[0] + t[1] + t[2] + t[3] + t[4];
  } else if constexpr (S == 4) {
    asm volatile(
        "ds_read_b32 %0, %4\n\tds_read_b32 %1, %4 offset:2048\n\tds_read_b32 %2, %4 offset:4096\n\t"
        "ds_read_b32 %3, %4 offset:6144\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3])
        : "v"(a)
        : "memory");
    return t[0] + t[1] + t[2] + t[3];
  } else {
    static_assert(S == 2, "S in {2, 4, 5, 8}");
    asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %2 offset:2048\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(t[0]), "=&v"(t[1])
                 : "v"(a)
                 : "memory");
    return t[0] + t[1];
  }
}

// KO (keys only: greedy-argmax keys and no other output): each lane's key goes out as one buffer store,
// lanes with nothing to store pointing past the key buffer (which drops the store).
template <int S, int NT, int DEPTH, bool KO>
__global__ __launch_bounds__(64 * S) void kernel_persist(const uint8_t* __restrict__ W, const int8_t* __restrict__ A,
                                                         int64_t lda, int M, int N, int C, int ntiles, Epilogue ep) {
  static_assert(DEPTH >= 2 && DEPTH <= 8 && 7 * 2 * NT < 64, "ring depth and vmcnt range");
  static_assert(NT == 2, "partial tiles 2048 bytes apart, four fragment reads per tile");
  constexpr int OPS = 2 * NT;  // LDS-DMA instructions of one tile's weights (per wave)
  __shared__ __attribute__((aligned(16))) int8_t wl[DEPTH][S][NT][2048];
  // partial tiles, double-buffered by tile parity: a wave only ever refills its own weight slot (program
  // order protects it), and a parity buffer is rewritten two tiles later, after a barrier every wave
  // passes only once done with the epilogue that read it -- one barrier per tile
  __shared__ __attribute__((aligned(16))) int redb[2][S][NT * 4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const uint32_t row_bytes = (uint32_t)C * 16;
  const uint32_t w_end = (uint32_t)N * row_bytes, a_end = (uint32_t)((int64_t)(M - 1) * lda + (int64_t)C * 64);
  const buf_t wb = make_buf(W, w_end);
  const buf_t ab = make_buf(A, a_end);
  const int T = (C + 3) >> 2, T2 = (C + 7) >> 3;
  const int p = w;  // this wave's step pair (TP = 1)

  // activation fragments of token nl over this wave's pair: the 16 bytes the MFMA takes from lane (nl, g)
  // (step bytes 128 (g / 2) + 16 (g % 2) + 32 f); tokens past M and bytes past K read as zeros
  v4i av[2][4];
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const int t = 2 * p + st;
      const int qg = 8 * (g >> 1) + (g & 1) + 2 * f;
      const uint32_t kb = 256u * t + 16u * qg;
      const bool ok = p < T2 && t < T && nl < M && kb < (uint32_t)(64 * C);
      av[st][f] = buf_load16(ab, ok ? (uint32_t)((int64_t)nl * lda) + kb : a_end);
    }
  // token scales of the four tokens this lane stores, and the weight scale (one segment)
  float as[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) as[j] = 4 * g + j < M ? epi_ascale(ep, 4 * g + j) : 0.0f;
  const float ws = ep.ws_dev ? ep.ws_dev[0] : ep.ws;
  // (keys only) the key buffer: slots of 16 rows x ld tokens
  const int nslots = (N + 15) / 16;
  const int ldk = ep.amax_ld ? ep.amax_ld : M;
  const uint32_t kbytes = (uint32_t)(nslots * ldk) * 8u;
  const buf_t kbuf = make_buf(ep.amax, KO ? kbytes : 0u);
  const bool key_bf16 = ep.amax_dt == WFB_BF16;

  auto dma = [&](int tile, int buf) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = lane >> 3;
        const int chunk = 8 * p + ((lane & 7) ^ (r ^ h));
        const int row = tile * 16 * NT + 16 * nt + 8 * h + r;
        const bool ok = p < T2 && chunk < C;
        dma16(wb, wl[buf][w][nt] + 1024 * h, ok ? (uint32_t)row * row_bytes + 16u * chunk : w_end);
      }
  };
#pragma unroll
  for (int i = 0; i < DEPTH - 1; ++i) {
    const int t = blockIdx.x + i * gridDim.x;
    if (t < ntiles) dma(t, i);
  }

  // sum(a) of token 4g + j over this wave's K range (the same for every tile)
  int sj[4];
  {
    int sa = 0;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int e = 0; e < 4; ++e) sa = __builtin_amdgcn_sdot4(av[st][f][e], 0x01010101, sa, false);
    sa += xor_lanes<16>(sa);
    sa += xor_lanes<32>(sa);
#pragma unroll
    for (int j = 0; j < 4; ++j) sj[j] = __shfl(sa, 4 * g + j, 64);
  }
  const int hh = nl >> 3, rr = nl & 7;

  for (int it = 0;; ++it) {
    const int tile = blockIdx.x + it * gridDim.x;
    if (tile >= ntiles) break;
    const int buf = it % DEPTH;
    const int ahead = blockIdx.x + (it + DEPTH - 1) * gridDim.x;
    if (ahead < ntiles) dma(ahead, (it + DEPTH - 1) % DEPTH);  // slot last read by this wave, for tile it - 1
    const int later = min(DEPTH - 1, (ntiles - 1 - tile) / (int)gridDim.x);
    wait_tiles_after<OPS>(later);

    // the wave's four weight fragments (steps 0 / 1 x row tiles 0 / 1), one wait
    v4i wv[2][NT];
    {
      const int8_t* base = &wl[buf][w][0][0] + 1024 * hh + 128 * rr;
      const int s0 = g ^ (rr ^ hh), s1 = (4 + g) ^ (rr ^ hh);
      asm volatile(
          "ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\tds_read_b128 %3, %7\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(wv[0][0]), "=&v"(wv[0][1]), "=&v"(wv[1][0]), "=&v"(wv[1][1])
          : "v"(lds_off(base + 16 * s0)), "v"(lds_off(base + 2048 + 16 * s0)), "v"(lds_off(base + 16 * s1)),
            "v"(lds_off(base + 2048 + 16 * s1))
          : "memory");
    }
    v4i acc1[NT], acc4[NT], acc16[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc1[nt] = acc4[nt] = acc16[nt] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        v4i b0, b1, b2, b3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = wv[st][nt][e];
          b0[e] = (d >> 2) & 0x30303030;
          b1[e] = d & 0x30303030;
          b2[e] = d & 0x0C0C0C0C;
          b3[e] = d & 0x03030303;
        }
        acc16[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[st][0], b0, acc16[nt], 0, 0, 0);
        acc16[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[st][1], b1, acc16[nt], 0, 0, 0);
        acc4[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[st][2], b2, acc4[nt], 0, 0, 0);
        acc1[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[st][3], b3, acc1[nt], 0, 0, 0);
      }
    const int par = it & 1;
    {
      // partial (nt, j) of this wave at redb[par][w][nt * 4 + j][lane] (256 bytes apart), then the barrier
      int v[NT * 4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          v[nt * 4 + j] = acc1[nt][j] + (acc4[nt][j] >> 2) + (acc16[nt][j] >> 4) - sj[j];
      asm volatile(
          "ds_write_b32 %0, %1\n\tds_write_b32 %0, %2 offset:256\n\tds_write_b32 %0, %3 offset:512\n\t"
          "ds_write_b32 %0, %4 offset:768\n\tds_write_b32 %0, %5 offset:1024\n\tds_write_b32 %0, %6 offset:1280\n\t"
          "ds_write_b32 %0, %7 offset:1536\n\tds_write_b32 %0, %8 offset:1792\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier"
          :
          : "v"(lds_off(&redb[par][w][0][lane])), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]),
            "v"(v[6]), "v"(v[7])
          : "memory");
    }
    // epilogue spread over the waves: (row tile nt, token slot j) pairs c = w, w + S, ...; lane (nl, g)
    // finishes row 16 nt + nl of token 4g + j
    for (int c = w; c < NT * 4; c += S) {
      const int nt = c >> 2, j = c & 3;
      const int tok = 4 * g + j;
      const int n = tile * 16 * NT + 16 * nt + nl;
      const int tot = lds_sum_parts<S>(lds_off(&redb[par][0][c][lane]));
      // (selects, not an indexed array: the compiler would place that in LDS, where each read would wait for
      // the ring's DMA)
      const float a = (j & 2) ? ((j & 1) ? as[3] : as[2]) : ((j & 1) ? as[1] : as[0]);
      if constexpr (KO) {
        const bool valid = tok < M && n < N;
        const float y = epi_y(ep, ws, a, 0.0f, tot);
        const float yk = key_bf16 ? bf16_bits_to_f32(f32_to_bf16_rne(y)) : y;
        uint64_t key = valid ? amax_key(yk, n) : 0;
        key = group_max_u64<16>(key);
        const int slot = tile * NT + nt;
        const bool st = nl == 0 && tok < M && slot < nslots;
        const u32x2 kv = {(uint32_t)key, (uint32_t)(key >> 32)};
        __builtin_amdgcn_raw_buffer_store_b64(kv, kbuf, st ? (uint32_t)(slot * ldk + tok) * 8u : kbytes, 0, 0);
      } else if (ep.amax) {  // greedy-argmax keys with other outputs: the maximum over the 16 rows of each token
        const bool valid = tok < M && n < N;
        uint64_t key = epi_store_key_r(ep, ws, a, 0.0f, 0.0f, tok, n, tot, valid);
        key = group_max_u64<16>(key);
        const int slot = tile * NT + nt;
        if (nl == 0 && tok < M && slot < nslots) ep.amax[(int64_t)slot * ldk + tok] = key;
      } else if (n < N && tok < M) {
        epi_store_r(ep, ws, a, 0.0f, 0.0f, tok, n, tot);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): nothing of this wave in flight at exit
}

// Persistent launch for grids of many tiles: two 16-row tiles per workgroup step, the ring as deep as the
// LDS allows (at most 8); hipErrorNotSupported where it does not apply (the caller then takes the one-shot
// kernel).
inline hipError_t launch_persist(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda,
                                 const Epilogue& e, int cus, hipStream_t s) {
  constexpr int NT = 2;
  const int T2 = (C + 7) / 8;
  const int ntiles = (n + 16 * NT - 1) / (16 * NT);
  const int grid = ntiles < cus ? ntiles : cus;
#define WFB_SL_P(S)                                                                                    \
  do {                                                                                                 \
    constexpr int D = (163840 - 2 * S * NT * 1024) / (S * NT * 2048) > 8 ? 8                          \
                                                                        : (163840 - 2 * S * NT * 1024) / (S * NT * 2048); \
    if (e.amax && !e.out && !e.acc_out &&                                                              \
        (int64_t)((n + 15) / 16) * (e.amax_ld ? e.amax_ld : m) * 8 < ((int64_t)1 << 32))                 \
      hipLaunchKernelGGL((kernel_persist<S, NT, D, true>), dim3(grid), dim3(64 * S), 0, s, W, A, lda, m, n, C, ntiles, e); \
    else                                                                                               \
      hipLaunchKernelGGL((kernel_persist<S, NT, D, false>), dim3(grid), dim3(64 * S), 0, s, W, A, lda, m, n, C, ntiles, e); \
    return hipGetLastError();                                                                          \
  } while (0)
  if (T2 <= 2) WFB_SL_P(2);
  if (T2 <= 4) WFB_SL_P(4);
  if (T2 <= 5) WFB_SL_P(5);
  if (T2 <= 8) WFB_SL_P(8);
#undef WFB_SL_P
  return hipErrorNotSupported;
}

// Shapes whose multi-token-tile forms stay within the registers of their occupancy (more row tiles or
// step pairs per wave spill): two tiles (MR = 32) with NT * S <= 20, four (MR = 64) with one row tile
// and one step pair per wave.
constexpr bool fits_tiles(int MR, int S, int NT, int TP) { return MR <= 16 || (MR == 32 ? NT * S <= 20 : NT == 1 && TP == 1); }

// (S, TP) by the number of 512-weight step pairs T2 = ceil(K / 512): S = T2 waves up to 8 (K = 2560: 5,
// K = 4096: 8, from sweeps), two pairs per wave up to 16 pairs, then 14 x 2 (K <= 14336, LDS permitting).
// XT = kF32 / kBf16: the norm prologue on x of that storage tag (K <= 4096); kAreg: codes A held in
// registers (rows whose activations do not fit the LDS beside the weights).
template <int MR, int GLUE, int XT>
hipError_t launch(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda, const Epilogue& e, int nt_pref,
                  const NormSrc& ns, hipStream_t s) {
  const int T2 = (C + 7) / 8;
  const bool staged = GLUE == 0 && e.out && !e.acc_out && !e.amax;
  // two-tile form over more than 32 tokens: one grid row of workgroups per 32 tokens (no argmax keys)
  const unsigned tblocks = MR == 32 && XT == kNone && m > 32 ? (unsigned)((m + 31) / 32) : 1u;
  if (tblocks > 1 && e.amax) return hipErrorNotSupported;
#define WFB_SL_GO(S, NT, TP)                                                                                   \
  do {                                                                                                         \
    if constexpr ((XT == kAreg ? lds_bytes_areg(S, NT, TP, (MR + 15) / 16) : lds_bytes(S, NT, TP, MR)) <= 163840 && \
                  (GLUE ? NT / 2 : NT) <= S && fits_tiles(MR, S, NT, TP)) {                    \
      const dim3 grid(GLUE ? (n / 2 + 8 * NT - 1) / (8 * NT) : (n + 16 * NT - 1) / (16 * NT), tblocks);        \
      if (GLUE == 0 && staged)                                                                                 \
        hipLaunchKernelGGL((kernel<S, NT, TP, MR, GLUE, GLUE == 0, XT>), grid, dim3(64 * S), 0, s, W, A, lda, m, n, \
                           C, e, ns);                                                                          \
      else                                                                                                     \
        hipLaunchKernelGGL((kernel<S, NT, TP, MR, GLUE, false, XT>), grid, dim3(64 * S), 0, s, W, A, lda, m, n, \
                           C, e, ns);                                                                          \
      return hipGetLastError();                                                                                \
    }                                                                                                          \
  } while (0)
#define WFB_SL_NT(S, TP)                                         \
  do {                                                           \
    if (nt_pref >= 8) WFB_SL_GO(S, 8, TP);                       \
    if (nt_pref >= 4) WFB_SL_GO(S, 4, TP);                       \
    if constexpr (GLUE != 0) {                                   \
      WFB_SL_GO(S, 2, TP);                                       \
    } else {                                                     \
      if constexpr (XT != kNone) if (nt_pref >= 2) WFB_SL_GO(S, 2, TP); \
      WFB_SL_GO(S, 1, TP);                                       \
    }                                                            \
    return hipErrorNotSupported;                                 \
  } while (0)
  // the register-activation mode serves the long rows below, and 64 tokens on rows past the staging
  if constexpr (XT != kAreg || MR == 64) {
    if (T2 <= 2) WFB_SL_NT(2, 1);
    if (T2 <= 4) WFB_SL_NT(4, 1);
    if (T2 <= 5) WFB_SL_NT(5, 1);
    if (T2 <= 8) WFB_SL_NT(8, 1);
  }
  if constexpr ((XT == kNone || XT == kAreg) && MR != 64) {
    if (T2 <= 14) WFB_SL_NT(7, 2);
    if (T2 <= 16) WFB_SL_NT(8, 2);
    if (T2 <= 28) WFB_SL_NT(14, 2);
  }
#undef WFB_SL_NT
#undef WFB_SL_GO
  return hipErrorNotSupported;
}

// Rows from which the persistent form is used: 2048 tiles of 16 rows (8 per CU at NT = 4, four
// one-workgroup-per-CU rounds of the one-shot kernel).
constexpr int kPersistMinRows = 32768;

// Compute units of the current device (cached per device).
inline int cu_count() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev] = v;
  }
  return cache[dev];
}

// The three modes of one staged token-row count: codes A (x null), or the norm prologue on bf16 / fp32 x.
template <int MR, int GLUE>
hipError_t launch_modes(const uint8_t* W, int n, int C, const int8_t* A, int m, int64_t lda, const Epilogue& e,
                        int nt_pref, const NormSrc& ns, hipStream_t s) {
  if (ns.x == nullptr) {
    if (A == nullptr) return hipErrorInvalidValue;
    // many row tiles with a per-lane epilogue (the greedy LM head): the persistent form (one token tile)
    if constexpr (MR <= 16) {
      if (GLUE == 0 && (e.amax || e.acc_out || !e.out) && !e.bias && !e.res && e.nseg == 1 && n >= kPersistMinRows) {
        const hipError_t st = launch_persist(W, n, C, A, m, lda, e, cu_count(), s);
        if (st != hipErrorNotSupported) return st;
      }
    }
    const hipError_t st = launch<MR, GLUE, kNone>(W, n, C, A, m, lda, e, nt_pref, ns, s);
    if constexpr (GLUE == 0 && MR != 32) {  // activations too long for the LDS beside the weights: in registers
      if (st == hipErrorNotSupported) return launch<MR, GLUE, kAreg>(W, n, C, A, m, lda, e, nt_pref, ns, s);
    }
    return st;
  }
  if constexpr (MR > 16) {  // the norm prologue serves one token tile
    return hipErrorNotSupported;
  } else {
    if (C > 64 || ns.h > 64 * C || (ns.xdt != WFB_F32 && ns.xdt != WFB_BF16)) return hipErrorInvalidValue;
    if (src_tag(ns.xdt) == kF32) return launch<MR, GLUE, kF32>(W, n, C, A, m, lda, e, nt_pref, ns, s);
    return launch<MR, GLUE, kBf16>(W, n, C, A, m, lda, e, nt_pref, ns, s);
  }
}

}  // namespace skinny_lds
}  // namespace wfb
