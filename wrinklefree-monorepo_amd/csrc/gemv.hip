// Decode GEMV for the I2_S ternary BitLinear (M <= 2 tokens): VALU sdot4 + DPP reductions, no MFMA.
//
// Replaces bitnet_vec_dot_i2_i8 / bitnet_gemv_cpu
// (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:325-808, SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:331-367):
//   acc[n] = sum_k code(W[n,k]) * a[k] - sum_k a[k] = sum_k w[n,k] * a[k].
//
// Work mapping (wave64).  A row of K weights is C = K/64 chunks of 16 packed bytes; each chunk is
// read with one 128-bit load and pairs with 4 x 16 activation bytes (one per 2-bit field).
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
//
// Norm prologue (XDT >= 0, rows longer than 4096): the workgroup forms the int8 codes of its M rows
// itself from the float rows x (RMSNorm/SubLN + per-token absmax quantisation) into LDS and reads its
// activation fragments from there -- bit for bit wfb_rmsnorm_quant_i8's codes and scales, because
// threads 0..255 run that quantiser's own 256-thread path (quant_rows.h) on each row.
#include "quant_rows.h"

namespace wfb {

namespace {

// Split-K GEMV.  A workgroup owns RB = RP * (64/L) consecutive weight rows and all of K; its S waves
// split K into S ranges of L*CPL chunks.  In a wave, L lanes share a row: lane s of a row group owns
// chunks kc0 + s + L*i (i < CPL) and keeps the activations of those chunks in registers for all RP
// row passes, so each activation byte is fetched once per wave and reused for 64/L * RP rows.
// Loads go through raw buffer descriptors: rows past N read as zeros, so nothing is masked when the
// chunk ranges tile K exactly (EXACT); otherwise chunks past K are zeroed explicitly.
// Load order: the activations of the lane's chunks and the bytes of its sum(a) slice first (L2 hits),
// then all weight loads of the wave (RP*CPL x 16 B per lane), so pass p's arithmetic waits only for its own
// weights (measured on MI355X: 2560x6912 and 6144x4096 4.05 -> 3.6-3.7 us against weights first).
// The code offset is removed with the wave's sum(a).
// Per pass, each row's partial is reduced over its L lanes with DPP and parked in LDS; after one
// barrier the first RB threads add the S partials of their row and store it (one coalesced store
// per token).
__device__ __forceinline__ int wave_sum(int v) {
  return group_sum<64>(v);
}

template <int M, int L, int CPL, int RP, int S, bool EXACT, bool PRE, int XDT = -1, bool STAGE = true, int GLU = 0>
__global__ __launch_bounds__(64 * S) void gemv_i2s_kernel(const uint8_t* __restrict__ W,
                                                          const int8_t* __restrict__ A, int64_t lda, int N,
                                                          int C, Epilogue ep, NormSrc ns) {
  constexpr int RPG = 64 / L;  // rows per pass
  constexpr int RB = RP * RPG; // rows per workgroup
  constexpr bool NORM = XDT >= 0;
  constexpr int KMAX = 64 * L * CPL * S;  // the longest row the launch shape covers
  static_assert(RB <= 64 * S, "one thread per row in the epilogue");
  static_assert(GLU == 0 || (!PRE && RB % 2 == 0), "gated rows load their epilogue operands late");
  static_assert(!NORM || S >= kTPB / 64 || KMAX <= kWaveMaxH, "rows past 4096 elements take the 256-thread order");
  __shared__ int red[S][M][RB];
  // norm prologue (one row): the row's elements, its codes and scale, the per-wave partials
  static_assert(!NORM || M == 1, "the norm prologue takes one row");
  __shared__ __attribute__((aligned(16))) float xs[NORM ? KMAX : 4];
  __shared__ __attribute__((aligned(16))) int8_t codes[1][NORM ? KMAX : 16];
  __shared__ float nscale[1], nred[kTPB / 64], mred[S];
  constexpr int XA = 64 * L * CPL;  // activation bytes of a wave's K range, per token
  constexpr bool XS = !NORM && STAGE;
  __shared__ __attribute__((aligned(16))) int8_t xa[XS ? S : 1][XS ? M : 1][XS ? XA : 16];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int r_in = lane / L, s = lane % L;
  const int t = threadIdx.x;
  const uint32_t row_bytes = (uint32_t)C * 16;
  const int row0 = blockIdx.x * RB;
  const int kc0 = w * (L * CPL);
  const buf_t wb = make_buf(W, (uint32_t)N * row_bytes);
  const buf_t ab = make_buf(A, NORM ? 0u : (uint32_t)((M - 1) * lda + (int64_t)C * 64));

  // norm prologue, first part: every thread loads its 8-element chunks of the row (chunks t + 64*S*j;
  // zeros past h) and the same elements of gamma, all issued before the weights: loads complete in issue
  // order, so a gamma load issued after the weights would hold the whole prologue until they arrived.
  // gamma is read as 32 raw bytes per chunk whatever its dtype (a bf16 chunk uses the first 16; a null
  // gamma reads zeros from an empty descriptor), so every path issues the same loads.
  constexpr int PCH = NORM ? KMAX / (kVec * 64 * S) : 1;  // chunks per thread (2 for 16 lanes x 1 chunk)
  static_assert(!NORM || PCH * kVec * 64 * S == KMAX, "chunks tile the row");
  float xv[PCH][kVec];
  v4i graw[PCH][2];
  if constexpr (NORM) {
    const buf_t xb = row_buf<XDT>(ns.x, ns.h);
#pragma unroll
    for (int j = 0; j < PCH; ++j) load_row8_full<XDT, 0>(xb, xb, (t + j * 64 * S) * kVec, xv[j]);
    const uint32_t gsz = ns.gdt == WFB_F32 ? 4u : 2u;
    const buf_t gb = make_buf(ns.gamma, ns.gamma ? (uint32_t)ns.h * gsz : 0u);
#pragma unroll
    for (int j = 0; j < PCH; ++j) {
      const uint32_t off = (uint32_t)((t + j * 64 * S) * kVec) * gsz;
      graw[j][0] = buf_load16(gb, off);
      graw[j][1] = buf_load16(gb, off + 16);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the weight loads
  }

  // a[m][i][q] = a_m[128b + 32q + j0 .. +15] for chunk c (b = c/2, j0 = 16*(c%2))
  v4i a[M][CPL][4];
  constexpr int SB = (L * CPL + 15) / 16;  // 16-byte pieces per lane (L*CPL = 8: one 8-byte piece)
  v4i sv[M][SB];
  if constexpr (!NORM && !STAGE) {
    // grids of many rounds: the fragments of the lane's chunks straight from global memory
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = kc0 + s + L * i;
        const uint32_t off = (uint32_t)(m * lda) + 128 * (c >> 1) + 16 * (c & 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          a[m][i][q] = buf_load16(ab, off + 32 * q);
          if (!EXACT && c >= C) a[m][i][q] = v4i{0, 0, 0, 0};
        }
      }
  }
  if constexpr (!NORM) {
    // the wave's activation slice (bytes 64*kc0 .. 64*(kc0 + L*CPL) of each token row), one piece per
    // lane: summed for sum(a) and (STAGE) copied into the wave's LDS slice, from which the chunk fragments
    // are read.  Loading the fragments from global memory instead -- every lane of a row group 4 x 16
    // bytes of the same few lines, in every workgroup -- measured 0.5 us slower at 13824x2560 (864
    // workgroups) on MI355X, the staging 5% slower at 128256x4096 (4008 workgroups, many rounds).
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint32_t boff = (uint32_t)(64 * kc0 + lane * (L * CPL));
      const bool in = EXACT || boff < (uint32_t)(64 * C);
      const uint32_t off = (uint32_t)(m * lda) + boff;
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        if constexpr (L * CPL == 8) {
          const auto v = __builtin_amdgcn_raw_buffer_load_b64(ab, in ? (int)off : 0x7FFFFFF0, 0, 0);
          sv[m][b] = v4i{(int)v[0], (int)v[1], 0, 0};
        } else {
          sv[m][b] = buf_load16(ab, in ? off + 16 * b : 0xFFFFFFF0u);
        }
      }
    }
  }
  // then the weights of every pass (the activation loads, L2 hits, go first so that pass p's arithmetic
  // waits only for its own weight loads -- loads return in issue order)
  v4i wv[RP][CPL];
#pragma unroll
  for (int p = 0; p < RP; ++p) {
    // GLU: local rows 0 .. RB/2-1 are gate rows b*RB/2 + i, the others their up rows N/2 + b*RB/2 + i
    const int lr = p * RPG + r_in;
    const int wr = GLU == 0 ? row0 + lr : lr < RB / 2 ? blockIdx.x * (RB / 2) + lr : N / 2 + blockIdx.x * (RB / 2) + lr - RB / 2;
    const uint32_t rowoff = (uint32_t)wr * row_bytes;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = kc0 + s + L * i;
      wv[p][i] = buf_load16<kLoadNT>(wb, rowoff + 16 * c);
      if (!EXACT && c >= C) wv[p][i] = v4i{0, 0, 0, 0};
    }
  }
  // Epilogue operands of the row this thread stores (thread t < RB stores row row0 + t): loaded below,
  // behind the weight loads (PRE), or after the final barrier.  With the activation-first load order,
  // loading them early measured faster on every BitNet-2B and Llama-3-8B shape (13824x2560 4.39 -> 4.23 us,
  // 28672x4096 7.30 -> 7.08).
  const int n = row0 + t;
  int toks[M];
#pragma unroll
  for (int m = 0; m < M; ++m) toks[m] = m;
  EpiCol<M> col;

  if constexpr (!NORM && STAGE) {
    // the slice into the wave's LDS (waits only for the slice loads, issued before the weights), then the
    // fragments of the lane's chunks; writer and readers are lanes of one wave
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        if constexpr (L * CPL == 8)
          *reinterpret_cast<uint2*>(&xa[w][m][lane * 8]) = make_uint2((uint32_t)sv[m][b][0], (uint32_t)sv[m][b][1]);
        else
          *reinterpret_cast<v4i*>(&xa[w][m][lane * (L * CPL) + 16 * b]) = sv[m][b];
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = kc0 + s + L * i;
        const int off = 128 * ((c - kc0) >> 1) + 16 * (c & 1);  // kc0 is even
#pragma unroll
        for (int q = 0; q < 4; ++q) a[m][i][q] = *reinterpret_cast<const v4i*>(&xa[w][m][off + 32 * q]);
      }
  }
  // issued after the slice copy (or after the norm prologue): issued before it, the copy's or the
  // prologue's wait for its own loads also covered weight loads in the storing wave (its counter holds
  // these loads too), and the prologue's barriers pass that wait on to every wave
  if (!NORM && PRE && t < RB) col.load_raw(ep, n, N, toks, M);

  if constexpr (NORM) {
    // norm prologue, second part: wfb_rmsnorm_quant_i8's summation order for the row length -- rows of up
    // to 4096 elements its one-wave path (lane l of wave 0 sequential over elements (j*64 + l)*8 + e, fixed
    // butterfly), longer rows its 256-thread path (thread t < 256 sequential over elements (it*256 + t)*8
    // + e, fixed butterfly, the 4 wave sums in wave order); then y = (x * r) * gamma, absmax scale,
    // round-half-even codes (the element-wise part spread over all threads), codes into LDS with zeros
    // from h to the end of the row
    const int h = ns.h;
    const int kpad = 64 * C;
    float g[PCH][kVec];  // gamma of the thread's elements (1 without gamma; past h the elements are 0)
#pragma unroll
    for (int j = 0; j < PCH; ++j) {
      if (ns.gamma == nullptr) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[j][e] = 1.0f;
      } else if (ns.gdt == WFB_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g[j][e] = __int_as_float(graw[j][0][e]);
          g[j][4 + e] = __int_as_float(graw[j][1][e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w2 = (uint32_t)graw[j][0][e];
          g[j][2 * e] = __uint_as_float(w2 << 16);
          g[j][2 * e + 1] = __uint_as_float(w2 & 0xFFFF0000u);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < PCH; ++j) {
      float* dst = &xs[(t + j * 64 * S) * kVec];
      *reinterpret_cast<float4*>(dst) = make_float4(xv[j][0], xv[j][1], xv[j][2], xv[j][3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(xv[j][4], xv[j][5], xv[j][6], xv[j][7]);
    }
    __syncthreads();
    const bool wave_order = h <= kWaveMaxH;
    const int nsum = wave_order ? 64 : kTPB;  // threads of the sum
    if (t < nsum) {
      float ss = 0.0f;
      // the staged row is zero from h to KMAX and adding +0 to a sum of squares changes nothing, so every
      // step the launch shape allows is read, all reads issued before the first add (the adds keep the
      // quantiser's order; a step past h reads zeros)
      // steps: the one-wave order covers at most kWaveMaxH elements, the 256-thread order at most KMAX
      constexpr int WMAX = KMAX < kWaveMaxH ? KMAX : kWaveMaxH;
      constexpr int NIT_W = (WMAX + 64 * kVec - 1) / (64 * kVec), NIT_B = (KMAX + kTPB * kVec - 1) / (kTPB * kVec);
      constexpr int NIT = NIT_W > NIT_B ? NIT_W : NIT_B;
      float4 p[NIT][2];
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int e0 = (it * nsum + t) * kVec;
        const bool in = (wave_order ? it < NIT_W : it < NIT_B) && e0 < KMAX;
        p[it][0] = in ? *reinterpret_cast<const float4*>(&xs[e0]) : make_float4(0.f, 0.f, 0.f, 0.f);
        p[it][1] = in ? *reinterpret_cast<const float4*>(&xs[e0 + 4]) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const float v[kVec] = {p[it][0].x, p[it][0].y, p[it][0].z, p[it][0].w,
                               p[it][1].x, p[it][1].y, p[it][1].z, p[it][1].w};
#pragma unroll
        for (int e = 0; e < kVec; ++e) ss = __fadd_rn(ss, __fmul_rn(v[e], v[e]));
      }
      ss = wave_sum_fixed(ss);
      if (lane == 0) nred[w] = ss;
    }
    __syncthreads();
    float tot = nred[0];
    if (!wave_order) {
#pragma unroll
      for (int k = 1; k < kTPB / 64; ++k) tot = __fadd_rn(tot, nred[k]);
    }
    const float r = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, (float)h), ns.eps)));
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < PCH; ++j)
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        xv[j][e] = __fmul_rn(__fmul_rn(xv[j][e], r), g[j][e]);
        mx = fmaxf(mx, fabsf(xv[j][e]));
      }
    mx = wave_max(mx);
    if (lane == 0) mred[w] = mx;
    __syncthreads();
    mx = mred[0];
#pragma unroll
    for (int k = 1; k < S; ++k) mx = fmaxf(mx, mred[k]);
    if (mx < 1e-6f) mx = 1.0f;
    const float inv = __fdiv_rn(127.0f, mx);
    if (t == 0) nscale[0] = __fdiv_rn(mx, 127.0f);
#pragma unroll
    for (int j = 0; j < PCH; ++j) {
      const int e0 = (t + j * 64 * S) * kVec;
      if (e0 < kpad) {
        uint32_t lo = 0, hi = 0;  // zeros past h
        if (e0 < h) {
          lo = quant4_i8(&xv[j][0], inv);
          hi = quant4_i8(&xv[j][4], inv);
        }
        *reinterpret_cast<uint2*>(&codes[0][e0]) = make_uint2(lo, hi);
      }
    }
    __syncthreads();  // codes and the scale complete
    // the activation fragments and sum(a) pieces from the LDS codes (same offsets as the global loads)
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = kc0 + s + L * i;
        const int off = 128 * (c >> 1) + 16 * (c & 1);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          a[m][i][q] = (EXACT || c < C) ? *reinterpret_cast<const v4i*>(&codes[m][off + 32 * q]) : v4i{0, 0, 0, 0};
      }
      const int boff = 64 * kc0 + lane * (L * CPL);
      const bool in = EXACT || boff < 64 * C;
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        if constexpr (L * CPL == 8) {
          const uint2 v = in ? *reinterpret_cast<const uint2*>(&codes[m][boff]) : make_uint2(0, 0);
          sv[m][b] = v4i{(int)v.x, (int)v.y, 0, 0};
        } else {
          sv[m][b] = in ? *reinterpret_cast<const v4i*>(&codes[m][boff + 16 * b]) : v4i{0, 0, 0, 0};
        }
      }
    }
    if (PRE && t < RB) {
      col.load_raw(ep, n, N, toks, M);
#pragma unroll
      for (int m = 0; m < M; ++m) col.as[m] = nscale[0];
    }
  }

  int suma[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int part = 0;
#pragma unroll
    for (int b = 0; b < SB; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) part = __builtin_amdgcn_sdot4(sv[m][b][e], 0x01010101, part, false);
    suma[m] = wave_sum(part);
  }
#pragma unroll
  for (int p = 0; p < RP; ++p) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      int acc_a = 0, acc_b = 0, acc_c = 0;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int d = wv[p][i][t];
          acc_c = __builtin_amdgcn_sdot4((d >> 2) & 0x30303030, a[m][i][0][t], acc_c, false);
          acc_c = __builtin_amdgcn_sdot4(d & 0x30303030, a[m][i][1][t], acc_c, false);
          acc_b = __builtin_amdgcn_sdot4(d & 0x0C0C0C0C, a[m][i][2][t], acc_b, false);
          acc_a = __builtin_amdgcn_sdot4(d & 0x03030303, a[m][i][3][t], acc_a, false);
        }
      }
      int tot = group_sum<L>(acc_a + (acc_b >> 2) + (acc_c >> 4));
      if (s == 0) red[w][m][p * RPG + r_in] = tot - suma[m];
    }
  }
  __syncthreads();
  if constexpr (PRE) col.finish(ep);
  if constexpr (GLU != 0) {
    // gated epilogue (the arithmetic of the batched kernels' gated epilogue): out[m, j] =
    // act(y_gate) * y_up with y = (acc * ws) * as per half, each rounded to mid_dtype, fp32 out
    constexpr int HB = RB / 2;
    const int half = N / 2, j = blockIdx.x * HB + t;
    if (t >= HB || j >= half) return;
    const float wsg = epi_wscale(ep, j), wsu = epi_wscale(ep, half + j);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      int tg = red[0][m][t], tu = red[0][m][t + HB];
#pragma unroll
      for (int k = 1; k < S; ++k) {
        tg += red[k][m][t];
        tu += red[k][m][t + HB];
      }
      const float as = NORM ? nscale[0] : epi_ascale(ep, m);
      float yg = __fmul_rn(__fmul_rn((float)tg, wsg), as), yu = __fmul_rn(__fmul_rn((float)tu, wsu), as);
      if (ep.mid_dtype == WFB_BF16) {
        yg = bf16_bits_to_f32(f32_to_bf16_rne(yg));
        yu = bf16_bits_to_f32(f32_to_bf16_rne(yu));
      }
      reinterpret_cast<float*>(ep.out)[(int64_t)m * ep.ldo + j] = glu<GLU>(yg, yu);
    }
    return;
  }
  if (ep.amax) {  // argmax epilogue: the RB <= 64 rows sit in wave 0
    if (t >= 64) return;
    const bool valid = t < RB && n < N;
    const float ws = PRE ? col.ws : valid ? epi_wscale(ep, n) : 0.0f;
    const float bias = PRE ? col.bias : valid ? epi_bias(ep, n) : 0.0f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      int tot = 0;
      if (valid) {
        tot = red[0][m][t];
#pragma unroll
        for (int k = 1; k < S; ++k) tot += red[k][m][t];
      }
      uint64_t key;
      if constexpr (PRE) key = epi_store_key_r(ep, ws, col.as[m], bias, col.res[m], m, n, tot, valid);
      else key = epi_store_key(ep, ws, NORM ? nscale[0] : epi_ascale(ep, m), bias, m, n, tot, valid);
      key = group_max_u64<64>(key);
      // slots are per 16 rows: the workgroup's first slot takes its maximum, the others key 0
      const int slot = row0 / 16 + t;
      if (t < RB / 16 && slot < (N + 15) / 16) ep.amax[(int64_t)slot * (ep.amax_ld ? ep.amax_ld : M) + m] = t == 0 ? key : 0;
    }
    return;
  }
  if (t >= RB) return;
  if (n >= N) return;
  const float ws = PRE ? col.ws : epi_wscale(ep, n);
  const float bias = PRE ? col.bias : epi_bias(ep, n);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int tot = red[0][m][t];
#pragma unroll
    for (int k = 1; k < S; ++k) tot += red[k][m][t];
    if constexpr (PRE) epi_store_r(ep, ws, col.as[m], bias, col.res[m], m, n, tot);
    else epi_store(ep, ws, NORM ? nscale[0] : epi_ascale(ep, m), bias, m, n, tot);
  }
}

// Grids above this many workgroups (many rounds over the 256 CUs: the LM-head shapes) load the activation
// fragments directly (STAGE = false) where the launch shape has that variant (WIDE).
constexpr int kStageMaxGrid = 2048;

template <int M, int L, int CPL, int RP, int S, bool PRE = true, int XDT = -1, bool WIDE = false, int GLU = 0>
hipError_t launch_cfg(const uint8_t* W, int n, int C, const int8_t* A, int64_t lda, const Epilogue& e,
                      hipStream_t st, const NormSrc& ns = NormSrc{}) {
  constexpr int RB = RP * (64 / L);
  const dim3 grid((n + RB - 1) / RB), block(64 * S);
  if constexpr (WIDE && XDT < 0) {
    if ((int)grid.x > kStageMaxGrid) {
      if (C == L * CPL * S)
        hipLaunchKernelGGL((gemv_i2s_kernel<M, L, CPL, RP, S, true, PRE, XDT, false, GLU>), grid, block, 0, st, W, A, lda, n,
                           C, e, ns);
      else
        hipLaunchKernelGGL((gemv_i2s_kernel<M, L, CPL, RP, S, false, PRE, XDT, false, GLU>), grid, block, 0, st, W, A, lda,
                           n, C, e, ns);
      return hipGetLastError();
    }
  }
  if (C == L * CPL * S)
    hipLaunchKernelGGL((gemv_i2s_kernel<M, L, CPL, RP, S, true, PRE, XDT, true, GLU>), grid, block, 0, st, W, A, lda, n, C, e, ns);
  else
    hipLaunchKernelGGL((gemv_i2s_kernel<M, L, CPL, RP, S, false, PRE, XDT, true, GLU>), grid, block, 0, st, W, A, lda, n, C, e, ns);
  return hipGetLastError();
}

// Norm prologue launches (rows up to 16384 elements): the launch shapes of the codes GEMV at those K, except
// K 2561..4096: 4 waves of 2 chunks per lane (Llama-3-8B q|k|v 6.09 -> 5.79 us, o 5.93 -> 5.64 against 8 waves
// of one chunk, cold weights on MI355X).
template <int M, int XDT>
hipError_t launch_norm_m(const uint8_t* W, int n, int C, const Epilogue& e, const NormSrc& ns, hipStream_t s) {
  if (C <= 8) return launch_cfg<M, 8, 1, 2, 1, true, XDT>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 16) return launch_cfg<M, 8, 1, 2, 2, true, XDT>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 24) return launch_cfg<M, 8, 1, 2, 3, true, XDT>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 40) return launch_cfg<M, 8, 1, 2, 5, true, XDT>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 64) return launch_cfg<M, 8, 2, 4, 4, true, XDT>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 112) return launch_cfg<M, 16, 1, 4, 7, true, XDT>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 224) return launch_cfg<M, 16, 1, 4, 14, true, XDT>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 256) return launch_cfg<M, 16, 1, 4, 16, true, XDT>(W, n, C, nullptr, 0, e, s, ns);
  return hipErrorNotSupported;
}

// Launch shape by K (C = K/64 chunks), from cold-HBM sweeps on MI355X at the BitNet-2B and Llama-3-8B
// shapes: 8 lanes x 1 chunk per row for K <= 4096 (2 row passes per wave at K = 2560: 13824 rows 4.31 ->
// 4.23 us against 4; 4 at K = 4096), 16 lanes for longer rows.  Other K take the nearest shape with masking.
template <int M>
hipError_t launch_m(const uint8_t* W, int n, int C, const int8_t* A, int64_t lda, const Epilogue& e, hipStream_t s) {
  if (C <= 8) return launch_cfg<M, 8, 1, 2, 1, true, -1, true>(W, n, C, A, lda, e, s);
  if (C <= 16) return launch_cfg<M, 8, 1, 2, 2, true, -1, true>(W, n, C, A, lda, e, s);
  if (C <= 24) return launch_cfg<M, 8, 1, 2, 3, true, -1, true>(W, n, C, A, lda, e, s);
  if (C <= 40) return launch_cfg<M, 8, 1, 2, 5, true, -1, true>(W, n, C, A, lda, e, s);
  if (C <= 64) return launch_cfg<M, 8, 1, 4, 8, true, -1, true>(W, n, C, A, lda, e, s);
  if (C <= 112) return launch_cfg<M, 16, 1, 4, 7>(W, n, C, A, lda, e, s);
  if (C <= 224) return launch_cfg<M, 16, 1, 4, 14>(W, n, C, A, lda, e, s);
  if (C <= 256) return launch_cfg<M, 16, 1, 4, 16>(W, n, C, A, lda, e, s);
  if (C <= 512) return launch_cfg<M, 16, 2, 4, 16>(W, n, C, A, lda, e, s);
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

hipError_t launch_gemv_i2s_norm(const uint8_t* W, int n, int k, int m, const Epilogue& e, const NormSrc& ns,
                                hipStream_t s) {
  const int C = k / 64;
  if (m != 1) return hipErrorNotSupported;  // one row: the prologue keeps the row's elements in registers
  if (ns.xdt == WFB_F32) return launch_norm_m<1, WFB_F32>(W, n, C, e, ns, s);
  if (ns.xdt == WFB_BF16) return launch_norm_m<1, WFB_BF16>(W, n, C, e, ns, s);
  return hipErrorNotSupported;
}

// Gated gate|up with the norm prologue, one token, K <= 4096: workgroups of RB/2 gate rows and their up rows;
// 64-row workgroups from K 2049 (fewer workgroups repeating the norm: Llama-3-8B 28672 x 4096 11.74 -> 10.46 us,
// BitNet-2B 13824 x 2560 7.26 -> 6.33 us against 32 and 16 rows, cold weights on MI355X).
template <int XDT, int GLU>
hipError_t launch_norm_glu(const uint8_t* W, int n, int C, const Epilogue& e, const NormSrc& ns, hipStream_t s) {
  if (C <= 8) return launch_cfg<1, 8, 1, 2, 1, false, XDT, false, GLU>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 16) return launch_cfg<1, 8, 1, 2, 2, false, XDT, false, GLU>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 24) return launch_cfg<1, 8, 1, 2, 3, false, XDT, false, GLU>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 40) return launch_cfg<1, 8, 1, 8, 5, false, XDT, false, GLU>(W, n, C, nullptr, 0, e, s, ns);
  if (C <= 64) return launch_cfg<1, 8, 2, 8, 4, false, XDT, false, GLU>(W, n, C, nullptr, 0, e, s, ns);
  return hipErrorNotSupported;
}

hipError_t launch_gemv_i2s_norm_glu(const uint8_t* W, int n, int k, const Epilogue& e, const NormSrc& ns, int act,
                                    hipStream_t s) {
  const int C = k / 64;
  if (n % 64 != 0) return hipErrorNotSupported;  // whole gate/up row groups per workgroup
  const bool silu = act == WFB_ACT_SILU;
  if (ns.xdt == WFB_F32)
    return silu ? launch_norm_glu<WFB_F32, WFB_ACT_SILU>(W, n, C, e, ns, s) : launch_norm_glu<WFB_F32, WFB_ACT_RELU2>(W, n, C, e, ns, s);
  if (ns.xdt == WFB_BF16)
    return silu ? launch_norm_glu<WFB_BF16, WFB_ACT_SILU>(W, n, C, e, ns, s)
                : launch_norm_glu<WFB_BF16, WFB_ACT_RELU2>(W, n, C, e, ns, s);
  return hipErrorNotSupported;
}

}  // namespace wfb
