/*
 * AVX2 restatement of the reference CPU I2_S GEMV op -- TEST INFRASTRUCTURE and the CPU BASELINE
 * that bench.py times beside the GPU.  Never linked into libwfbitnet.
 *
 * What it restates (paths in the reference repository):
 *   GEMV = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp
 *   OPS  = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp
 *   - the per-row dot of bitnet_vec_dot_i2_i8 on AVX2 (GEMV:516-685): each 128-weight block is one
 *     32-byte load; the four 2-bit fields are taken out with a 16-bit shift and a 0x03 byte mask, so
 *     they are the unsigned codes {0,1,2}; vpmaddubsw multiplies them with the signed activation bytes
 *     (pairs summed into int16: at most 2*2*128 = 512 per pair, no saturation), the four fields are
 *     summed in int16 (<= 2048), vpmaddwd with ones widens to int32, and the +1 code offset is removed
 *     at the end with the sum of the activations (GEMV:342-402, 685);
 *   - the op's OpenMP row loop, fp32 output = float(acc) * scale (OPS:355-366), and the batched form
 *     that writes [out, batch] (GEMV:814-874, OPS:370-406).
 * Differences in how, not what: the activation sum is taken once per call instead of once per row;
 * two row-independent accumulators come from the two halves of each 64-byte step instead of four
 * blocks round-robin; no software prefetch.  Integer arithmetic is exact either way, so the outputs
 * equal the reference build's bit for bit (tests/test_oracle.py checks that).
 */
#include <immintrin.h>
#include <stdint.h>

static inline int32_t hsum8_i32(__m256i v) {
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
  return _mm_cvtsi128_si32(s);
}

/* sum of k int8 activations */
static int32_t act_sum(int k, const int8_t* a) {
  __m256i acc = _mm256_setzero_si256();
  const __m256i ones16 = _mm256_set1_epi16(1);
  int i = 0;
  for (; i + 32 <= k; i += 32) {
    __m256i v = _mm256_loadu_si256((const __m256i*)(a + i));
    __m256i lo = _mm256_cvtepi8_epi16(_mm256_castsi256_si128(v));
    __m256i hi = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(v, 1));
    acc = _mm256_add_epi32(acc, _mm256_madd_epi16(_mm256_add_epi16(lo, hi), ones16));
  }
  int32_t s = hsum8_i32(acc);
  for (; i < k; ++i) s += a[i];
  return s;
}

/* sum over k of code(w[k]) * a[k] for one I2_S row, codes in {0,1,2} (k % 128 == 0) */
static inline int32_t code_dot(int k, const uint8_t* w, const int8_t* a) {
  const __m256i m3 = _mm256_set1_epi8(0x03);
  const __m256i ones16 = _mm256_set1_epi16(1);
  __m256i acc0 = _mm256_setzero_si256(), acc1 = _mm256_setzero_si256();
  const int nb = k / 128;
  int b = 0;
  for (; b + 2 <= nb; b += 2) {
    for (int h = 0; h < 2; ++h) {
      const __m256i wb = _mm256_loadu_si256((const __m256i*)(w + 32 * (b + h)));
      const int8_t* ab = a + 128 * (b + h);
      /* field f (bits 7-2f .. 6-2f of byte j) holds the weight at k = 128b + 32f + j */
      __m256i p = _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(wb, 6), m3),
                                       _mm256_loadu_si256((const __m256i*)(ab)));
      p = _mm256_add_epi16(p, _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(wb, 4), m3),
                                                   _mm256_loadu_si256((const __m256i*)(ab + 32))));
      p = _mm256_add_epi16(p, _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(wb, 2), m3),
                                                   _mm256_loadu_si256((const __m256i*)(ab + 64))));
      p = _mm256_add_epi16(p, _mm256_maddubs_epi16(_mm256_and_si256(wb, m3),
                                                   _mm256_loadu_si256((const __m256i*)(ab + 96))));
      if (h == 0)
        acc0 = _mm256_add_epi32(acc0, _mm256_madd_epi16(p, ones16));
      else
        acc1 = _mm256_add_epi32(acc1, _mm256_madd_epi16(p, ones16));
    }
  }
  for (; b < nb; ++b) {
    const __m256i wb = _mm256_loadu_si256((const __m256i*)(w + 32 * b));
    const int8_t* ab = a + 128 * b;
    __m256i p = _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(wb, 6), m3),
                                     _mm256_loadu_si256((const __m256i*)(ab)));
    p = _mm256_add_epi16(p, _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(wb, 4), m3),
                                                 _mm256_loadu_si256((const __m256i*)(ab + 32))));
    p = _mm256_add_epi16(p, _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(wb, 2), m3),
                                                 _mm256_loadu_si256((const __m256i*)(ab + 64))));
    p = _mm256_add_epi16(p, _mm256_maddubs_epi16(_mm256_and_si256(wb, m3),
                                                 _mm256_loadu_si256((const __m256i*)(ab + 96))));
    acc0 = _mm256_add_epi32(acc0, _mm256_madd_epi16(p, ones16));
  }
  return hsum8_i32(_mm256_add_epi32(acc0, acc1));
}

/* bitnet_gemv_cpu: out[n] = float(sum_k w[n,k] * a[k]) * scale, OpenMP over rows.
 * Returns -1 if k is not a positive multiple of 128 (GEMV:331-336). */
int cpu_gemv_i2s_avx2(int n_out, int k, float* out, const uint8_t* w, const int8_t* a, float scale) {
  if (k <= 0 || k % 128 != 0) return -1;
  const int32_t sa = act_sum(k, a);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < n_out; ++n)
    out[n] = (float)(code_dot(k, w + (int64_t)n * (k / 4), a) - sa) * scale;
  return 0;
}

/* bitnet_gemm_cpu: out[n * batch + b] (the reference's [out, batch] order), OpenMP over rows. */
int cpu_gemm_i2s_avx2(int n_out, int batch, int k, float* out, const uint8_t* w, const int8_t* a, float scale) {
  if (k <= 0 || k % 128 != 0 || batch < 0) return -1;
  if (batch == 0) return 0;
  int32_t sa_stack[64];
  int32_t* sa = sa_stack;
  if (batch > 64) return -1; /* the CPU baseline's batches are small; larger ones go through the oracle */
  for (int b = 0; b < batch; ++b) sa[b] = act_sum(k, a + (int64_t)b * k);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < n_out; ++n)
    for (int b = 0; b < batch; ++b)
      out[(int64_t)n * batch + b] =
          (float)(code_dot(k, w + (int64_t)n * (k / 4), a + (int64_t)b * k) - sa[b]) * scale;
  return 0;
}
