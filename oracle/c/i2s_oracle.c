/*
 * C restatement of the reference CPU BitLinear path -- TEST INFRASTRUCTURE ONLY.
 * Used by tests/ (cross-check of the numpy oracle) and by bench.py's cpu_baseline leg when the
 * reference build in oracle/_ref is absent.  Never linked into libwfbitnet.
 *
 * Follows (paths in the reference repository):
 *   ENG  = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/inference/bitnet_engine.cpp
 *   GEMV = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp
 *   OPS  = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp
 */
#include <math.h>
#include <stdint.h>

/* I2_S dot product of one packed row with int8 activations; scalar decode of ENG:51-81. */
int32_t orc_vec_dot_i2_i8(int k, const uint8_t* w, const int8_t* a) {
  int32_t sum = 0;
  for (int blk = 0; blk < k / 128; ++blk) {
    const uint8_t* wb = w + 32 * blk;
    const int8_t* ab = a + 128 * blk;
    for (int j = 0; j < 32; ++j) {
      const int byte = wb[j];
      sum += (((byte >> 6) & 3) - 1) * ab[j];
      sum += (((byte >> 4) & 3) - 1) * ab[j + 32];
      sum += (((byte >> 2) & 3) - 1) * ab[j + 64];
      sum += (((byte >> 0) & 3) - 1) * ab[j + 96];
    }
  }
  return sum;
}

/* out[m * n_batch + b] = dot(row m, token b) * scale: the [out, batch] layout and OpenMP row loop of
 * bitnet_gemm_i2_i8 (GEMV:814-874).  Returns -1 if k is not a multiple of 128 (GEMV:824-829). */
int orc_gemm_i2_i8(int m_out, int n_batch, int k, float* out, const uint8_t* w, const int8_t* a, float scale) {
  if (k % 128 != 0) return -1;
#pragma omp parallel for schedule(static)
  for (int m = 0; m < m_out; ++m)
    for (int b = 0; b < n_batch; ++b)
      out[(int64_t)m * n_batch + b] = (float)orc_vec_dot_i2_i8(k, w + (int64_t)m * (k / 4), a + (int64_t)b * k) * scale;
  return 0;
}

/* acc[b * m_out + m] as int32 (exact accumulators, [batch, out]). */
int orc_acc_i2_i8(int m_out, int n_batch, int k, int32_t* acc, const uint8_t* w, const int8_t* a) {
  if (k % 128 != 0) return -1;
#pragma omp parallel for schedule(static)
  for (int m = 0; m < m_out; ++m)
    for (int b = 0; b < n_batch; ++b)
      acc[(int64_t)b * m_out + m] = orc_vec_dot_i2_i8(k, w + (int64_t)m * (k / 4), a + (int64_t)b * k);
  return 0;
}

/* quantize_activations_i8 on n values (GEMV:880-1135, vector-path rounding: half to even). */
void orc_quantize_i8(int n, int8_t* out, const float* x, float* scale) {
  float mx = 0.0f;
  for (int i = 0; i < n; ++i) {
    float v = fabsf(x[i]);
    if (v > mx) mx = v;
  }
  if (mx < 1e-6f) mx = 1.0f;
  *scale = mx / 127.0f;
  const float inv = 127.0f / mx;
  for (int i = 0; i < n; ++i) {
    float r = nearbyintf(x[i] * inv); /* default rounding mode: to nearest even */
    if (r > 127.0f) r = 127.0f;
    if (r < -128.0f) r = -128.0f;
    out[i] = (int8_t)r;
  }
}
