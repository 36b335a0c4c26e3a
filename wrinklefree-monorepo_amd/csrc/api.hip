// extern "C" entry points of libwfbitnet: argument validation, error reporting and kernel choice.
//
// Validation mirrors the reference op boundary (TORCH_CHECK on dtype/rank/shape in
// SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:336-346, 375-386, 410 and the K % 128 check of
// SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:331-336, 824-829) and adds the alignment the 128-bit
// loads need.  Every check runs on the host before anything touches the GPU.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "wfb_common.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return WFB_OK;
}

int hip_status(hipError_t e, const char* where) {
  if (e != hipSuccess) return fail(WFB_EHIP, "%s: HIP error %d (%s)", where, (int)e, hipGetErrorString(e));
  return ok();
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

bool valid_dtype(int dt) { return dt == WFB_F32 || dt == WFB_BF16 || dt == WFB_F16; }

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

enum class Kernel { Auto, Gemv, Gemm };

// Decode (M <= 2) runs the VALU GEMV; everything else runs MFMA.  The GEMV addresses weights and
// activations through 32-bit buffer offsets.
bool use_gemv(int64_t m, int64_t n, int64_t k, int64_t lda) {
  return m >= 1 && m <= 2 && k <= 32768 && n * (k / 4) <= INT32_MAX && (m - 1) * lda + k <= INT32_MAX;
}

int linear_impl(Kernel kind, const char* name, const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act,
                int64_t m, int64_t lda, const float* a_scale, const float* w_scale_dev, float w_scale,
                const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo, int32_t* acc_out,
                void* stream, int n_seg = 1, const int64_t* seg_rows = nullptr, uint64_t* amax = nullptr,
                int amax_dt = WFB_F32, int64_t* tokens = nullptr, const void* res = nullptr, int res_dtype = 0,
                int64_t ldr = 0) {
  if (n <= 0 || k <= 0 || m < 0) return fail(WFB_EINVAL, "%s: bad sizes m=%lld n=%lld k=%lld", name, (long long)m, (long long)n, (long long)k);
  if (k % WFB_QK_I2S != 0)
    return fail(WFB_EINVAL, "%s: K (%lld) must be multiple of %d", name, (long long)k, WFB_QK_I2S);
  if (n > INT32_MAX / 2 || m > INT32_MAX / 2 || k > (1 << 20))
    return fail(WFB_EINVAL, "%s: sizes too large m=%lld n=%lld k=%lld", name, (long long)m, (long long)n, (long long)k);
  if (m == 0) return ok();
  if (!qweight || !act) return fail(WFB_EINVAL, "%s: null qweight or activations", name);
  if (!out && !acc_out && !amax) return fail(WFB_EINVAL, "%s: out and acc_out are both null", name);
  if (!aligned(qweight, 16) || !aligned(act, 16))
    return fail(WFB_EINVAL, "%s: qweight and activations must be 16-byte aligned", name);
  if (lda < k || lda % 16 != 0)
    return fail(WFB_EINVAL, "%s: activation row stride (%lld) must be >= K and a multiple of 16", name, (long long)lda);
  if (ldo < n) return fail(WFB_EINVAL, "%s: output row stride (%lld) < N (%lld)", name, (long long)ldo, (long long)n);
  if (out && out_dtype != WFB_F32 && out_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: out dtype must be WFB_F32 or WFB_BF16", name);
  if (bias && !valid_dtype(bias_dtype)) return fail(WFB_EINVAL, "%s: bad bias dtype %d", name, bias_dtype);
  if (kind == Kernel::Gemv && !use_gemv(m, n, k, lda))
    return fail(WFB_EINVAL, "%s: the GEMV kernel takes M <= 2 tokens, K <= 32768 and N*K/4 < 2^31 (got M=%lld N=%lld K=%lld)",
                name, (long long)m, (long long)n, (long long)k);
  // The prefill GEMM (M > 64) addresses each tile of up to 128 activation rows through 32-bit offsets
  // from the tile's first row; any M and N are fine, only a very long row stride is not.
  if (m > 64 && 127 * lda + k > INT32_MAX)
    return fail(WFB_EINVAL, "%s: activation row stride (%lld) too large for the prefill GEMM: 127 * lda + K must be "
                "below 2^31", name, (long long)lda);

  wfb::Epilogue e;
  e.nseg = n_seg;
  for (int j = 0; j < WFB_MAX_SEGMENTS - 1; ++j) e.seg_end[j] = 0;
  if (n_seg > 1) {
    int64_t end = 0;
    for (int j = 0; j + 1 < n_seg; ++j) e.seg_end[j] = (int)(end += seg_rows[j]);
  }
  e.a_scale = a_scale;
  e.ws_dev = w_scale_dev;
  e.ws = w_scale;
  e.bias = bias;
  e.bias_dtype = bias_dtype;
  e.out = out;
  e.out_dtype = out_dtype;
  e.ldo = ldo;
  e.acc_out = acc_out;
  e.amax = amax;
  e.amax_dt = amax_dt;
  e.amax_ld = 0;
  e.res = res;
  e.res_dtype = res_dtype;
  e.ldr = ldr;
  e.mid_dtype = 0;

  const bool gemv = kind == Kernel::Gemv || (kind == Kernel::Auto && use_gemv(m, n, k, lda));
  if (amax) {  // greedy argmax: GEMV (M <= 2) or the skinny MFMA kernel, then the cross-workgroup maximum
    hipError_t st = hipSuccess;
    if (!gemv && m > 16 && n >= wfb::kHeadChunkMinRows) {
      // more than 16 tokens on a head of many rows: chunks of 16 tokens through the persistent form,
      // each writing its tokens' keys into the full [slots, M] layout (measured on MI355X, 128256 x 4096:
      // M = 64 453 -> 140 us, M = 48 386 -> 109, M = 32 127 -> 79, M = 17 94 -> 77)
      for (int64_t c0 = 0; c0 < m && st == hipSuccess; c0 += 16) {
        wfb::Epilogue ec = e;
        ec.amax = amax + c0;
        ec.amax_ld = (int)m;
        if (ec.a_scale) ec.a_scale += c0;
        if (ec.out) ec.out = static_cast<char*>(ec.out) + c0 * ldo * (out_dtype == WFB_F32 ? 4 : 2);
        if (ec.acc_out) ec.acc_out += c0 * ldo;
        st = wfb::launch_gemm_i2s_skinny(qweight, (int)n, (int)k, act + c0 * lda, (int)std::min<int64_t>(16, m - c0), lda,
                                         ec, as_stream(stream));
      }
    } else {
      st = gemv ? wfb::launch_gemv_i2s(qweight, (int)n, (int)k, act, (int)m, lda, e, as_stream(stream))
                : wfb::launch_gemm_i2s_skinny(qweight, (int)n, (int)k, act, (int)m, lda, e, as_stream(stream));
    }
    if (st == hipSuccess) st = wfb::launch_argmax_finalize(amax, (n + 15) / 16, m, tokens, as_stream(stream));
    return hip_status(st, name);
  }
  hipError_t st = gemv ? wfb::launch_gemv_i2s(qweight, (int)n, (int)k, act, (int)m, lda, e, as_stream(stream))
                       : wfb::launch_gemm_i2s(qweight, (int)n, (int)k, act, (int)m, lda, e, as_stream(stream));
  return hip_status(st, name);
}


// Host checks shared by the decode attention entry points; WFB_OK when the call may go ahead.
int check_decode_attention(const char* name, const void* q, int64_t ldq, const void* k_new, int64_t ldk,
                           const void* v_new, int64_t ldv, int dtype, const float* rope_cos, const float* rope_sin,
                           void* k_cache, void* v_cache, int64_t max_len, const int64_t* pos, int64_t batch,
                           int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, float scale, void* out,
                           int64_t ldo) {
  if (dtype != WFB_F32 && dtype != WFB_BF16) return fail(WFB_EINVAL, "%s: dtype must be WFB_F32 or WFB_BF16", name);
  if (head_dim != 64 && head_dim != 128) return fail(WFB_EINVAL, "%s: head_dim (%lld) must be 64 or 128", name, (long long)head_dim);
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0 || num_heads / num_kv_heads > 8)
    return fail(WFB_EINVAL, "%s: num_heads (%lld) must be 1..8 times num_kv_heads (%lld)", name, (long long)num_heads,
                (long long)num_kv_heads);
  const int64_t esz = dtype == WFB_F32 ? 4 : 2;
  if (batch < 0 || batch > 65535 || num_kv_heads > 65535)
    return fail(WFB_EINVAL, "%s: batch (%lld) and num_kv_heads must be <= 65535", name, (long long)batch);
  if (max_len <= 0 || max_len * head_dim * esz > INT32_MAX)
    return fail(WFB_EINVAL, "%s: max_len (%lld) must be positive with max_len*head_dim*elem_size < 2^31", name,
                (long long)max_len);
  if (ldq < num_heads * head_dim || ldo < num_heads * head_dim || ldk < num_kv_heads * head_dim ||
      ldv < num_kv_heads * head_dim)
    return fail(WFB_EINVAL, "%s: row strides must cover num_heads*head_dim (q, out) and num_kv_heads*head_dim (k, v)",
                name);
  if ((rope_cos == nullptr) != (rope_sin == nullptr))
    return fail(WFB_EINVAL, "%s: rope_cos and rope_sin must both be given or both be NULL", name);
  if (!(scale == scale) || scale == __builtin_inff() || scale == -__builtin_inff())
    return fail(WFB_EINVAL, "%s: scale must be finite", name);
  if (batch == 0) return ok();
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !pos || !out) return fail(WFB_EINVAL, "%s: null pointer", name);
  if (!aligned(k_cache, 16) || !aligned(v_cache, 16)) return fail(WFB_EINVAL, "%s: caches must be 16-byte aligned", name);
  return WFB_OK;
}
}  // namespace

extern "C" {

const char* wfb_last_error(void) { return g_err.c_str(); }

int wfb_version(void) { return 1; }

int wfb_weight_absmean(const void* w, int w_dtype, int64_t numel, float* scale_dev, double* workspace, void* stream) {
  if (!valid_dtype(w_dtype)) return fail(WFB_EINVAL, "wfb_weight_absmean: bad dtype %d", w_dtype);
  if (numel < 0) return fail(WFB_EINVAL, "wfb_weight_absmean: numel < 0");
  if (!scale_dev || !workspace || (numel > 0 && !w)) return fail(WFB_EINVAL, "wfb_weight_absmean: null pointer");
  return hip_status(wfb::launch_weight_absmean(w, w_dtype, numel, scale_dev, workspace, as_stream(stream)),
                    "wfb_weight_absmean");
}

int wfb_pack_i2s(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw, const float* scale_dev,
                 uint8_t* qweight, void* stream) {
  if (!valid_dtype(w_dtype)) return fail(WFB_EINVAL, "wfb_pack_i2s: bad dtype %d", w_dtype);
  if (n < 0 || k <= 0 || k % WFB_QK_I2S != 0)
    return fail(WFB_EINVAL, "wfb_pack_i2s: K (%lld) must be multiple of %d", (long long)k, WFB_QK_I2S);
  if (ldw < k) return fail(WFB_EINVAL, "wfb_pack_i2s: row stride %lld < K %lld", (long long)ldw, (long long)k);
  if (n > 0 && (!w || !qweight || !scale_dev)) return fail(WFB_EINVAL, "wfb_pack_i2s: null pointer");
  if (!aligned(qweight, 4)) return fail(WFB_EINVAL, "wfb_pack_i2s: qweight must be 4-byte aligned");
  return hip_status(wfb::launch_pack_i2s(w, w_dtype, n, k, ldw, scale_dev, qweight, as_stream(stream)), "wfb_pack_i2s");
}

int wfb_unpack_i2s(const uint8_t* qweight, int64_t n, int64_t k, int8_t* w_out, void* stream) {
  if (n < 0 || k <= 0 || k % WFB_QK_I2S != 0)
    return fail(WFB_EINVAL, "wfb_unpack_i2s: K (%lld) must be multiple of %d", (long long)k, WFB_QK_I2S);
  if (n > 0 && (!qweight || !w_out)) return fail(WFB_EINVAL, "wfb_unpack_i2s: null pointer");
  return hip_status(wfb::launch_unpack_i2s(qweight, n, k, w_out, as_stream(stream)), "wfb_unpack_i2s");
}

int wfb_quantize_act_i8(const void* x, int x_dtype, int64_t m, int64_t h, int64_t ldx, int8_t* q, int64_t k_pad,
                        int64_t ldq, float* a_scale, void* stream) {
  if (!valid_dtype(x_dtype)) return fail(WFB_EINVAL, "wfb_quantize_act_i8: bad dtype %d", x_dtype);
  if (m < 0 || h <= 0 || h > WFB_NORM_MAX_H)
    return fail(WFB_EINVAL, "wfb_quantize_act_i8: row length %lld outside 1..%d", (long long)h, WFB_NORM_MAX_H);
  if (ldx < h || k_pad < h || ldq < k_pad)
    return fail(WFB_EINVAL, "wfb_quantize_act_i8: strides must satisfy ldx >= H, ldq >= k_pad >= H");
  if (m == 0) return ok();
  if (!x || !q || !a_scale) return fail(WFB_EINVAL, "wfb_quantize_act_i8: null pointer");
  if (!aligned(q, 8) || ldq % 8 != 0) return fail(WFB_EINVAL, "wfb_quantize_act_i8: q must be 8-byte aligned rows");
  return hip_status(wfb::launch_quant_rows(x, x_dtype, ldx, nullptr, 0, false, 0.0f, m, h, q, k_pad, ldq, a_scale,
                                           as_stream(stream)),
                    "wfb_quantize_act_i8");
}

int wfb_quantize_act_i8_tensor(const void* x, int x_dtype, int64_t numel, int8_t* q, float* a_scale, void* stream) {
  if (!valid_dtype(x_dtype)) return fail(WFB_EINVAL, "wfb_quantize_act_i8_tensor: bad dtype %d", x_dtype);
  if (numel < 0) return fail(WFB_EINVAL, "wfb_quantize_act_i8_tensor: numel < 0");
  if (!a_scale || (numel > 0 && (!x || !q))) return fail(WFB_EINVAL, "wfb_quantize_act_i8_tensor: null pointer");
  if (!aligned(a_scale, 4)) return fail(WFB_EINVAL, "wfb_quantize_act_i8_tensor: a_scale misaligned");
  return hip_status(wfb::launch_quant_tensor(x, x_dtype, numel, q, a_scale, as_stream(stream)),
                    "wfb_quantize_act_i8_tensor");
}

int wfb_rmsnorm_quant_i8(const void* x, int x_dtype, int64_t ldx, const void* gamma, int gamma_dtype, float eps,
                         int64_t m, int64_t h, int8_t* q, int64_t k_pad, int64_t ldq, float* a_scale, void* stream) {
  if (!valid_dtype(x_dtype) || (gamma && !valid_dtype(gamma_dtype)))
    return fail(WFB_EINVAL, "wfb_rmsnorm_quant_i8: bad dtype");
  if (m < 0 || h <= 0 || h > WFB_NORM_MAX_H || h % 8 != 0)
    return fail(WFB_EINVAL, "wfb_rmsnorm_quant_i8: H (%lld) must be a multiple of 8 in 8..%d", (long long)h,
                WFB_NORM_MAX_H);
  if (ldx < h || k_pad < h || ldq < k_pad)
    return fail(WFB_EINVAL, "wfb_rmsnorm_quant_i8: strides must satisfy ldx >= H, ldq >= k_pad >= H");
  if (!(eps >= 0.0f)) return fail(WFB_EINVAL, "wfb_rmsnorm_quant_i8: eps must be >= 0");
  if (m == 0) return ok();
  if (!x || !q || !a_scale) return fail(WFB_EINVAL, "wfb_rmsnorm_quant_i8: null pointer");
  if (!aligned(q, 8) || ldq % 8 != 0) return fail(WFB_EINVAL, "wfb_rmsnorm_quant_i8: q must be 8-byte aligned rows");
  return hip_status(wfb::launch_quant_rows(x, x_dtype, ldx, gamma, gamma_dtype, true, eps, m, h, q, k_pad, ldq,
                                           a_scale, as_stream(stream)),
                    "wfb_rmsnorm_quant_i8");
}

int wfb_linear_i2s(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m, int64_t lda,
                   const float* a_scale, const float* w_scale_dev, float w_scale, const void* bias, int bias_dtype,
                   void* out, int out_dtype, int64_t ldo, int32_t* acc_out, void* stream) {
  return linear_impl(Kernel::Auto, "wfb_linear_i2s", qweight, n, k, act, m, lda, a_scale, w_scale_dev, w_scale, bias,
                     bias_dtype, out, out_dtype, ldo, acc_out, stream);
}

int wfb_gemv_i2s(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m, int64_t lda,
                 const float* a_scale, const float* w_scale_dev, float w_scale, const void* bias, int bias_dtype,
                 void* out, int out_dtype, int64_t ldo, int32_t* acc_out, void* stream) {
  return linear_impl(Kernel::Gemv, "wfb_gemv_i2s", qweight, n, k, act, m, lda, a_scale, w_scale_dev, w_scale, bias,
                     bias_dtype, out, out_dtype, ldo, acc_out, stream);
}

int wfb_gemm_i2s(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m, int64_t lda,
                 const float* a_scale, const float* w_scale_dev, float w_scale, const void* bias, int bias_dtype,
                 void* out, int out_dtype, int64_t ldo, int32_t* acc_out, void* stream) {
  return linear_impl(Kernel::Gemm, "wfb_gemm_i2s", qweight, n, k, act, m, lda, a_scale, w_scale_dev, w_scale, bias,
                     bias_dtype, out, out_dtype, ldo, acc_out, stream);
}

int wfb_linear_i2s_segmented(const uint8_t* qweight, int64_t n, int64_t k, int n_seg, const int64_t* seg_rows,
                             const float* w_scales_dev, const int8_t* act, int64_t m, int64_t lda,
                             const float* a_scale, const void* bias, int bias_dtype, void* out, int out_dtype,
                             int64_t ldo, int32_t* acc_out, void* stream) {
  const char* name = "wfb_linear_i2s_segmented";
  if (n_seg < 1 || n_seg > WFB_MAX_SEGMENTS)
    return fail(WFB_EINVAL, "%s: n_seg (%d) must be in 1..%d", name, n_seg, WFB_MAX_SEGMENTS);
  if (!seg_rows || !w_scales_dev) return fail(WFB_EINVAL, "%s: null seg_rows or w_scales_dev", name);
  int64_t total = 0;
  for (int j = 0; j < n_seg; ++j) {
    if (seg_rows[j] <= 0 || seg_rows[j] % 8 != 0)
      return fail(WFB_EINVAL, "%s: segment %d has %lld rows (must be a positive multiple of 8)", name, j,
                  (long long)seg_rows[j]);
    total += seg_rows[j];
  }
  if (total != n) return fail(WFB_EINVAL, "%s: segment rows sum to %lld, N is %lld", name, (long long)total, (long long)n);
  return linear_impl(Kernel::Auto, name, qweight, n, k, act, m, lda, a_scale, w_scales_dev, 0.0f, bias, bias_dtype,
                     out, out_dtype, ldo, acc_out, stream, n_seg, seg_rows);
}

int wfb_glu_rmsnorm_quant_i8(const void* gate, const void* up, int x_dtype, int64_t ldx, int act,
                             const void* gamma, int gamma_dtype, float eps, int64_t m, int64_t h, int8_t* q,
                             int64_t k_pad, int64_t ldq, float* a_scale, void* stream) {
  const char* name = "wfb_glu_rmsnorm_quant_i8";
  if (!valid_dtype(x_dtype) || (gamma && !valid_dtype(gamma_dtype))) return fail(WFB_EINVAL, "%s: bad dtype", name);
  if (act != WFB_ACT_SILU && act != WFB_ACT_RELU2) return fail(WFB_EINVAL, "%s: bad activation %d", name, act);
  if (m < 0 || h <= 0 || h > WFB_NORM_MAX_H || h % 8 != 0)
    return fail(WFB_EINVAL, "%s: H (%lld) must be a multiple of 8 in 8..%d", name, (long long)h, WFB_NORM_MAX_H);
  if (ldx < h || k_pad < h || ldq < k_pad)
    return fail(WFB_EINVAL, "%s: strides must satisfy ldx >= H, ldq >= k_pad >= H", name);
  if (!(eps >= 0.0f)) return fail(WFB_EINVAL, "%s: eps must be >= 0", name);
  if (m == 0) return ok();
  if (!gate || !up || !q || !a_scale) return fail(WFB_EINVAL, "%s: null pointer", name);
  if (!aligned(q, 8) || ldq % 8 != 0) return fail(WFB_EINVAL, "%s: q must be 8-byte aligned rows", name);
  return hip_status(wfb::launch_glu_quant_rows(gate, up, x_dtype, ldx, act, gamma, gamma_dtype, eps, m, h, q, k_pad,
                                               ldq, a_scale, as_stream(stream)),
                    name);
}

int wfb_convert_hf_offline_i2s(const uint8_t* packed_hf, int64_t nb, int64_t n, int64_t k, int64_t k_pad,
                               const void* weight_scale_dev, int scale_dtype, float weight_scale, int scale_mode,
                               uint8_t* qweight, float* scale_out, int64_t* workspace, void* stream) {
  const char* name = "wfb_convert_hf_offline_i2s";
  if (nb <= 0 || k <= 0 || n <= 4 * (nb - 1) || n > 4 * nb)
    return fail(WFB_EINVAL, "%s: need 4*(NB-1) < N <= 4*NB and K > 0 (NB=%lld N=%lld K=%lld)", name, (long long)nb,
                (long long)n, (long long)k);
  if (k_pad < k || k_pad % WFB_QK_I2S != 0)
    return fail(WFB_EINVAL, "%s: k_pad (%lld) must be >= K and a multiple of %d", name, (long long)k_pad, WFB_QK_I2S);
  if (n * (k_pad / 16) > (int64_t)INT32_MAX * 64 || nb * k > ((int64_t)1 << 40))
    return fail(WFB_EINVAL, "%s: tensor too large", name);
  if (scale_mode != WFB_SCALE_REFERENCE && scale_mode != WFB_SCALE_CHECKPOINT)
    return fail(WFB_EINVAL, "%s: bad scale mode %d", name, scale_mode);
  if (weight_scale_dev && scale_dtype != WFB_F32 && scale_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: weight scale dtype must be WFB_F32 or WFB_BF16", name);
  if (!packed_hf || !qweight || !scale_out || !workspace) return fail(WFB_EINVAL, "%s: null pointer", name);
  if (!aligned(qweight, 4)) return fail(WFB_EINVAL, "%s: qweight must be 4-byte aligned", name);
  return hip_status(wfb::launch_convert_hf_offline(packed_hf, nb, n, k, k_pad, weight_scale_dev, scale_dtype,
                                                   weight_scale, scale_mode, qweight, scale_out, workspace,
                                                   as_stream(stream)),
                    name);
}

int wfb_linear_i2s_residual(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m, int64_t lda,
                            const float* a_scale, const float* w_scale_dev, float w_scale, const void* residual,
                            int residual_dtype, int64_t ldr, void* out, int out_dtype, int64_t ldo, void* stream) {
  const char* name = "wfb_linear_i2s_residual";
  if (residual_dtype != WFB_F32 && residual_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: residual dtype must be WFB_F32 or WFB_BF16", name);
  if (m > 0 && (!residual || !out)) return fail(WFB_EINVAL, "%s: null residual or out", name);
  if (ldr < n) return fail(WFB_EINVAL, "%s: residual row stride (%lld) < N (%lld)", name, (long long)ldr, (long long)n);
  return linear_impl(Kernel::Auto, name, qweight, n, k, act, m, lda, a_scale, w_scale_dev, w_scale, nullptr, 0, out,
                     out_dtype, ldo, nullptr, stream, 1, nullptr, nullptr, WFB_F32, nullptr, residual, residual_dtype,
                     ldr);
}

int wfb_linear_i2s_argmax(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m, int64_t lda,
                          const float* a_scale, const float* w_scale_dev, float w_scale, void* logits,
                          int logits_dtype, int64_t ldo, uint64_t* workspace, int64_t* token_out, void* stream) {
  const char* name = "wfb_linear_i2s_argmax";
  if (logits_dtype != WFB_F32 && logits_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: logits dtype must be WFB_F32 or WFB_BF16", name);
  if (m > 64) return fail(WFB_EINVAL, "%s: M (%lld) must be <= 64", name, (long long)m);
  if (m > 0 && (!workspace || !token_out)) return fail(WFB_EINVAL, "%s: null workspace or token_out", name);
  if (n > 0 && k > 0 && m > 0 && (n * (k / 4) > INT32_MAX || (m - 1) * lda + k > INT32_MAX))
    return fail(WFB_EINVAL, "%s: N*K/4 and (M-1)*lda + K must stay below 2^31", name);
  if (ldo < n) return fail(WFB_EINVAL, "%s: logits row stride (%lld) < N (%lld)", name, (long long)ldo, (long long)n);
  return linear_impl(Kernel::Auto, name, qweight, n, k, act, m, lda, a_scale, w_scale_dev, w_scale, nullptr, 0,
                     logits, logits_dtype, ldo, nullptr, stream, 1, nullptr, workspace, logits_dtype, token_out);
}

int wfb_lm_head_argmax(const void* x, int x_dtype, int64_t ldx, const void* gamma, int gamma_dtype, float eps,
                       const void* weight, int w_dtype, int64_t ldw, int64_t m, int64_t n, int64_t h, float* logits,
                       int64_t ldo, uint64_t* workspace, int64_t* token_out, void* stream) {
  const char* name = "wfb_lm_head_argmax";
  if ((x_dtype != WFB_F32 && x_dtype != WFB_BF16) || (w_dtype != WFB_F32 && w_dtype != WFB_BF16) ||
      (gamma && !valid_dtype(gamma_dtype)))
    return fail(WFB_EINVAL, "%s: x and weight must be WFB_F32 or WFB_BF16", name);
  if (m < 0 || m > 16) return fail(WFB_EINVAL, "%s: M (%lld) must be in 0..16", name, (long long)m);
  if (n <= 0 || n > INT32_MAX / 2 || h <= 0 || h % 8 != 0)
    return fail(WFB_EINVAL, "%s: need N > 0 and H a positive multiple of 8 (N=%lld H=%lld)", name, (long long)n,
                (long long)h);
  if (m * h > 16384) return fail(WFB_EINVAL, "%s: M*H (%lld) must be <= 16384", name, (long long)(m * h));
  const int64_t wsz = w_dtype == WFB_F32 ? 4 : 2;
  if (ldx < h || ldw < h || (logits && ldo < n) || ldw % 8 != 0)
    return fail(WFB_EINVAL, "%s: strides must satisfy ldx >= H, ldw >= H (multiple of 8), ldo >= N", name);
  if (n * ldw * wsz > INT32_MAX) return fail(WFB_EINVAL, "%s: weight larger than 2^31 bytes", name);
  if (!(eps >= 0.0f)) return fail(WFB_EINVAL, "%s: eps must be >= 0", name);
  if (m == 0) return ok();
  if (!x || !weight || !workspace || !token_out) return fail(WFB_EINVAL, "%s: null pointer", name);
  if (!aligned(weight, 16)) return fail(WFB_EINVAL, "%s: weight must be 16-byte aligned", name);
  hipError_t st = wfb::launch_lm_head_argmax(x, x_dtype, ldx, gamma, gamma_dtype, eps, weight, w_dtype, ldw, m, n, h,
                                             logits, ldo, workspace, as_stream(stream));
  if (st == hipSuccess) st = wfb::launch_argmax_finalize(workspace, (n + 15) / 16, m, token_out, as_stream(stream));
  return hip_status(st, name);
}

int wfb_gqa_decode_attention(const void* q, int64_t ldq, const void* k_new, int64_t ldk, const void* v_new,
                             int64_t ldv, int dtype, const float* rope_cos, const float* rope_sin, void* k_cache,
                             void* v_cache, int64_t max_len, const int64_t* pos, int64_t batch, int64_t num_heads,
                             int64_t num_kv_heads, int64_t head_dim, float scale, void* out, int64_t ldo,
                             float* workspace, void* stream) {
  const char* name = "wfb_gqa_decode_attention";
  const int st = check_decode_attention(name, q, ldq, k_new, ldk, v_new, ldv, dtype, rope_cos, rope_sin, k_cache,
                                        v_cache, max_len, pos, batch, num_heads, num_kv_heads, head_dim, scale, out,
                                        ldo);
  if (st != WFB_OK || batch == 0) return st;
  return hip_status(wfb::launch_gqa_decode(dtype, (int)head_dim, (int)(num_heads / num_kv_heads), q, ldq, k_new, ldk,
                                           v_new, ldv, rope_cos, rope_sin, k_cache, v_cache, max_len, pos, (int)batch,
                                           (int)num_kv_heads, scale, out, ldo, workspace, as_stream(stream)),
                    name);
}

int wfb_gqa_decode_attention_noalloc(const void* q, int64_t ldq, const void* k_new, int64_t ldk, const void* v_new,
                                     int64_t ldv, int dtype, const float* rope_cos, const float* rope_sin,
                                     void* k_cache, void* v_cache, int64_t max_len, const int64_t* pos, int64_t batch,
                                     int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, float scale,
                                     void* out, int64_t ldo, void* stream) {
  const char* name = "wfb_gqa_decode_attention_noalloc";
  const int st = check_decode_attention(name, q, ldq, k_new, ldk, v_new, ldv, dtype, rope_cos, rope_sin, k_cache,
                                        v_cache, max_len, pos, batch, num_heads, num_kv_heads, head_dim, scale, out,
                                        ldo);
  if (st != WFB_OK || batch == 0) return st;
  const int g = (int)(num_heads / num_kv_heads);
  const int64_t need = wfb::gqa_decode_workspace_floats(max_len, g, batch, num_kv_heads, (int)head_dim);
  if (need > wfb::kAttnScratchFloats)
    return fail(WFB_EINVAL, "%s: these sizes need %lld floats of split partials, more than the %lld (32 MiB) of the "
                "library's scratch; pass a workspace to wfb_gqa_decode_attention instead", name, (long long)need,
                (long long)wfb::kAttnScratchFloats);
  float* part = nullptr;
  if (need > 0) {
    const hipError_t e = wfb::gqa_decode_scratch(as_stream(stream), &part);
    if (e != hipSuccess) return hip_status(e, name);
  }
  return hip_status(wfb::launch_gqa_decode(dtype, (int)head_dim, g, q, ldq, k_new, ldk, v_new, ldv, rope_cos,
                                           rope_sin, k_cache, v_cache, max_len, pos, (int)batch, (int)num_kv_heads,
                                           scale, out, ldo, part, as_stream(stream)),
                    name);
}

int wfb_gqa_prefill_attention(const void* q, int64_t ldq, const void* k_new, int64_t ldk, const void* v_new,
                              int64_t ldv, int dtype, const float* rope_cos, const float* rope_sin, void* k_cache,
                              void* v_cache, int64_t max_len, int64_t start, int64_t batch, int64_t t,
                              int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, float scale, void* out,
                              int64_t ldo, void* stream) {
  const char* name = "wfb_gqa_prefill_attention";
  if (dtype != WFB_BF16) return fail(WFB_EINVAL, "%s: dtype must be WFB_BF16", name);
  if (head_dim != 64 && head_dim != 128) return fail(WFB_EINVAL, "%s: head_dim (%lld) must be 64 or 128", name, (long long)head_dim);
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0 || num_heads / num_kv_heads > 8)
    return fail(WFB_EINVAL, "%s: num_heads (%lld) must be 1..8 times num_kv_heads (%lld)", name, (long long)num_heads,
                (long long)num_kv_heads);
  if (batch < 0 || batch > 65535 || num_kv_heads > 65535 || t < 0 || t > INT32_MAX / 2)
    return fail(WFB_EINVAL, "%s: batch (%lld) and num_kv_heads must be <= 65535, T (%lld) in range", name,
                (long long)batch, (long long)t);
  if (max_len <= 0 || max_len * head_dim * 2 > INT32_MAX)
    return fail(WFB_EINVAL, "%s: max_len (%lld) must be positive with max_len*head_dim*2 < 2^31", name, (long long)max_len);
  if (start < 0 || start + t > max_len)
    return fail(WFB_EINVAL, "%s: start (%lld) + T (%lld) must be within max_len (%lld)", name, (long long)start,
                (long long)t, (long long)max_len);
  if (ldq < num_heads * head_dim || ldo < num_heads * head_dim || ldk < num_kv_heads * head_dim ||
      ldv < num_kv_heads * head_dim)
    return fail(WFB_EINVAL, "%s: row strides must cover num_heads*head_dim (q, out) and num_kv_heads*head_dim (k, v)",
                name);
  if (ldq % 8 || ldo % 8) return fail(WFB_EINVAL, "%s: q and out row strides must be multiples of 8 elements", name);
  if ((rope_cos == nullptr) != (rope_sin == nullptr))
    return fail(WFB_EINVAL, "%s: rope_cos and rope_sin must both be given or both be NULL", name);
  if (!(scale == scale) || scale == __builtin_inff() || scale == -__builtin_inff())
    return fail(WFB_EINVAL, "%s: scale must be finite", name);
  if (batch == 0 || t == 0) return ok();
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !out) return fail(WFB_EINVAL, "%s: null pointer", name);
  if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(q, 16) || !aligned(out, 16) ||
      !aligned(rope_cos, 16) || !aligned(rope_sin, 16))
    return fail(WFB_EINVAL, "%s: q, out, the caches and the rope tables must be 16-byte aligned", name);
  return hip_status(wfb::launch_gqa_prefill((int)head_dim, (int)(num_heads / num_kv_heads), q, ldq, k_new, ldk, v_new,
                                            ldv, rope_cos, rope_sin, k_cache, v_cache, max_len, (int)batch,
                                            (int)num_kv_heads, (int)t, start, scale, out, ldo, as_stream(stream)),
                    name);
}

int wfb_rmsnorm_linear_i2s(const void* x, int x_dtype, int64_t ldx, const void* gamma, int gamma_dtype, float eps,
                           int64_t m, int64_t h, const uint8_t* qweight, int64_t n, int64_t k, int n_seg,
                           const int64_t* seg_rows, const float* w_scales_dev, const void* residual,
                           int residual_dtype, int64_t ldr, void* out, int out_dtype, int64_t ldo, void* stream) {
  const char* name = "wfb_rmsnorm_linear_i2s";
  if (x_dtype != WFB_F32 && x_dtype != WFB_BF16) return fail(WFB_EINVAL, "%s: x dtype must be WFB_F32 or WFB_BF16", name);
  if (gamma && gamma_dtype != WFB_F32 && gamma_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: gamma dtype must be WFB_F32 or WFB_BF16", name);
  if (m < 0 || m > 16) return fail(WFB_EINVAL, "%s: M (%lld) must be in 0..16", name, (long long)m);
  if (h <= 0 || h % 8 != 0 || h > k || k % WFB_QK_I2S != 0)
    return fail(WFB_EINVAL, "%s: need H %% 8 == 0, H <= K, K %% %d == 0 (got H=%lld K=%lld)", name, WFB_QK_I2S,
                (long long)h, (long long)k);
  // one token: the GEMV's prologue (rows up to WFB_NORM_MAX_H; the quantiser's one-wave order for H <= 4096,
  // its 256-thread order beyond); 2..16 tokens with K <= 4096: the LDS-staged batched kernel's prologue
  if (k > 4096 && !(m <= 1 && k <= WFB_NORM_MAX_H))
    return fail(WFB_EINVAL, "%s: K > 4096 needs M == 1 and K <= %d (got M=%lld H=%lld K=%lld)", name,
                WFB_NORM_MAX_H, (long long)m, (long long)h, (long long)k);
  if (n <= 0 || n > INT32_MAX / 2 || n * (k / 4) > INT32_MAX)
    return fail(WFB_EINVAL, "%s: bad N (%lld) for K %lld", name, (long long)n, (long long)k);
  if (ldx < h || ldo < n || (residual && ldr < n)) return fail(WFB_EINVAL, "%s: row strides too small", name);
  if (!(eps >= 0.0f)) return fail(WFB_EINVAL, "%s: eps must be >= 0", name);
  if (!out || (out_dtype != WFB_F32 && out_dtype != WFB_BF16))
    return fail(WFB_EINVAL, "%s: out must be non-null WFB_F32 or WFB_BF16", name);
  if (residual && residual_dtype != WFB_F32 && residual_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: residual dtype must be WFB_F32 or WFB_BF16", name);
  if (!w_scales_dev) return fail(WFB_EINVAL, "%s: null w_scales_dev", name);
  if (n_seg < 1 || n_seg > WFB_MAX_SEGMENTS || (n_seg > 1 && !seg_rows))
    return fail(WFB_EINVAL, "%s: n_seg (%d) must be in 1..%d with seg_rows for more than one", name, n_seg,
                WFB_MAX_SEGMENTS);
  wfb::Epilogue e{};  // everything not set below is null / zero
  e.nseg = n_seg;
  if (n_seg > 1) {
    int64_t total = 0;
    for (int j = 0; j < n_seg; ++j) {
      if (seg_rows[j] <= 0 || seg_rows[j] % 8 != 0)
        return fail(WFB_EINVAL, "%s: segment %d has %lld rows (must be a positive multiple of 8)", name, j,
                    (long long)seg_rows[j]);
      total += seg_rows[j];
      if (j + 1 < n_seg) e.seg_end[j] = (int)total;
    }
    if (total != n) return fail(WFB_EINVAL, "%s: segment rows sum to %lld, N is %lld", name, (long long)total, (long long)n);
  }
  if (m == 0) return ok();
  if (!x || !qweight) return fail(WFB_EINVAL, "%s: null x or qweight", name);
  const int esz = x_dtype == WFB_F32 ? 4 : 2;
  if (!aligned(x, 16) || (ldx * esz) % 16 != 0 || (gamma && !aligned(gamma, 16)) || !aligned(qweight, 16))
    return fail(WFB_EINVAL, "%s: x rows, gamma and qweight must be 16-byte aligned", name);
  e.ws_dev = w_scales_dev;
  e.out = out;
  e.out_dtype = out_dtype;
  e.ldo = ldo;
  e.res = residual;
  e.res_dtype = residual_dtype;
  e.ldr = ldr;
  const wfb::NormSrc ns{x, x_dtype, ldx, gamma, gamma_dtype, eps, (int)h};
  if (m == 1)
    return hip_status(wfb::launch_gemv_i2s_norm(qweight, (int)n, (int)k, (int)m, e, ns, as_stream(stream)), name);
  return hip_status(wfb::launch_skinny_lds(qweight, (int)n, (int)k, nullptr, (int)m, 0, e, 0, as_stream(stream), ns),
                    name);
}

int wfb_rmsnorm_linear_i2s_glu(const void* x, int x_dtype, int64_t ldx, const void* gamma, int gamma_dtype, float eps,
                               int64_t m, int64_t h, const uint8_t* qweight, int64_t n, int64_t k,
                               const float* w_scales_dev, int act_kind, int mid_dtype, float* out, int64_t ldo,
                               void* stream) {
  const char* name = "wfb_rmsnorm_linear_i2s_glu";
  if (x_dtype != WFB_F32 && x_dtype != WFB_BF16) return fail(WFB_EINVAL, "%s: x dtype must be WFB_F32 or WFB_BF16", name);
  if (gamma && gamma_dtype != WFB_F32 && gamma_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: gamma dtype must be WFB_F32 or WFB_BF16", name);
  if (act_kind != WFB_ACT_SILU && act_kind != WFB_ACT_RELU2) return fail(WFB_EINVAL, "%s: bad activation %d", name, act_kind);
  if (mid_dtype != WFB_F32 && mid_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: mid dtype must be WFB_F32 or WFB_BF16", name);
  if (m < 0 || m > 16) return fail(WFB_EINVAL, "%s: M (%lld) must be in 0..16", name, (long long)m);
  if (h <= 0 || h % 8 != 0 || h > k || k % WFB_QK_I2S != 0 || k > 4096)
    return fail(WFB_EINVAL, "%s: need H %% 8 == 0, H <= K <= 4096, K %% %d == 0 (got H=%lld K=%lld)", name, WFB_QK_I2S,
                (long long)h, (long long)k);
  if (n <= 0 || n % 64 != 0 || n * (k / 4) > INT32_MAX)
    return fail(WFB_EINVAL, "%s: N (%lld) must be 2 x a multiple of 32 with N*K/4 below 2^31", name, (long long)n);
  if (ldx < h || ldo < n / 2) return fail(WFB_EINVAL, "%s: row strides too small", name);
  if (!(eps >= 0.0f)) return fail(WFB_EINVAL, "%s: eps must be >= 0", name);
  if (m == 0) return ok();
  if (!x || !qweight || !w_scales_dev || !out) return fail(WFB_EINVAL, "%s: null pointer", name);
  const int esz = x_dtype == WFB_F32 ? 4 : 2;
  if (!aligned(x, 16) || (ldx * esz) % 16 != 0 || (gamma && !aligned(gamma, 16)) || !aligned(qweight, 16))
    return fail(WFB_EINVAL, "%s: x rows, gamma and qweight must be 16-byte aligned", name);
  wfb::Epilogue e{};
  e.nseg = 2;
  e.seg_end[0] = (int)(n / 2);
  e.ws_dev = w_scales_dev;
  e.out = out;
  e.out_dtype = WFB_F32;
  e.ldo = ldo;
  e.mid_dtype = mid_dtype;
  const wfb::NormSrc ns{x, x_dtype, ldx, gamma, gamma_dtype, eps, (int)h};
  if (m == 1)  // one token: the GEMV with gate and up rows side by side in each workgroup
    return hip_status(wfb::launch_gemv_i2s_norm_glu(qweight, (int)n, (int)k, e, ns, act_kind, as_stream(stream)), name);
  return hip_status(wfb::launch_skinny_lds(qweight, (int)n, (int)k, nullptr, (int)m, 0, e, act_kind, as_stream(stream), ns),
                    name);
}

int wfb_linear_i2s_glu(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m, int64_t lda,
                       const float* a_scale, const float* w_scales_dev, int act_kind, int mid_dtype, float* out,
                       int64_t ldo, void* stream) {
  const char* name = "wfb_linear_i2s_glu";
  if (act_kind != WFB_ACT_SILU && act_kind != WFB_ACT_RELU2) return fail(WFB_EINVAL, "%s: bad activation %d", name, act_kind);
  if (mid_dtype != WFB_F32 && mid_dtype != WFB_BF16)
    return fail(WFB_EINVAL, "%s: mid dtype must be WFB_F32 or WFB_BF16", name);
  if (m < 0 || m > 64) return fail(WFB_EINVAL, "%s: M (%lld) must be in 0..64", name, (long long)m);
  if (n <= 0 || n % 64 != 0 || k <= 0 || k % WFB_QK_I2S != 0)
    return fail(WFB_EINVAL, "%s: N (%lld) must be 2 x a multiple of 32 and K (%lld) a multiple of %d", name,
                (long long)n, (long long)k, WFB_QK_I2S);
  if (n * (k / 4) > INT32_MAX || (m > 0 && (m - 1) * lda + k > INT32_MAX))
    return fail(WFB_EINVAL, "%s: sizes too large for 32-bit offsets", name);
  if (lda < k || lda % 16 != 0) return fail(WFB_EINVAL, "%s: activation row stride must be >= K and a multiple of 16", name);
  if (ldo < n / 2) return fail(WFB_EINVAL, "%s: output row stride (%lld) < N/2 (%lld)", name, (long long)ldo, (long long)(n / 2));
  if (m == 0) return ok();
  if (!qweight || !act || !w_scales_dev || !out) return fail(WFB_EINVAL, "%s: null pointer", name);
  if (!aligned(qweight, 16) || !aligned(act, 16)) return fail(WFB_EINVAL, "%s: qweight and activations must be 16-byte aligned", name);
  wfb::Epilogue e{};
  e.nseg = 2;
  e.seg_end[0] = (int)(n / 2);
  e.a_scale = a_scale;
  e.ws_dev = w_scales_dev;
  e.out = out;
  e.out_dtype = WFB_F32;
  e.ldo = ldo;
  e.mid_dtype = mid_dtype;
  return hip_status(wfb::launch_gemm_i2s_glu(qweight, (int)n, (int)k, act, (int)m, lda, act_kind, e, as_stream(stream)),
                    name);
}

int wfb_rope_tables(double theta, int64_t head_dim, int64_t max_len, float* cos_out, float* sin_out) {
  const char* name = "wfb_rope_tables";
  if (!(theta > 0.0) || head_dim < 2 || head_dim % 2 != 0 || max_len < 1)
    return fail(WFB_EINVAL, "%s: bad theta / head_dim / max_len", name);
  if (!cos_out || !sin_out) return fail(WFB_EINVAL, "%s: null output", name);
  const int64_t half = head_dim / 2;
  for (int64_t i = 0; i < half; ++i) {
    const double inv = 1.0 / std::pow(theta, (double)(2 * i) / (double)head_dim);
    for (int64_t p = 0; p < max_len; ++p) {
      const double a = (double)p * inv;
      cos_out[p * half + i] = (float)std::cos(a);
      sin_out[p * half + i] = (float)std::sin(a);
    }
  }
  return ok();
}

}  // extern "C"
