/*
 * wfbitnet.h - C ABI of the MI355X (gfx950) ternary BitLinear hot path.
 *
 * One shared library, libwfbitnet.so, built from wrinklefree-monorepo_amd/csrc.
 * Every entry point:
 *   - takes plain device pointers and sizes (no torch or HIP types in the signature);
 *   - takes the HIP stream as `void* stream` (NULL = the default stream) and only enqueues
 *     work on it: nothing synchronises the host, nothing allocates device memory;
 *   - returns WFB_OK (0) or a negative status; the message of the last failure on the
 *     calling thread is returned by wfb_last_error().
 *
 * Packed weight layout ("I2_S", 2 bits per ternary weight, per-tensor fp32 scale):
 *   qweight is uint8 [N, K/4], row-major, K a multiple of 128.  Each row is split into
 *   128-weight blocks of 32 bytes; byte j of block b holds
 *       bits 7:6 -> k = 128b + j        bits 5:4 -> k = 128b + 32 + j
 *       bits 3:2 -> k = 128b + 64 + j   bits 1:0 -> k = 128b + 96 + j
 *   with code = w + 1 (00 -> -1, 01 -> 0, 10 -> +1; 11 never produced).
 *   Reference: packages/inference/scripts/convert_to_sglkernel.py:55-61, 96-111 and
 *   packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/inference/bitnet_engine.cpp:51-81.
 *
 * Reference citations below use
 *   SGB = packages/inference/extern/sglang-bitnet
 *   MSB = packages/inference/extern/BitNet
 *   WF  = packages/training/src/wrinklefree
 */
#ifndef WFBITNET_H
#define WFBITNET_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WFB_QK_I2S 128          /* weights per I2_S block (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.h:29) */
#define WFB_ABSMEAN_WS_DOUBLES 1024 /* workspace size (in doubles) of wfb_weight_absmean */
#define WFB_NORM_MAX_H 16384    /* largest row length of the per-token quantisers */
#define WFB_MAX_SEGMENTS 8      /* weight segments of one wfb_linear_i2s_segmented call */

/* status codes */
#define WFB_OK 0
#define WFB_EINVAL (-1)         /* bad argument (shape, dtype, alignment, null pointer) */
#define WFB_EHIP (-2)           /* the HIP runtime reported an error */

/* gated activations of wfb_glu_rmsnorm_quant_i8 */
#define WFB_ACT_SILU 1          /* silu(gate) * up (SwiGLU) */
#define WFB_ACT_RELU2 2         /* relu(gate)^2 * up */

/* element types of floating-point buffers */
#define WFB_F32 0
#define WFB_BF16 1
#define WFB_F16 2

/* Message of the last failed call on this thread ("" if none).  Replaces the thread-local
 * error of SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:86,167-169 (bitnet_get_error). */
const char* wfb_last_error(void);

/* Library ABI version (bumped on any signature change). */
int wfb_version(void);

/* ---- a1: offline pack -------------------------------------------------------------------- */

/* scale_dev[0] = mean(|w|) over numel elements, summed in fp64 in a fixed order (deterministic),
 * rounded to fp32; a mean below 1e-8 becomes 1.0.  workspace: >= WFB_ABSMEAN_WS_DOUBLES doubles
 * of device memory.  Replaces the scale of pack_ternary_sglkernel
 * (packages/inference/scripts/convert_to_sglkernel.py:81-85). */
int wfb_weight_absmean(const void* w, int w_dtype, int64_t numel, float* scale_dev,
                       double* workspace, void* stream);

/* qweight[N, K/4] = I2_S pack of clamp(round_half_even(w / scale), -1, 1), w row-major [N, K]
 * (row stride ldw elements).  scale is read from scale_dev[0].  Replaces the quantise + pack
 * loop of pack_ternary_sglkernel (convert_to_sglkernel.py:87-111). */
int wfb_pack_i2s(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw,
                 const float* scale_dev, uint8_t* qweight, void* stream);

/* w_out[N, K] int8 in {-1, 0, +1} from qweight (inspection / format conversion).
 * Same decode as the scalar reference dot, bitnet_engine.cpp:51-81. */
int wfb_unpack_i2s(const uint8_t* qweight, int64_t n, int64_t k, int8_t* w_out, void* stream);

/* Load-time conversion of the HF "offline" ternary layout to I2_S.
 *   packed_hf : uint8 [NB, K], NB = ceil(N/4); byte (j, k) = codes (w + 1) of column k of rows j, j+NB,
 *               j+2NB, j+3NB in bits 1:0, 3:2, 5:4, 7:6 (packages/inference/scripts/quantize_dlm_to_offline.py:27-98)
 *   qweight   : uint8 [N, k_pad/4] I2_S (columns K..k_pad-1 zero weights); 4*(NB-1) < N <= 4*NB,
 *               k_pad >= K a multiple of 128
 *   scale_out : fp32 [1] device.  scale_mode WFB_SCALE_REFERENCE: weight_scale * nnz / (4*NB*K) (< 1e-8 -> 1),
 *               what the reference converter's repack yields; WFB_SCALE_CHECKPOINT: weight_scale itself.
 *   weight_scale: read from weight_scale_dev[0] (scale_dtype WFB_F32 or WFB_BF16) or, if that is NULL,
 *               the host value weight_scale.
 *   workspace : WFB_CONVERT_WS(N, k_pad) int64 of device memory.
 * Replaces the offline branch of convert_checkpoint (packages/inference/scripts/convert_to_sglkernel.py:221-246). */
#define WFB_SCALE_REFERENCE 0
#define WFB_SCALE_CHECKPOINT 1
#define WFB_CONVERT_WS(n, k_pad) (((n) * ((k_pad) / 16) + 255) / 256)
int wfb_convert_hf_offline_i2s(const uint8_t* packed_hf, int64_t nb, int64_t n, int64_t k, int64_t k_pad,
                               const void* weight_scale_dev, int scale_dtype, float weight_scale,
                               int scale_mode, uint8_t* qweight, float* scale_out, int64_t* workspace,
                               void* stream);

/* ---- a2: activation quantisation ------------------------------------------------------- */

/* Per-token absmax int8 quantisation of x [M, H] (row stride ldx elements) into q [M, k_pad]
 * (row stride ldq bytes; columns H..k_pad-1 are written as 0) and a_scale[M]:
 *   mx = max|x_row| (mx < 1e-6 -> 1), a_scale = mx / 127, q = sat_i8(rint(x * (127 / mx))).
 * Row-wise restatement of quantize_activations_i8, SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:880-1135
 * (vector path: round half to even, saturating pack).  H <= WFB_NORM_MAX_H. */
int wfb_quantize_act_i8(const void* x, int x_dtype, int64_t m, int64_t h, int64_t ldx,
                        int8_t* q, int64_t k_pad, int64_t ldq, float* a_scale, void* stream);

/* Same quantiser with ONE scale for the whole buffer of numel elements (a_scale[0]), as the
 * reference op bitnet_quantize_activations_cpu does (SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:409-426). */
int wfb_quantize_act_i8_tensor(const void* x, int x_dtype, int64_t numel, int8_t* q,
                               float* a_scale, void* stream);

/* ---- a3: RMSNorm / SubLN fused with a2 --------------------------------------------------- */

/* y = x * (1 / sqrt(sum(x^2) / H + eps)) * gamma in fp32, then the per-token quantiser of
 * wfb_quantize_act_i8 on y.  Sum of squares in a fixed order.  H <= 4096: one wave per row, lane l
 * accumulates elements (l + 64*j)*8 + e, j ascending, e = 0..7, then a xor butterfly over the wave
 * (offsets 32,16,8,4,2,1).  H > 4096: each of 256 threads accumulates elements (it*256 + t)*8 + e,
 * it ascending, e = 0..7, then the butterfly per wave and the 4 wave sums added in wave order.
 * gamma may be NULL (no affine).  Replaces SubLN.forward / RMSNorm.forward (WF/models/subln.py:42-59, 64-97) followed
 * by activation quantisation (WF/models/bitlinear.py:66-84).  H % 8 == 0, H <= WFB_NORM_MAX_H. */
int wfb_rmsnorm_quant_i8(const void* x, int x_dtype, int64_t ldx, const void* gamma, int gamma_dtype,
                         float eps, int64_t m, int64_t h, int8_t* q, int64_t k_pad, int64_t ldq,
                         float* a_scale, void* stream);

/* ---- a4 / a5 / a6: ternary BitLinear forward --------------------------------------------- */

/* acc[m, n] = sum_k w[n, k] * act[m, k]        (int32, exact)
 * y[m, n]   = ((float)acc * w_scale) * a_scale[m]  (+ bias[n]), stored as out_dtype
 *
 *   qweight : uint8 [N, K/4] I2_S, 16-byte aligned
 *   act     : int8  [M, K] with row stride lda bytes (lda % 16 == 0, 16-byte aligned)
 *   a_scale : fp32 [M] device, or NULL for 1.0
 *   w_scale_dev : fp32 [1] device, or NULL to use the host value w_scale (no host sync either way)
 *   bias    : [N] of bias_dtype, or NULL
 *   out     : [M, N] of out_dtype (WFB_F32 or WFB_BF16) with row stride ldo elements, or NULL
 *   acc_out : int32 [M, N] with row stride ldo, or NULL (parity / debugging)
 *
 * wfb_linear_i2s picks the kernel from (M, N, K).  wfb_gemv_i2s forces the VALU decode GEMV
 * (M <= 2, K <= 32768, N*K/4 < 2^31) and wfb_gemm_i2s forces the int8-MFMA GEMM (any M).  All three give identical acc.
 * Replace bitnet_gemv_cpu / bitnet_gemm_cpu (SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:331-406,
 * kernels SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:325-874) and the rescale of
 * BitNetLinearMethod.apply (SGB/python/sglang/srt/layers/quantization/bitnet.py:232-253). */
int wfb_linear_i2s(const uint8_t* qweight, int64_t n, int64_t k,
                   const int8_t* act, int64_t m, int64_t lda,
                   const float* a_scale, const float* w_scale_dev, float w_scale,
                   const void* bias, int bias_dtype,
                   void* out, int out_dtype, int64_t ldo, int32_t* acc_out, void* stream);

int wfb_gemv_i2s(const uint8_t* qweight, int64_t n, int64_t k,
                 const int8_t* act, int64_t m, int64_t lda,
                 const float* a_scale, const float* w_scale_dev, float w_scale,
                 const void* bias, int bias_dtype,
                 void* out, int out_dtype, int64_t ldo, int32_t* acc_out, void* stream);

int wfb_gemm_i2s(const uint8_t* qweight, int64_t n, int64_t k,
                 const int8_t* act, int64_t m, int64_t lda,
                 const float* a_scale, const float* w_scale_dev, float w_scale,
                 const void* bias, int bias_dtype,
                 void* out, int out_dtype, int64_t ldo, int32_t* acc_out, void* stream);

/* ---- fused decode layer pieces ------------------------------------------------------------ */

/* One wfb_linear_i2s over weights that are the row-wise concatenation of n_seg projections sharing
 * the same input (fused QKV: q|k|v; gate+up: gate|up), each with its own per-tensor scale:
 *   qweight  : uint8 [N, K/4], rows of segment s are [sum(seg_rows[:s]), sum(seg_rows[:s+1]))
 *   seg_rows : host array of n_seg row counts, each a multiple of 8, summing to N (1 <= n_seg <= 8)
 *   w_scales_dev : fp32 [n_seg] device
 *   out[m, n] = ((float)acc[m, n] * w_scales_dev[seg(n)]) * a_scale[m] (+ bias[n])
 * Accumulators and outputs equal those of n_seg separate wfb_linear_i2s calls on the segments.
 * Intent of the fused QKV / gate-up GEMVs of SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:150-231,
 * 289-375 (each projection scaled by its own weight scale; the reference's double sum(a) subtraction
 * and missing weight scales are not reproduced) and the segment scale lookup of the MS CUDA kernel
 * (MSB/gpu/bitnet_kernels/bitnet_kernels.h:80-82). */
int wfb_linear_i2s_segmented(const uint8_t* qweight, int64_t n, int64_t k, int n_seg, const int64_t* seg_rows,
                             const float* w_scales_dev, const int8_t* act, int64_t m, int64_t lda,
                             const float* a_scale, const void* bias, int bias_dtype,
                             void* out, int out_dtype, int64_t ldo, int32_t* acc_out, void* stream);

/* Gated activation fused with SubLN and the per-token quantiser, the middle of the BitNet MLP
 * (gate|up GEMV -> this -> down GEMV):
 *   v = act(gate[m, :H]) * up[m, :H]  (fp32; gate and up rows share the row stride ldx)
 *   then exactly wfb_rmsnorm_quant_i8 on v (same reduction order, gamma = the FFN SubLN weight).
 * act = WFB_ACT_SILU: silu(g) = g / (1 + 2^(-g*log2(e))) with 2^x evaluated as 2^n * p(x - n)
 * (n = rint(x) clamped to [-125, 125], p a degree-7 Taylor polynomial of 2^f in Horner form), every
 * step one correctly rounded fp32 operation, so a float32 CPU restatement reproduces it bit for bit;
 * against exact silu: relative error below 1e-6 for |g| <= 16, absolute error below 2e-6 everywhere
 * (finite inputs).  act = WFB_ACT_RELU2: max(g, 0)^2 * u.
 * Replaces the relu^2 * up -> rms_norm -> quantize steps of bitnet_mlp_fused
 * (SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:200-216) and SiLU-gated MLP + SubLN of the
 * stage-1 model (WF/models/subln.py:42-59; WF/training/stage1.py:63-214).
 * H % 8 == 0, H <= WFB_NORM_MAX_H. */
int wfb_glu_rmsnorm_quant_i8(const void* gate, const void* up, int x_dtype, int64_t ldx, int act,
                             const void* gamma, int gamma_dtype, float eps, int64_t m, int64_t h,
                             int8_t* q, int64_t k_pad, int64_t ldq, float* a_scale, void* stream);

/* The BitLinear with the residual connection fused into the epilogue:
 *   out[m, n] = ((float)acc * w_scale) * a_scale[m] + residual[m, n]   (fp32 add, then out_dtype)
 * residual [M, N] of residual_dtype (WFB_F32 or WFB_BF16, row stride ldr); out may be the residual
 * buffer itself (each element is read and written by the same thread).  Other arguments as
 * wfb_linear_i2s.  Replaces the linear + residual add of the engine's layer step
 * (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:517-536: hidden = residual + attn_out / mlp_out). */
int wfb_linear_i2s_residual(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m,
                            int64_t lda, const float* a_scale, const float* w_scale_dev, float w_scale,
                            const void* residual, int residual_dtype, int64_t ldr, void* out, int out_dtype,
                            int64_t ldo, void* stream);

/* ---- greedy decoding: LM head + argmax ------------------------------------------------------ */

/* uint64 elements of the workspace of the argmax entry points for M tokens and N vocabulary rows
 * (one slot per 16 rows and token; every call writes all slots it reads, no initialisation needed). */
#define WFB_ARGMAX_WS(m, n) ((((n) + 15) / 16) * (m))

/* Ternary LM head with the greedy pick fused in: the logits of wfb_linear_i2s (no bias), rounded to
 * logits_dtype (WFB_F32 or WFB_BF16), are stored to logits [M, N] (row stride ldo) unless logits is
 * NULL, and token_out[m] (int64, device) = the first index of the maximal logit of token m.
 * M <= 64; N*K/4 and (M-1)*lda + K below 2^31.  workspace: WFB_ARGMAX_WS(M, N) uint64 of device memory.
 * Replaces the packed lm_head of the engine (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:544-549;
 * packed by packages/inference/scripts/convert_to_sglkernel.py:264-286) and its greedy
 * std::max_element (bitnet_engine.cpp:774-779). */
int wfb_linear_i2s_argmax(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m,
                          int64_t lda, const float* a_scale, const float* w_scale_dev, float w_scale,
                          void* logits, int logits_dtype, int64_t ldo, uint64_t* workspace,
                          int64_t* token_out, void* stream);

/* Dense LM head (e.g. a tied embedding) with the final RMSNorm and the greedy pick fused in:
 *   y[m, :] = x[m, :] * (1 / sqrt(sum(x[m, :]^2) / H + eps)) * gamma   (fp32, rounded to x_dtype)
 *   logits[m, v] = sum_k y[m, k] * weight[v, k]                        (fp32 accumulation)
 *   token_out[m] = first index of the maximal logits[m, :]
 * x [M, H] of x_dtype (row stride ldx), gamma [H] or NULL, weight [N, H] of w_dtype (row stride ldw,
 * a multiple of 8, 16-byte aligned); x_dtype and w_dtype WFB_F32 or WFB_BF16; logits fp32 [M, N]
 * (row stride ldo) or NULL.  M <= 16, H % 8 == 0, M*H <= 16384, N*ldw*elem_size < 2^31.
 * Replaces the final rms_norm + fp32_linear + greedy pick of the engine
 * (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:539-553, 774-779). */
int wfb_lm_head_argmax(const void* x, int x_dtype, int64_t ldx, const void* gamma, int gamma_dtype,
                       float eps, const void* weight, int w_dtype, int64_t ldw, int64_t m, int64_t n,
                       int64_t h, float* logits, int64_t ldo, uint64_t* workspace, int64_t* token_out,
                       void* stream);

/* ---- rotary tables ------------------------------------------------------------------------- */

/* Host buffers cos_out / sin_out fp32 [max_len, head_dim/2] of the HF rotate-half rotary embedding:
 * angle(p, i) = p * theta^(-2i / head_dim), evaluated in double precision (pow, product, cos / sin of
 * the C library) and rounded once to float, so every caller that takes its tables from here uses the
 * same values.  Host memory only; touches no GPU.  head_dim even and >= 2, max_len >= 1, theta > 0.
 * The angles of the stage-1 HF model's rotary embedding (WF/training/stage1.py:169-214; the reference
 * C engine has none, SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:381-441). */
int wfb_rope_tables(double theta, int64_t head_dim, int64_t max_len, float* cos_out, float* sin_out);

/* ---- GQA decode attention over a KV cache (one new token per sequence) --------------------- */

/* For each sequence b < batch at position p = pos[b] (device int64 [batch]):
 *   1. rotary embedding (HF rotate-half form) of the new query heads q[b] and key k_new[b] with
 *      rope_cos/rope_sin [max_len, head_dim/2] fp32 (row p), each product and sum an fp32 operation,
 *      the result rounded to dtype; both tables NULL = no rotary embedding (the C engine's form);
 *   2. k_cache[b, kvh, p, :] = rotated key, v_cache[b, kvh, p, :] = v_new[b, kvh, :]
 *      (caches [batch, num_kv_heads, max_len, head_dim] of dtype, 16-byte aligned);
 *   3. out[b, h*D:(h+1)*D] = softmax_j(q_h . K[b, h/G, j] * scale) @ V[b, h/G, j], j = 0..p,
 *      G = num_heads / num_kv_heads (query head h reads kv head h / G), fp32 math, stored as dtype.
 * q [batch, num_heads*head_dim] (row stride ldq), k_new/v_new [batch, num_kv_heads*head_dim] (ldk,
 * ldv), out row stride ldo, all in elements.  dtype WFB_F32 or WFB_BF16 for every buffer;
 * head_dim 64 or 128; G <= 8.  A position outside [0, max_len) writes NaN to that sequence's output
 * and leaves the cache untouched (positions live on the device and are not checked on the host).
 * workspace: WFB_ATTN_WS(batch, num_heads, head_dim, max_len) floats of device memory for the
 * split-context pass (keys cut into 64-key splits, doubled only while splits x query heads per kv head
 * would pass 4096, the combine's LDS staging; chosen from max_len alone; merged by a second kernel), or
 * NULL for one workgroup per (kv head, sequence) over all keys.
 * Replaces attention_forward (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:381-441) with the
 * cache writes of kv_cache_update_key / kv_cache_update_value
 * (SGB/sgl-kernel/csrc/inference/kv_cache.h:81-101) and the rotary embedding of the stage-1 HF model
 * (WF/training/stage1.py:169-214). */
#define WFB_ATTN_WS(batch, num_heads, head_dim, max_len) \
  ((batch) * (num_heads) * ((head_dim) + 2) * (((max_len) + 63) / 64))
int wfb_gqa_decode_attention(const void* q, int64_t ldq, const void* k_new, int64_t ldk,
                             const void* v_new, int64_t ldv, int dtype,
                             const float* rope_cos, const float* rope_sin,
                             void* k_cache, void* v_cache, int64_t max_len, const int64_t* pos,
                             int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                             float scale, void* out, int64_t ldo, float* workspace, void* stream);

/* wfb_gqa_decode_attention without the workspace argument, allocating nothing.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The split partials go to a scratch array the
 * library holds on each GPU for the life of the process: WFB_ATTN_SCRATCH_FLOATS floats (32 MiB);
 * sizes whose partials would not fit are rejected with WFB_EINVAL (the exact need is
 * batch * num_heads * (head_dim + 2) * splits, at most WFB_ATTN_WS(...)).  Same arguments, checks and
 * results as wfb_gqa_decode_attention with a workspace.  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (other streams, other threads) race; calls ordered on one
 * stream do not.  Nothing in it needs clearing between calls (each split writes all it is read for).
 * The scratch used is that of the stream's device (the current device for the null stream), whichever
 * device is current. */
#define WFB_ATTN_SCRATCH_FLOATS (8 * 1024 * 1024)
int wfb_gqa_decode_attention_noalloc(const void* q, int64_t ldq, const void* k_new, int64_t ldk,
                                     const void* v_new, int64_t ldv, int dtype,
                                     const float* rope_cos, const float* rope_sin,
                                     void* k_cache, void* v_cache, int64_t max_len, const int64_t* pos,
                                     int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                     float scale, void* out, int64_t ldo, void* stream);

/* Causal GQA attention of a prefill chunk: T new tokens per sequence at positions start .. start+T-1.
 * Rotary embedding of the new queries and keys (rope_cos / rope_sin fp32 [max_len, head_dim/2], or both
 * NULL for none), cache append of the T keys and values at their positions, then for token i of
 * sequence b and query head h: softmax(q . k_j * scale, j = 0 .. start+i) . v over the cache of kv head
 * h / (num_heads / num_kv_heads).  bf16 only (dtype WFB_BF16): q rows [batch*T, ldq] (row b*T + i holds
 * the num_heads*head_dim query elements), k_new / v_new rows [batch*T, ldk / ldv] (num_kv_heads*head_dim
 * each); the three may be column slices of one q|k|v projection output.  Caches [batch, num_kv_heads,
 * max_len, head_dim], 16-byte aligned, as are q, out and the rope tables; out [batch*T, ldo]
 * (num_heads*head_dim per row).  head_dim 64 or
 * 128, num_heads / num_kv_heads in 1..8, start + T <= max_len, row strides multiples of 8 elements and
 * row bases 16-byte aligned.  The cache rows written are bit-identical to the rotary + append of the
 * decode call; scores, softmax and the weighted sum are fp32 (products of bf16 operands on the matrix
 * cores, the probabilities as two bf16 parts), the output rounded to bf16.
 * Replaces attention_forward (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:381-441) run once per
 * prompt token, with the cache writes of kv_cache_update_key / kv_cache_update_value
 * (SGB/sgl-kernel/csrc/inference/kv_cache.h:81-101) and the stage-1 rotary embedding
 * (WF/training/stage1.py:169-214). */
int wfb_gqa_prefill_attention(const void* q, int64_t ldq, const void* k_new, int64_t ldk,
                              const void* v_new, int64_t ldv, int dtype,
                              const float* rope_cos, const float* rope_sin,
                              void* k_cache, void* v_cache, int64_t max_len, int64_t start,
                              int64_t batch, int64_t t, int64_t num_heads, int64_t num_kv_heads,
                              int64_t head_dim, float scale, void* out, int64_t ldo, void* stream);

/* Decode-time fusion of wfb_rmsnorm_quant_i8 and the BitLinear that consumes its codes (one launch):
 *   q, a_scale = rmsnorm_quant(x, gamma, eps)          (exactly wfb_rmsnorm_quant_i8, codes zero past H)
 *   out = linear_i2s_segmented(qweight, q, a_scale)      (exactly wfb_linear_i2s_segmented; one segment =
 *                                                         wfb_linear_i2s with a device scale)
 *         (+ residual, exactly as wfb_linear_i2s_residual when residual is not NULL)
 * x [M, H] (x_dtype WFB_F32 or WFB_BF16, row stride ldx elements, rows 16-byte aligned), gamma [H]
 * (WFB_F32 or WFB_BF16, 16-byte aligned) or NULL; H % 8 == 0, H <= K and either M == 1 with K <= 16384
 * (the decode GEMV's prologue: every workgroup forms the row's codes in LDS in the quantiser's order for
 * the row length) or 2 <= M <= 16 with K <= 4096 (the LDS-staged batched kernel's prologue); N * K / 4
 * below 2^31; other sizes take the two-call path.  seg_rows /
 * w_scales_dev as wfb_linear_i2s_segmented (n_seg = 1 with seg_rows NULL: one segment of N rows).
 * out [M, N] WFB_F32 or WFB_BF16 (row stride ldo); residual [M, N] WFB_F32 or WFB_BF16 (row stride ldr)
 * or NULL; out may alias residual.  Every workgroup recomputes the codes of the M rows in the
 * quantiser's own summation order, so results are bit-identical to the two calls.
 * Replaces, per decode token, SubLN/RMSNorm -> activation_quant -> BitLinear
 * (WF/models/subln.py:42-59, 64-97; WF/models/bitlinear.py:66-113) as fused by
 * bitnet_qkv_fused / bitnet_mlp_fused (SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:150-231, 289-375). */
int wfb_rmsnorm_linear_i2s(const void* x, int x_dtype, int64_t ldx, const void* gamma, int gamma_dtype, float eps,
                           int64_t m, int64_t h, const uint8_t* qweight, int64_t n, int64_t k, int n_seg,
                           const int64_t* seg_rows, const float* w_scales_dev, const void* residual,
                           int residual_dtype, int64_t ldr, void* out, int out_dtype, int64_t ldo, void* stream);

/* The MLP's first half for a decode batch in one launch: RMSNorm + per-token int8 quantisation of x in the
 * prologue (exactly wfb_rmsnorm_quant_i8's codes and scales), the gate|up projection, and the gated
 * product in the epilogue (exactly wfb_linear_i2s_glu on those codes):
 *   out[m, j] = act(y[m, j]) * y[m, half + j],  y = linear_i2s_segmented(qweight, rmsnorm_quant(x, gamma, eps))
 * x, gamma, M, H, K as wfb_rmsnorm_linear_i2s (M <= 16, H % 8 == 0, H <= K <= 4096); qweight gate|up
 * (N = 2 * half rows, half % 32 == 0), w_scales_dev[2]; act_kind / mid_dtype / out [M, half] fp32 (row
 * stride ldo) as wfb_linear_i2s_glu.  Replaces, per decode token, RMSNorm -> activation_quant -> gate and
 * up BitLinears -> act(gate) * up of bitnet_mlp_fused (SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:289-375,
 * 189-216). */
int wfb_rmsnorm_linear_i2s_glu(const void* x, int x_dtype, int64_t ldx, const void* gamma, int gamma_dtype, float eps,
                               int64_t m, int64_t h, const uint8_t* qweight, int64_t n, int64_t k,
                               const float* w_scales_dev, int act_kind, int mid_dtype, float* out, int64_t ldo,
                               void* stream);

/* The gated MLP middle in the gate|up linear's epilogue (decode batches, M <= 64):
 *   out[m, j] = act(y[m, j]) * y[m, half + j],  j < half = N / 2,
 * where y is exactly what wfb_linear_i2s_segmented stores for qweight = gate|up (two segments of half
 * rows, w_scales_dev[2]) with out_dtype = mid_dtype (WFB_F32 or WFB_BF16), and act(g) * u is formed
 * with the same fixed fp32 operations as wfb_glu_rmsnorm_quant_i8 (act WFB_ACT_SILU / WFB_ACT_RELU2).
 * out: fp32 [M, half], row stride ldo.  So wfb_rmsnorm_quant_i8 on out gives, bit for bit, the codes
 * of wfb_glu_rmsnorm_quant_i8 on the stored gate and up.  half % 32 == 0; N * K / 4 and
 * (M - 1) * lda + K below 2^31.  Replaces the gate/up GEMV + act * up of bitnet_mlp_fused
 * (SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:189-216). */
int wfb_linear_i2s_glu(const uint8_t* qweight, int64_t n, int64_t k, const int8_t* act, int64_t m, int64_t lda,
                       const float* a_scale, const float* w_scales_dev, int act_kind, int mid_dtype, float* out,
                       int64_t ldo, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WFBITNET_H */
