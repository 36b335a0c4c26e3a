/*
 * Greedy decoding of the stage-1 BitNet Llama model on the host CPU -- the END-TO-END CPU BASELINE that
 * bench.py times beside the GPU (test infrastructure; never linked into libwfbitnet).
 *
 * It restates the reference's native CPU engine loop (packages/inference/extern/sglang-bitnet/sgl-kernel/
 * csrc/inference/bitnet_engine.cpp, ENG below) over this repository's model: every token, prompt included,
 * runs through one forward_one_token (ENG:490-554): embedding row, per layer RMSNorm -> quantised q/k/v
 * -> attention over an fp32 KV cache (ENG:381-441) -> SubLN -> o -> residual, RMSNorm -> gate/up ->
 * act(gate) * up -> SubLN -> down -> residual; final RMSNorm, fp32 LM head, first-maximum argmax
 * (ENG:774-779).  Each BitLinear quantises its input per token (ENG:262-285) and runs the AVX2 port of the
 * reference I2_S GEMV (i2s_cpu_avx2.c, OpenMP over output rows); the dense fp32 LM head and the heads of the
 * attention are OpenMP loops too.  Differences from ENG, as in the GPU model: the rotary embedding of the
 * stage-1 model (ENG has none, reference anomaly v), SubLN with its own eps, the activation from the model
 * (silu or relu^2), and one quantisation shared by the projections that read the same input.
 *
 * Floating point is fp32 throughout in straightforward order; it is a throughput baseline, pinned against
 * the GPU model's logits by a tolerance (tests/test_gpu_e2e.py), not a bit-exact restatement.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <immintrin.h>

int cpu_gemv_i2s_avx2(int n_out, int k, float* out, const uint8_t* w, const int8_t* a, float scale);

/* Model description: every array contiguous fp32 / uint8, per-layer blocks stacked along the first axis. */
typedef struct {
  int32_t layers, hidden, inter, heads, kv_heads, head_dim, vocab, max_len;
  int32_t kpad_h, kpad_qd, kpad_f;  /* packed row lengths (multiples of 128) of the three input widths */
  int32_t act;                      /* 1 = silu, 2 = relu^2 */
  float rms_eps, subln_eps;
  const float* embed;               /* [vocab, hidden] */
  const float* head;                /* [vocab, hidden] fp32 LM head (the embedding when tied) */
  const float* final_norm;          /* [hidden] */
  const float* in_norm;             /* [layers, hidden] */
  const float* post_norm;           /* [layers, hidden] */
  const float* attn_sub;            /* [layers, heads * head_dim] */
  const float* ffn_sub;             /* [layers, inter] */
  const float* scales;              /* [layers, 7]: q k v o gate up down */
  const uint8_t* wq;                /* [layers, heads * head_dim, kpad_h / 4] */
  const uint8_t* wk;                /* [layers, kv_heads * head_dim, kpad_h / 4] */
  const uint8_t* wv;                /* [layers, kv_heads * head_dim, kpad_h / 4] */
  const uint8_t* wo;                /* [layers, hidden, kpad_qd / 4] */
  const uint8_t* wg;                /* [layers, inter, kpad_h / 4] */
  const uint8_t* wu;                /* [layers, inter, kpad_h / 4] */
  const uint8_t* wd;                /* [layers, hidden, kpad_f / 4] */
  const float* rope_cos;            /* [max_len, head_dim / 2] */
  const float* rope_sin;            /* [max_len, head_dim / 2] */
} cpu_model;

static void rms_norm(float* out, const float* x, const float* w, int n, float eps) {
  float ss = 0.0f;
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  const float r = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) out[i] = x[i] * r * w[i];
}

/* per-token absmax int8 of n values into kpad bytes (zeros past n); returns the token scale max / 127 */
static float quantize(int8_t* q, const float* x, int n, int kpad) {
  float mx = 0.0f;
  for (int i = 0; i < n; ++i) mx = fmaxf(mx, fabsf(x[i]));
  if (mx < 1e-6f) mx = 1.0f;
  const float inv = 127.0f / mx;
  for (int i = 0; i < n; ++i) {
    float r = nearbyintf(x[i] * inv);
    q[i] = (int8_t)(r > 127.0f ? 127.0f : r < -128.0f ? -128.0f : r);
  }
  memset(q + n, 0, (size_t)(kpad - n));
  return mx / 127.0f;
}

/* HF rotate-half rotary embedding of one head at position p */
static void rope(float* v, const cpu_model* m, int p) {
  const int h2 = m->head_dim / 2;
  const float* c = m->rope_cos + (size_t)p * h2;
  const float* s = m->rope_sin + (size_t)p * h2;
  for (int i = 0; i < h2; ++i) {
    const float a = v[i], b = v[i + h2];
    v[i] = a * c[i] - b * s[i];
    v[i + h2] = b * c[i] + a * s[i];
  }
}

static float dot_f32(const float* a, const float* b, int n) {
  __m256 acc = _mm256_setzero_ps();
  int i = 0;
  for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
  float t[8];
  _mm256_storeu_ps(t, acc);
  float s = t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];
  for (; i < n; ++i) s += a[i] * b[i];
  return s;
}

typedef struct {
  float *x, *xn, *q, *k, *v, *att, *gate, *up, *tmp, *logits, *kc, *vc, *scores;
  int8_t* codes;
} bufs;

static void free_bufs(bufs* b) {
  free(b->x); free(b->xn); free(b->q); free(b->k); free(b->v); free(b->att); free(b->gate); free(b->up);
  free(b->tmp); free(b->logits); free(b->kc); free(b->vc); free(b->scores); free(b->codes);
}

static int token_forward(const cpu_model* m, bufs* b, int32_t tok, int pos) {
  const int H = m->hidden, F = m->inter, hd = m->head_dim, qd = m->heads * hd, kvd = m->kv_heads * hd;
  const int g = m->heads / m->kv_heads;
  memcpy(b->x, m->embed + (size_t)tok * H, (size_t)H * sizeof(float));
  for (int l = 0; l < m->layers; ++l) {
    const float* sc = m->scales + 7 * l;
    /* attention block */
    rms_norm(b->xn, b->x, m->in_norm + (size_t)l * H, H, m->rms_eps);
    float as = quantize(b->codes, b->xn, H, m->kpad_h);
    cpu_gemv_i2s_avx2(qd, m->kpad_h, b->q, m->wq + (size_t)l * qd * (m->kpad_h / 4), b->codes, sc[0] * as);
    cpu_gemv_i2s_avx2(kvd, m->kpad_h, b->k, m->wk + (size_t)l * kvd * (m->kpad_h / 4), b->codes, sc[1] * as);
    cpu_gemv_i2s_avx2(kvd, m->kpad_h, b->v, m->wv + (size_t)l * kvd * (m->kpad_h / 4), b->codes, sc[2] * as);
    for (int h = 0; h < m->heads; ++h) rope(b->q + h * hd, m, pos);
    for (int h = 0; h < m->kv_heads; ++h) rope(b->k + h * hd, m, pos);
    float* kc = b->kc + (size_t)l * m->max_len * kvd;
    float* vc = b->vc + (size_t)l * m->max_len * kvd;
    memcpy(kc + (size_t)pos * kvd, b->k, (size_t)kvd * sizeof(float));
    memcpy(vc + (size_t)pos * kvd, b->v, (size_t)kvd * sizeof(float));
    const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < m->heads; ++h) {
      const int kh = h / g;
      float* sco = b->scores + (size_t)h * m->max_len;
      float mx = -INFINITY;
      for (int p = 0; p <= pos; ++p) {
        sco[p] = dot_f32(b->q + h * hd, kc + (size_t)p * kvd + kh * hd, hd) * scale;
        mx = fmaxf(mx, sco[p]);
      }
      float sum = 0.0f;
      for (int p = 0; p <= pos; ++p) {
        sco[p] = expf(sco[p] - mx);
        sum += sco[p];
      }
      float* o = b->att + h * hd;
      for (int d = 0; d < hd; ++d) o[d] = 0.0f;
      for (int p = 0; p <= pos; ++p) {
        const float w = sco[p] / sum;
        const float* vp = vc + (size_t)p * kvd + kh * hd;
        for (int d = 0; d < hd; ++d) o[d] += w * vp[d];
      }
    }
    rms_norm(b->att, b->att, m->attn_sub + (size_t)l * qd, qd, m->subln_eps);
    as = quantize(b->codes, b->att, qd, m->kpad_qd);
    cpu_gemv_i2s_avx2(H, m->kpad_qd, b->tmp, m->wo + (size_t)l * H * (m->kpad_qd / 4), b->codes, sc[3] * as);
    for (int i = 0; i < H; ++i) b->x[i] += b->tmp[i];
    /* MLP block */
    rms_norm(b->xn, b->x, m->post_norm + (size_t)l * H, H, m->rms_eps);
    as = quantize(b->codes, b->xn, H, m->kpad_h);
    cpu_gemv_i2s_avx2(F, m->kpad_h, b->gate, m->wg + (size_t)l * F * (m->kpad_h / 4), b->codes, sc[4] * as);
    cpu_gemv_i2s_avx2(F, m->kpad_h, b->up, m->wu + (size_t)l * F * (m->kpad_h / 4), b->codes, sc[5] * as);
    for (int i = 0; i < F; ++i) {
      const float gv = b->gate[i];
      const float a = m->act == 2 ? (gv > 0.0f ? gv * gv : 0.0f) : gv / (1.0f + expf(-gv));
      b->gate[i] = a * b->up[i];
    }
    rms_norm(b->gate, b->gate, m->ffn_sub + (size_t)l * F, F, m->subln_eps);
    as = quantize(b->codes, b->gate, F, m->kpad_f);
    cpu_gemv_i2s_avx2(H, m->kpad_f, b->tmp, m->wd + (size_t)l * H * (m->kpad_f / 4), b->codes, sc[6] * as);
    for (int i = 0; i < H; ++i) b->x[i] += b->tmp[i];
  }
  rms_norm(b->xn, b->x, m->final_norm, H, m->rms_eps);
#pragma omp parallel for schedule(static)
  for (int v = 0; v < m->vocab; ++v) b->logits[v] = dot_f32(m->head + (size_t)v * H, b->xn, H);
  int best = 0;
  for (int v = 1; v < m->vocab; ++v)
    if (b->logits[v] > b->logits[best]) best = v;
  return best;
}

/* Greedy decoding: the n_prompt prompt tokens one by one, then n_new generated tokens into out (each run
 * through the model as well, except the last).  logits_out (optional, [vocab]): the logits after the
 * prompt.  Returns 0, or -1 on bad sizes or allocation failure. */
int cpu_decode_greedy(const cpu_model* m, const int32_t* prompt, int n_prompt, int n_new, int32_t* out,
                      float* logits_out) {
  if (!m || !prompt || n_prompt < 1 || n_new < 0 || n_prompt + n_new > m->max_len || m->heads % m->kv_heads ||
      m->kpad_h % 128 || m->kpad_qd % 128 || m->kpad_f % 128 || m->kpad_h < m->hidden || m->kpad_f < m->inter ||
      m->kpad_qd < m->heads * m->head_dim)
    return -1;
  const int H = m->hidden, F = m->inter, qd = m->heads * m->head_dim, kvd = m->kv_heads * m->head_dim;
  int kmax = m->kpad_h > m->kpad_qd ? m->kpad_h : m->kpad_qd;
  if (m->kpad_f > kmax) kmax = m->kpad_f;
  bufs b;
  b.x = malloc(sizeof(float) * H); b.xn = malloc(sizeof(float) * H); b.q = malloc(sizeof(float) * qd);
  b.k = malloc(sizeof(float) * kvd); b.v = malloc(sizeof(float) * kvd); b.att = malloc(sizeof(float) * qd);
  b.gate = malloc(sizeof(float) * F); b.up = malloc(sizeof(float) * F); b.tmp = malloc(sizeof(float) * H);
  b.logits = malloc(sizeof(float) * m->vocab);
  b.kc = malloc(sizeof(float) * (size_t)m->layers * m->max_len * kvd);
  b.vc = malloc(sizeof(float) * (size_t)m->layers * m->max_len * kvd);
  b.scores = malloc(sizeof(float) * (size_t)m->heads * m->max_len);
  b.codes = malloc((size_t)kmax);
  if (!b.x || !b.xn || !b.q || !b.k || !b.v || !b.att || !b.gate || !b.up || !b.tmp || !b.logits || !b.kc ||
      !b.vc || !b.scores || !b.codes) {
    free_bufs(&b);
    return -1;
  }
  int tok = 0;
  for (int i = 0; i < n_prompt; ++i) tok = token_forward(m, &b, prompt[i], i);
  if (logits_out) memcpy(logits_out, b.logits, sizeof(float) * (size_t)m->vocab);
  for (int i = 0; i < n_new; ++i) {
    out[i] = tok;
    if (i + 1 < n_new) tok = token_forward(m, &b, tok, n_prompt + i);
  }
  free_bufs(&b);
  return 0;
}
