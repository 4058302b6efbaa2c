/*
 * fletcher_oracle.c -- CPU restatement of Fletcher's encoder forward pass.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); the
 * product library never links or calls this file.  Each function cites the
 * reference Go source it restates.  Build with -ffp-contract=off so float32
 * expressions are evaluated one rounded operation at a time, as Go does on
 * amd64.
 */
#include "fletcher_oracle.h"

#include <dlfcn.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* OpenBLAS (gonum blas32 -> netlib -> cblas_sgemm, blas_cgo.go:14-18)      */
/* ------------------------------------------------------------------------ */
typedef void (*sgemm_fn)(int order, int ta, int tb, int m, int n, int k,
                         float alpha, const float *a, int lda, const float *b,
                         int ldb, float beta, float *c, int ldc);
typedef void (*set_threads_fn)(int);

static sgemm_fn g_sgemm = NULL;
static set_threads_fn g_set_threads = NULL;
static set_threads_fn g_set_threads_local = NULL;
static int g_threads = 1;

enum { CBLAS_ROW_MAJOR = 101, CBLAS_NO_TRANS = 111, CBLAS_TRANS = 112 };

int orc_blas_init(const char *path) {
  if (g_sgemm) return 0;
  void *h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!h) return 1;
  g_sgemm = (sgemm_fn)dlsym(h, "scipy_cblas_sgemm");
  if (!g_sgemm) g_sgemm = (sgemm_fn)dlsym(h, "cblas_sgemm");
  g_set_threads = (set_threads_fn)dlsym(h, "scipy_openblas_set_num_threads");
  if (!g_set_threads) g_set_threads = (set_threads_fn)dlsym(h, "openblas_set_num_threads");
  g_set_threads_local = (set_threads_fn)dlsym(h, "openblas_set_num_threads_local");
  return g_sgemm ? 0 : 2;
}

void orc_set_threads(int n) {
  if (n < 1) n = 1;
  g_threads = n;
  if (g_set_threads) g_set_threads(n);
}

int orc_get_threads(void) { return g_threads; }

void orc_sgemm(int trans_a, int trans_b, int m, int n, int k, float alpha,
               const float *a, int lda, const float *b, int ldb, float beta,
               float *c, int ldc) {
  g_sgemm(CBLAS_ROW_MAJOR, trans_a ? CBLAS_TRANS : CBLAS_NO_TRANS,
          trans_b ? CBLAS_TRANS : CBLAS_NO_TRANS, m, n, k, alpha, a, lda, b,
          ldb, beta, c, ldc);
}

/* ------------------------------------------------------------------------ */
/* internal/simd/simd.go                                                     */
/* ------------------------------------------------------------------------ */

/* simd.go:7-46.  2^(x*log2e) split into k = floor(t) (truncate, then k--
 * for negative t, which also fires for exact negative integers) and a cubic
 * in the fraction f; 2^k is float32(math.Pow(2, k)). */
float orc_exp_fast(float x) {
  if (x > 88.0f) return 1e38f;
  if (x < -88.0f) return 0.0f;
  const float log2e = 1.442695f;
  float t = x * log2e;
  int k = (int)t;
  if (t < 0.0f) k--;
  float f = t - (float)k;
  float p = 1.0f + f * (0.6931472f + f * (0.2402265f + f * 0.0555041f));
  /* float32(math.Pow(2, k)) is exactly 2^k for the k reachable here; ldexp
   * produces the same value without a pow() call. */
  return p * (float)ldexp(1.0, k);
}

/* simd.go:49-64: clamp at |x| > 4, else x*(27+x^2)/(27+9x^2). */
float orc_tanh_fast(float x) {
  if (x > 4.0f) return 1.0f;
  if (x < -4.0f) return -1.0f;
  float x2 = x * x;
  return x * (27.0f + x2) / (27.0f + 9.0f * x2);
}

/* simd.go:66-76 */
void orc_gelu_fast(float *data, int64_t n) {
  const float sqrt2_over_pi = 0.7978846f;
  const float coeff = 0.044715f;
  for (int64_t i = 0; i < n; i++) {
    float x = data[i];
    data[i] = 0.5f * x * (1.0f + orc_tanh_fast(sqrt2_over_pi * (x + coeff * x * x * x)));
  }
}

/* simd.go:78-100: max from row[0], ExpFast(v-max), sequential f32 sum,
 * multiply by 1/sum. */
void orc_softmax_fast(float *row, int64_t n) {
  float mx = row[0];
  for (int64_t i = 0; i < n; i++)
    if (row[i] > mx) mx = row[i];
  float sum = 0.0f;
  for (int64_t i = 0; i < n; i++) {
    row[i] = orc_exp_fast(row[i] - mx);
    sum += row[i];
  }
  float inv = 1.0f / sum;
  for (int64_t i = 0; i < n; i++) row[i] *= inv;
}

/* Exact-math counterparts (ORC_MATH_EXACT): used to bound the fast-math
 * error and to compare against an fp64 evaluation of the same network. */
static void softmax_exact(float *row, int64_t n) {
  float mx = row[0];
  for (int64_t i = 0; i < n; i++)
    if (row[i] > mx) mx = row[i];
  double sum = 0.0;
  for (int64_t i = 0; i < n; i++) {
    row[i] = (float)exp((double)row[i] - (double)mx);
    sum += row[i];
  }
  float inv = (float)(1.0 / sum);
  for (int64_t i = 0; i < n; i++) row[i] *= inv;
}

static void gelu_exact(float *data, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    double x = data[i];
    data[i] = (float)(0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))));
  }
}

/* simd.go:132-146 (4-way unrolled sequential accumulation into one sum). */
float orc_dot(const float *a, const float *b, int64_t n) {
  float sum = 0.0f;
  int64_t i = 0;
  for (; i + 4 <= n; i += 4) {
    sum += a[i] * b[i];
    sum += a[i + 1] * b[i + 1];
    sum += a[i + 2] * b[i + 2];
    sum += a[i + 3] * b[i + 3];
  }
  for (; i < n; i++) sum += a[i] * b[i];
  return sum;
}

/* ------------------------------------------------------------------------ */
/* internal/device/utils.go                                                  */
/* ------------------------------------------------------------------------ */

/* utils.go:13-72: NaN/Inf passthrough, clamp to +-65504, flush |f| < 2^-14
 * to signed zero, truncate the mantissa (bits >> 13), saturate exponent
 * overflow to 0x7BFF. */
uint16_t orc_f32_to_f16(float f) {
  if (isnan(f)) return 0x7E00;
  if (isinf(f)) return f > 0 ? 0x7C00 : 0xFC00;
  const float max_f16 = 65504.0f;
  const float min_normal = 6.10351562e-5f;
  if (f > max_f16) f = max_f16;
  else if (f < -max_f16) f = -max_f16;
  float a = f < 0 ? -f : f;
  if (a < min_normal && a > 0) return f < 0 ? 0x8000 : 0x0000;
  uint32_t bits;
  memcpy(&bits, &f, 4);
  uint32_t sign = (bits >> 16) & 0x8000u;
  int exp = (int)((bits >> 23) & 0xFF) - 127 + 15;
  uint32_t frac = (bits >> 13) & 0x3FFu;
  if (exp >= 0x1F) return (uint16_t)(sign | 0x7BFFu);
  if (exp <= 0) return (uint16_t)sign;
  return (uint16_t)(sign | ((uint32_t)exp << 10) | frac);
}

/* utils.go:75-91: subnormals read back as +0. */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h >> 15) & 1u;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t frac = (uint32_t)h & 0x3FFu;
  uint32_t bits;
  float out;
  if (exp == 0) return 0.0f;
  if (exp == 31) bits = (sign << 31) | (0xFFu << 23) | (frac << 13);
  else bits = (sign << 31) | ((exp - 15 + 127) << 23) | (frac << 13);
  memcpy(&out, &bits, 4);
  return out;
}

/* ------------------------------------------------------------------------ */
/* internal/device/cpu_backend.go                                            */
/* ------------------------------------------------------------------------ */

/* simd.go:102-115 VecAdd, used by Add (:415-440) and AddBias (:448-488). */
static void vec_add(float *dst, const float *src, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] += src[i];
}

void orc_add(float *t, const float *other, int64_t n) { vec_add(t, other, n); }

void orc_scale(float *t, int64_t n, float v) {
  for (int64_t i = 0; i < n; i++) t[i] *= v;
}

void orc_add_scalar(float *t, int64_t n, float v) {
  for (int64_t i = 0; i < n; i++) t[i] += v;
}

void orc_add_bias(float *t, int rows, int cols, const float *bias) {
  for (int i = 0; i < rows; i++) vec_add(t + (int64_t)i * cols, bias, cols);
}

void orc_tanh_inplace(float *t, int64_t n) {
  for (int64_t i = 0; i < n; i++) t[i] = orc_tanh_fast(t[i]);
}

void orc_softmax_rows(float *t, int rows, int cols) {
  for (int i = 0; i < rows; i++) orc_softmax_fast(t + (int64_t)i * cols, cols);
}

/* cpu_backend.go:541-601: sequential f32 sum -> mean; sequential sum of
 * squared deviations -> variance; invStd = 1/float32(sqrt(float64(var+eps)));
 * y = (x-mean)*invStd*gamma + beta. */
void orc_layernorm(float *t, int rows, int cols, const float *gamma,
                   const float *beta, float eps) {
  for (int i = 0; i < rows; i++) {
    float *row = t + (int64_t)i * cols;
    float sum = 0.0f;
    for (int j = 0; j < cols; j++) sum += row[j];
    float mean = sum / (float)cols;
    float var_sum = 0.0f;
    for (int j = 0; j < cols; j++) {
      float d = row[j] - mean;
      var_sum += d * d;
    }
    float variance = var_sum / (float)cols;
    float inv_std = 1.0f / (float)sqrt((double)(variance + eps));
    for (int j = 0; j < cols; j++)
      row[j] = (row[j] - mean) * inv_std * gamma[j] + beta[j];
  }
}

/* cpu_backend.go:603-610: t += residual, then LayerNorm(t). */
void orc_add_layernorm(float *t, const float *residual, int rows, int cols,
                       const float *gamma, const float *beta, float eps) {
  vec_add(t, residual, (int64_t)rows * cols);
  orc_layernorm(t, rows, cols, gamma, beta, eps);
}

/* cpu_backend.go:316-372 (mulBLAS): lda/ldb are the physical column counts. */
void orc_mul(float *c, const float *a, int a_rows, int a_cols, int trans_a,
             const float *b, int b_rows, int b_cols, int trans_b) {
  int m = trans_a ? a_cols : a_rows;
  int k = trans_a ? a_rows : a_cols;
  int n = trans_b ? b_rows : b_cols;
  orc_sgemm(trans_a, trans_b, m, n, k, 1.0f, a, a_cols, b, b_cols, 0.0f, c, n);
}

/* cpu_backend.go:612-624 */
void orc_linear(const float *x, int r, int k, const float *w, int n,
                const float *bias, float *out) {
  orc_sgemm(0, 0, r, n, k, 1.0f, x, k, w, n, 0.0f, out, n);
  if (bias) orc_add_bias(out, r, n, bias);
}

static void linear_activation(const float *x, int r, int k, const float *w,
                              int n, const float *bias, int act, int math_mode,
                              float *out) {
  if (act != ORC_ACT_SWIGLU) {
    orc_linear(x, r, k, w, n, bias, out);
    int64_t total = (int64_t)r * n;
    if (act == ORC_ACT_GELU) {
      if (math_mode == ORC_MATH_EXACT) gelu_exact(out, total);
      else orc_gelu_fast(out, total);
    } else if (act == ORC_ACT_TANH) {
      if (math_mode == ORC_MATH_EXACT)
        for (int64_t i = 0; i < total; i++) out[i] = (float)tanh((double)out[i]);
      else orc_tanh_inplace(out, total);
    } else if (act == ORC_ACT_SOFTMAX) {
      if (math_mode == ORC_MATH_EXACT)
        for (int i = 0; i < r; i++) softmax_exact(out + (int64_t)i * n, n);
      else orc_softmax_rows(out, r, n);
    }
    return;
  }
  /* SwiGLU (:636-654): gate = first half, x/(1+float32(exp(float64(-x)))) * up. */
  float *tmp = (float *)malloc(sizeof(float) * (size_t)r * n);
  orc_linear(x, r, k, w, n, bias, tmp);
  int inter = n / 2;
  for (int row = 0; row < r; row++) {
    const float *src = tmp + (int64_t)row * n;
    float *dst = out + (int64_t)row * inter;
    for (int i = 0; i < inter; i++) {
      float g = src[i];
      float u = src[i + inter];
      float swish = g / (1.0f + (float)exp((double)(-g)));
      dst[i] = swish * u;
    }
  }
  free(tmp);
}

void orc_linear_activation(const float *x, int r, int k, const float *w, int n,
                           const float *bias, int act, float *out) {
  linear_activation(x, r, k, w, n, bias, act, ORC_MATH_REFERENCE, out);
}

/* cpu_backend.go:496-510 */
void orc_gather(const float *table, int rows, int cols, const int64_t *idx,
                int n, float *out) {
  (void)rows;
  for (int i = 0; i < n; i++)
    memcpy(out + (int64_t)i * cols, table + idx[i] * cols, sizeof(float) * cols);
}

/* ---- attention ---------------------------------------------------------- */
typedef struct {
  const float *q, *k, *v;
  float *out;
  int start, end, seq, heads, hidden, math_mode, spawned;
  float scale;
} attn_job;

/* Rows [r0, r1) of an s x s score matrix through the row softmax. */
typedef struct {
  float *scores;
  int s, r0, r1, math_mode;
} softmax_job;

static void *softmax_rows_worker(void *arg) {
  softmax_job *j = (softmax_job *)arg;
  for (int r = j->r0; r < j->r1; r++) {
    if (j->math_mode == ORC_MATH_EXACT) softmax_exact(j->scores + (int64_t)r * j->s, j->s);
    else orc_softmax_fast(j->scores + (int64_t)r * j->s, j->s);
  }
  return NULL;
}

/* Every row of the score matrix; rows are independent, so splitting them
 * over threads (when the caller is the only attention worker) leaves each
 * row's result unchanged. */
static void softmax_rows(float *scores, int s, int math_mode, int threads) {
  if (threads > 64) threads = 64;
  if (threads <= 1 || s < 256) {
    softmax_job one = {scores, s, 0, s, math_mode};
    softmax_rows_worker(&one);
    return;
  }
  pthread_t th[64];
  softmax_job jobs[64];
  int per = (s + threads - 1) / threads, n = 0;
  for (int t = 0; t < threads; t++) {
    int r0 = t * per, r1 = r0 + per < s ? r0 + per : s;
    if (r0 >= r1) break;
    softmax_job jb = {scores, s, r0, r1, math_mode};
    jobs[n] = jb;
    pthread_create(&th[n], NULL, softmax_rows_worker, &jobs[n]);
    n++;
  }
  for (int t = 0; t < n; t++) pthread_join(th[t], NULL);
}

/* Body of one worker of cpu_backend.go:695-753: for each batch item and
 * head, scores = scale * Q_h K_h^T (sgemm, alpha = scale), SoftmaxFast per
 * row, out_h = scores V_h (sgemm into the head's column slice). */
static void *attn_worker(void *arg) {
  attn_job *j = (attn_job *)arg;
  int s = j->seq, c = j->hidden, hd = c / j->heads;
  if (j->spawned && g_set_threads_local) g_set_threads_local(1);
  float *scores = (float *)malloc(sizeof(float) * (size_t)s * s);
  for (int i = j->start; i < j->end; i++) {
    int64_t q_start = (int64_t)i * s * c;
    for (int h = 0; h < j->heads; h++) {
      int64_t off = q_start + (int64_t)h * hd;
      orc_sgemm(0, 1, s, s, hd, j->scale, j->q + off, c, j->k + off, c, 0.0f,
                scores, s);
      softmax_rows(scores, s, j->math_mode, j->spawned ? 1 : g_threads);
      orc_sgemm(0, 0, s, hd, s, 1.0f, scores, s, j->v + off, c, 0.0f,
                j->out + off, c);
    }
  }
  free(scores);
  return NULL;
}

static void attention_impl(const float *q, const float *k, const float *v,
                           int batch, int seq, int heads, int hidden,
                           float scale, int math_mode, float *out) {
  int workers = g_threads < batch ? g_threads : batch;
  if (workers < 1) workers = 1;
  int per = (batch + workers - 1) / workers;
  attn_job *jobs = (attn_job *)calloc((size_t)workers, sizeof(attn_job));
  pthread_t *th = (pthread_t *)calloc((size_t)workers, sizeof(pthread_t));
  int launched = 0;
  for (int w = 0; w < workers; w++) {
    int st = w * per, en = st + per;
    if (en > batch) en = batch;
    if (st >= en) break;
    attn_job jb = {q, k, v, out, st, en, seq, heads, hidden, math_mode, 0, scale};
    jobs[w] = jb;
    launched++;
  }
  if (launched == 1) {
    attn_worker(&jobs[0]);
  } else {
    for (int w = 0; w < launched; w++) {
      jobs[w].spawned = 1;
      pthread_create(&th[w], NULL, attn_worker, &jobs[w]);
    }
    for (int w = 0; w < launched; w++) pthread_join(th[w], NULL);
  }
  free(jobs);
  free(th);
}

void orc_attention(const float *q, const float *k, const float *v, int batch,
                   int seq, int heads, int hidden, float scale, float *out) {
  attention_impl(q, k, v, batch, seq, heads, hidden, scale, ORC_MATH_REFERENCE, out);
}

/* cpu_backend.go:66-132: per sequence and head, scores = Q K^T, then
 * Scale(scale), SoftmaxFast, times V. */
void orc_attention_varlen(const float *q, const float *k, const float *v,
                          const int64_t *lengths, int nseq, int heads,
                          int hidden, float scale, float *out) {
  int hd = hidden / heads;
  int64_t start = 0;
  for (int b = 0; b < nseq; b++) {
    int len = (int)lengths[b];
    float *scores = (float *)malloc(sizeof(float) * (size_t)len * len + 4);
    for (int h = 0; h < heads && len > 0; h++) {
      int64_t off = start * hidden + (int64_t)h * hd;
      orc_sgemm(0, 1, len, len, hd, 1.0f, q + off, hidden, k + off, hidden, 0.0f,
                scores, len);
      orc_scale(scores, (int64_t)len * len, scale);
      orc_softmax_rows(scores, len, len);
      orc_sgemm(0, 0, len, hd, len, 1.0f, scores, len, v + off, hidden, 0.0f,
                out + off, hidden);
    }
    free(scores);
    start += len;
  }
}

/* cpu_backend.go:760-805 with the base as a parameter (reference: 10000):
 * theta = float64(pos) * base^(-2i/d) in float64, cos/sin cast to float32,
 * rotate-half pairs (i, i + d/2). */
void orc_rope(float *t, int batch, int seq, int heads, int head_dim,
              double base) {
  int64_t rows = (int64_t)batch * seq;
  int half = head_dim / 2;
  for (int64_t r = 0; r < rows; r++) {
    int pos = (int)(r % seq);
    float *row = t + r * (int64_t)heads * head_dim;
    for (int h = 0; h < heads; h++) {
      float *x = row + (int64_t)h * head_dim;
      for (int i = 0; i < half; i++) {
        double theta = (double)pos * pow(base, -2.0 * (double)i / (double)head_dim);
        float c = (float)cos(theta), s = (float)sin(theta);
        float x1 = x[i], x2 = x[i + half];
        x[i] = x1 * c - x2 * s;
        x[i + half] = x1 * s + x2 * c;
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* internal/embeddings/model/bert.go                                         */
/* ------------------------------------------------------------------------ */

/* One encoder layer, bert.go:364-384 -> 610-728 (uniform path), 748-824. */
static void encoder_layer(const orc_config *cfg, const orc_weights *w, int l,
                          float *x, int64_t T, const int64_t *lengths, int nseq,
                          int uniform) {
  int H = cfg->hidden, heads = cfg->heads, hd = H / heads;
  int I = cfg->intermediate;
  int n_inter = cfg->activation == ORC_ACT_SWIGLU ? 2 * I : I;
  size_t th = (size_t)T * H;
  float *q = (float *)malloc(sizeof(float) * th);
  float *k = (float *)malloc(sizeof(float) * th);
  float *v = (float *)malloc(sizeof(float) * th);
  float *ctx = (float *)calloc(th, sizeof(float));
  float *proj = (float *)malloc(sizeof(float) * th);

  orc_linear(x, (int)T, H, w->q_w[l], H, w->q_b ? w->q_b[l] : NULL, q);
  orc_linear(x, (int)T, H, w->k_w[l], H, w->k_b ? w->k_b[l] : NULL, k);
  orc_linear(x, (int)T, H, w->v_w[l], H, w->v_b ? w->v_b[l] : NULL, v);
  float scale = 1.0f / (float)sqrt((double)hd); /* bert.go:643 */

  if (uniform) {
    int S = (int)lengths[0];
    if (cfg->position == ORC_POS_ROPE) {
      orc_rope(q, nseq, S, heads, hd, cfg->rope_base);
      orc_rope(k, nseq, S, heads, hd, cfg->rope_base);
    }
    attention_impl(q, k, v, nseq, S, heads, H, scale, cfg->math, ctx);
  } else {
    int64_t start = 0;
    for (int b = 0; b < nseq; b++) {
      int L = (int)lengths[b];
      int64_t off = start * H;
      if (cfg->position == ORC_POS_ROPE) {
        orc_rope(q + off, 1, L, heads, hd, cfg->rope_base);
        orc_rope(k + off, 1, L, heads, hd, cfg->rope_base);
      }
      attention_impl(q + off, k + off, v + off, 1, L, heads, H, scale, cfg->math,
                     ctx + off);
      start += L;
    }
  }

  /* BertSelfOutput: Linear, then residual.AddLayerNorm(projected). */
  orc_linear(ctx, (int)T, H, w->o_w[l], H, w->o_b ? w->o_b[l] : NULL, proj);
  orc_add_layernorm(x, proj, (int)T, H, w->attn_ln_g[l], w->attn_ln_b[l], cfg->ln_eps);

  /* BertIntermediate + BertOutput. */
  float *inter = (float *)malloc(sizeof(float) * (size_t)T * I);
  linear_activation(x, (int)T, H, w->inter_w[l], n_inter,
                    w->inter_b ? w->inter_b[l] : NULL, cfg->activation, cfg->math,
                    inter);
  orc_linear(inter, (int)T, I, w->out_w[l], H, w->out_b ? w->out_b[l] : NULL, proj);
  orc_add_layernorm(x, proj, (int)T, H, w->out_ln_g[l], w->out_ln_b[l], cfg->ln_eps);

  free(inter);
  free(q);
  free(k);
  free(v);
  free(ctx);
  free(proj);
}

int orc_forward_batch(const orc_config *cfg, const orc_weights *w,
                      const int64_t *ids, const int64_t *lengths, int nseq,
                      float *out, float *hidden_out) {
  if (!g_sgemm || nseq <= 0) return 1;
  int H = cfg->hidden;
  int64_t T = 0;
  int uniform = 1;
  for (int b = 0; b < nseq; b++) {
    if (lengths[b] <= 0) return 2;
    T += lengths[b];
    if (lengths[b] != lengths[0]) uniform = 0;
  }
  for (int64_t t = 0; t < T; t++)
    if (ids[t] < 0 || ids[t] >= cfg->vocab_size) return 3;

  /* BertEmbeddings.ForwardBatch (bert.go:215-261). */
  float *x = (float *)malloc(sizeof(float) * (size_t)T * H);
  float *tmp = (float *)malloc(sizeof(float) * (size_t)T * H);
  orc_gather(w->word_emb, cfg->vocab_size, H, ids, (int)T, x);
  int64_t *idx = (int64_t *)malloc(sizeof(int64_t) * (size_t)T);
  if (cfg->position == ORC_POS_ABSOLUTE) {
    int64_t p = 0;
    for (int b = 0; b < nseq; b++)
      for (int64_t i = 0; i < lengths[b]; i++)
        idx[p++] = i >= cfg->max_pos ? cfg->max_pos - 1 : i;
    orc_gather(w->pos_emb, cfg->max_pos, H, idx, (int)T, tmp);
    orc_add(x, tmp, T * H);
  }
  memset(idx, 0, sizeof(int64_t) * (size_t)T);
  orc_gather(w->type_emb, 2, H, idx, (int)T, tmp);
  orc_add(x, tmp, T * H);
  orc_layernorm(x, (int)T, H, w->emb_ln_g, w->emb_ln_b, cfg->ln_eps);
  free(idx);
  free(tmp);

  /* BertEncoder.ForwardBatch (bert.go:329-341). */
  for (int l = 0; l < cfg->layers; l++) encoder_layer(cfg, w, l, x, T, lengths, nseq, uniform);
  if (hidden_out) memcpy(hidden_out, x, sizeof(float) * (size_t)T * H);

  if (cfg->pool == ORC_POOL_CLS_TANH) {
    /* BertPooler.ForwardBatch (bert.go:441-488): CLS row of each sequence,
     * LinearActivation(Tanh). */
    float *cls = (float *)malloc(sizeof(float) * (size_t)nseq * H);
    int64_t off = 0;
    for (int b = 0; b < nseq; b++) {
      memcpy(cls + (int64_t)b * H, x + off * H, sizeof(float) * H);
      off += lengths[b];
    }
    linear_activation(cls, nseq, H, w->pool_w, H, w->pool_b, ORC_ACT_TANH,
                      cfg->math, out);
    free(cls);
  } else {
    /* Masked mean-pool (+ L2): not in the reference; defined in closed form
     * p_b = (1/L_b) sum_t h_t, out = p / max(||p||_2, 1e-12), f64 sums. */
    int64_t off = 0;
    double *acc = (double *)malloc(sizeof(double) * H);
    for (int b = 0; b < nseq; b++) {
      for (int j = 0; j < H; j++) acc[j] = 0.0;
      for (int64_t t = 0; t < lengths[b]; t++) {
        const float *row = x + (off + t) * H;
        for (int j = 0; j < H; j++) acc[j] += row[j];
      }
      double nrm = 0.0;
      for (int j = 0; j < H; j++) {
        acc[j] /= (double)lengths[b];
        nrm += acc[j] * acc[j];
      }
      nrm = sqrt(nrm);
      if (nrm < 1e-12) nrm = 1e-12;
      for (int j = 0; j < H; j++)
        out[(int64_t)b * H + j] =
            (float)(cfg->pool == ORC_POOL_MEAN_L2 ? acc[j] / nrm : acc[j]);
      off += lengths[b];
    }
    free(acc);
  }
  free(x);
  return 0;
}
