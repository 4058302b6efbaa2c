/*
 * fletcher_oracle.h -- CPU restatement of Fletcher's encoder forward pass.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * backend and the timed CPU baseline in bench.py.  Only tests/, the smoke
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it;
 * the product library never links, loads or calls it.
 *
 * Every function restates the reference Go code cited next to it
 * (paths relative to the longbow-fletcher repository root).  GEMMs go to
 * OpenBLAS sgemm with the same row-major / transpose / alpha / beta
 * arguments as gonum blas32 -> netlib -> cblas_sgemm
 * (internal/device/cpu_backend.go:365-371, 725-731, 744-750).
 *
 * Arithmetic is float32 evaluated operation by operation (the build uses
 * -ffp-contract=off), matching Go's unfused float32 semantics on amd64.
 */
#ifndef FLETCHER_ORACLE_H
#define FLETCHER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- OpenBLAS binding ------------------------------------------------ */
/* dlopen()s an OpenBLAS exposing scipy_cblas_sgemm or cblas_sgemm.
 * Returns 0 on success. */
int orc_blas_init(const char *path);
void orc_set_threads(int n); /* OpenBLAS threads + worker threads */
int orc_get_threads(void);
/* Row-major sgemm: C = alpha*op(A)*op(B) + beta*C. */
void orc_sgemm(int trans_a, int trans_b, int m, int n, int k, float alpha,
               const float *a, int lda, const float *b, int ldb, float beta,
               float *c, int ldc);

/* ---- internal/simd/simd.go ------------------------------------------- */
float orc_exp_fast(float x);                    /* simd.go:7-46   */
float orc_tanh_fast(float x);                   /* simd.go:49-64  */
void orc_gelu_fast(float *data, int64_t n);     /* simd.go:66-76  */
void orc_softmax_fast(float *row, int64_t n);   /* simd.go:78-100 */
float orc_dot(const float *a, const float *b, int64_t n); /* simd.go:132-146 */

/* ---- internal/device/utils.go ---------------------------------------- */
uint16_t orc_f32_to_f16(float f);   /* utils.go:13-72 (truncating) */
float orc_f16_to_f32(uint16_t h);   /* utils.go:75-91 */

/* ---- internal/device/cpu_backend.go (Tensor ops) --------------------- */
void orc_add(float *t, const float *other, int64_t n);          /* :415-440 */
void orc_scale(float *t, int64_t n, float v);                   /* :490-494 */
void orc_add_scalar(float *t, int64_t n, float v);              /* :442-446 */
void orc_add_bias(float *t, int rows, int cols, const float *bias); /* :448-488 */
void orc_tanh_inplace(float *t, int64_t n);                     /* :531-539 */
void orc_softmax_rows(float *t, int rows, int cols);            /* :512-522 */
void orc_layernorm(float *t, int rows, int cols, const float *gamma,
                   const float *beta, float eps);               /* :541-601 */
void orc_add_layernorm(float *t, const float *residual, int rows, int cols,
                       const float *gamma, const float *beta, float eps); /* :603-610 */
/* Mul: c[ar x bc] = op(a) * op(b); a stored [a_rows x a_cols] (physical). */
void orc_mul(float *c, const float *a, int a_rows, int a_cols, int trans_a,
             const float *b, int b_rows, int b_cols, int trans_b); /* :316-372 */
/* Linear: out[r x n] = x[r x k] * w[k x n] + bias (bias may be NULL). */
void orc_linear(const float *x, int r, int k, const float *w, int n,
                const float *bias, float *out);                 /* :612-624 */
/* LinearActivation; act follows device.go:126-134.  For SwiGLU, n is the
 * fused width 2I and out has n/2 columns. */
void orc_linear_activation(const float *x, int r, int k, const float *w, int n,
                           const float *bias, int act, float *out); /* :626-660 */
void orc_gather(const float *table, int rows, int cols, const int64_t *idx,
                int n, float *out);                              /* :496-510 */
/* Attention over uniform [batch*seq, hidden] inputs (no mask). */
void orc_attention(const float *q, const float *k, const float *v, int batch,
                   int seq, int heads, int hidden, float scale, float *out); /* :662-758 */
/* Per-sequence multi-head attention over packed rows. */
void orc_attention_varlen(const float *q, const float *k, const float *v,
                          const int64_t *lengths, int nseq, int heads,
                          int hidden, float scale, float *out);  /* :66-132 */
/* RoPE in place, pos = row % seq; the reference hard-codes base 10000. */
void orc_rope(float *t, int batch, int seq, int heads, int head_dim,
              double base);                                      /* :760-805 */

/* ---- internal/embeddings/model/bert.go -------------------------------- */
enum { ORC_ACT_IDENTITY = 0, ORC_ACT_GELU = 1, ORC_ACT_TANH = 2,
       ORC_ACT_SOFTMAX = 3, ORC_ACT_SWIGLU = 4 };
enum { ORC_POS_ABSOLUTE = 0, ORC_POS_ROPE = 1 };
enum { ORC_POOL_CLS_TANH = 0, ORC_POOL_MEAN = 1, ORC_POOL_MEAN_L2 = 2 };
enum { ORC_MATH_REFERENCE = 0, ORC_MATH_EXACT = 1 };

typedef struct {
  int32_t vocab_size, hidden, layers, heads, intermediate, max_pos;
  int32_t activation;  /* ORC_ACT_GELU or ORC_ACT_SWIGLU */
  int32_t position;    /* ORC_POS_* */
  float rope_base;     /* reference: 10000 (cpu_backend.go:790) */
  float ln_eps;        /* reference: 1e-7 (bert.go:281) */
  int32_t pool;        /* ORC_POOL_* */
  int32_t math;        /* ORC_MATH_REFERENCE = simd.go fast math */
} orc_config;

/* Weight pointers, reference layout: matrices are [in, out] row-major. */
typedef struct {
  const float *word_emb, *pos_emb, *type_emb, *emb_ln_g, *emb_ln_b;
  const float **q_w, **q_b, **k_w, **k_b, **v_w, **v_b, **o_w, **o_b;
  const float **attn_ln_g, **attn_ln_b;
  const float **inter_w, **inter_b, **out_w, **out_b;
  const float **out_ln_g, **out_ln_b;
  const float *pool_w, *pool_b;
} orc_weights;

/* BertModel.ForwardBatch (bert.go:149-169) followed by the pooling mode.
 * ids are flat (sum of lengths), out is [nseq x hidden].  When lengths
 * differ the batch is evaluated per sequence (positions restart at 0 for
 * every sequence), which is the reference's uniform path applied to each
 * sequence.  hidden_out (optional, [sum(lengths) x hidden]) receives the
 * last hidden states.  Returns 0 on success. */
int orc_forward_batch(const orc_config *cfg, const orc_weights *w,
                      const int64_t *ids, const int64_t *lengths, int nseq,
                      float *out, float *hidden_out);

#ifdef __cplusplus
}
#endif
#endif
