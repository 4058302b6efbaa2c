/*
 * fletcher_hip.h -- C ABI of the MI355X (gfx950) encoder-forward backend for
 * Fletcher (23skdu/longbow-fletcher).
 *
 * This library fills the slot of the reference's native GPU bridge
 * (internal/device/cuda_bridge.h:11-53 called from cuda_linux.go) behind the
 * Go `device.Backend` / `device.Tensor` interfaces
 * (internal/device/device.go:5-162).  A Go cgo file binds it the way
 * cuda_linux.go binds cuda_bridge.h.
 *
 * Conventions
 *  - Every entry point returns an int status: FL_OK (0) or an FL_ERR_* code;
 *    fl_last_error() returns the calling thread's message for the last failure.
 *    (The reference bridge returns void / NULL and panics in Go; the Go wrapper
 *    panics on non-zero so the existing recover paths in embeddings.go keep
 *    working.)
 *  - Buffers are plain device pointers obtained from fl_alloc; views are
 *    pointer arithmetic on them.  Tensors are 2-D row-major; `ld` arguments are
 *    row strides in elements.  Tensor.Slice of whole rows (all columns) is
 *    such a view, not a copy, as in the reference's Metal backend
 *    (metal_darwin.go:487-521): src + r0 * cols * element size, owned by the
 *    tensor it points into (never passed to fl_free); writes through it land
 *    in that tensor.  Every entry point accepts views.  Other slices are
 *    copies (fl_slice).
 *  - Every per-op entry point checks each operand's byte extent against the
 *    fl_alloc buffer the pointer lies in (views included) and returns
 *    FL_ERR_INVALID, before anything is enqueued, for an operand that would
 *    run past the end of its buffer (e.g. an fp16 buffer passed as fp32).
 *    Pointers from other allocators are not sized and not checked.
 *  - Operands of different storage types follow the reference's Metal
 *    backend: Linear's result and arithmetic take the weight's type, its input
 *    is converted (metal_darwin.go:806-829); Add / AddLayerNorm convert the
 *    other operand to the receiver's type (:603-619, 798-804).  Conversions
 *    happen in the kernels (loads, or the producing kernel's store), not in
 *    extra passes over the data, except the first time an fp32 tensor is
 *    read by a 16-bit Linear (one conversion, kept for the Q, K and V
 *    projections of the same hidden state and refreshed by the LayerNorm
 *    that next rewrites it).
 *  - All work of a context is enqueued in order on the context's HIP stream;
 *    entry points that hand data back to the host synchronise that stream,
 *    and the others return without waiting for the device.
 *    Entry points lock the context, so several host threads may share it
 *    (concurrent HTTP requests may share one backend, server.go:225-261).
 *  - fl_linear / fl_gemm keep the packed form of a weight that lies in an
 *    fl_alloc buffer between calls; every entry point that writes a buffer
 *    marks it, so the next call packs it again.  A buffer written by other
 *    means (kernels of the caller on the context stream) must be marked with
 *    fl_buffer_written.
 *  - Host arrays (ids, lengths, indices) are int64 like Go's `int` on amd64.
 */
#ifndef FLETCHER_HIP_H
#define FLETCHER_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fl_context fl_context;
typedef struct fl_model fl_model;

/* status codes */
#define FL_OK 0
#define FL_ERR_INVALID 1     /* bad argument / shape */
#define FL_ERR_HIP 2         /* HIP runtime error */
#define FL_ERR_OOM 3         /* device allocation failed */
#define FL_ERR_UNSUPPORTED 4 /* valid request this backend does not implement */
#define FL_ERR_IO 5          /* weight file missing, unreadable or malformed */

/* device.DataType (device.go:119-124): Float32 = 0, Float16 = 1; BF16 added. */
#define FL_F32 0
#define FL_F16 1
#define FL_BF16 2

/* device.ActivationType (device.go:126-134). */
#define FL_ACT_IDENTITY 0
#define FL_ACT_GELU 1
#define FL_ACT_TANH 2
#define FL_ACT_SOFTMAX 3
#define FL_ACT_SWIGLU 4

/* Math mode.  REFERENCE evaluates the CPU path's fast-math formulas
 * (simd.go:7-100: ExpFast softmax with an exact row max, TanhFast GELU/tanh)
 * so fp32 results match it to ~1e-6; EXACT uses hardware exp2 with an online
 * softmax and an accurate tanh. */
#define FL_MATH_REFERENCE 0
#define FL_MATH_EXACT 1

/* Host fp32 -> device fp16 rounding for fl_upload_f32.  TRUNCATE reproduces
 * Float32ToFloat16 (utils.go:13-72: mantissa truncation, flush below 2^-14,
 * clamp to 65504). */
#define FL_ROUND_NEAREST 0
#define FL_ROUND_TRUNCATE 1

/* Weight layouts accepted by fl_linear. */
#define FL_W_IN_OUT 0 /* [in, out] row-major, Y = X*W: the reference layout (bert.go:542-547) */
#define FL_W_OUT_IN 1 /* [out, in] row-major (pre-packed; fastest) */

/* Pooling modes of the model-level forward. */
#define FL_POOL_CLS_TANH 0 /* BertPooler: tanh(CLS*Wp + bp) (bert.go:441-488) */
#define FL_POOL_MEAN 1     /* masked mean over each sequence's tokens */
#define FL_POOL_MEAN_L2 2  /* masked mean, then p / max(||p||_2, 1e-12) */

/* Position embedding type (bert.go:12-17). */
#define FL_POS_ABSOLUTE 0
#define FL_POS_ROPE 1

const char *fl_last_error(void);
const char *fl_version(void);

/* ---- Backend / context ------------------------------------------------- */
/* Backend.DeviceCount (device.go:152-154); Cuda_GetDeviceCount (cuda_bridge.h:18). */
int fl_device_count(int *count);
/* Cuda_Init (cuda_bridge.h:17) on an explicit device. */
int fl_init(int device, fl_context **out);
/* Cuda_FreeContext (cuda_bridge.h:20).  Frees every buffer still owned. */
int fl_free_context(fl_context *ctx);
/* Backend.SetDevice (device.go:155-157); Cuda_SetDevice (cuda_bridge.h:19).
 * Later allocations and ops go to `device`; earlier buffers stay where they are. */
int fl_set_device(fl_context *ctx, int device);
/* Backend.Synchronize (device.go:148); Cuda_Synchronize (cuda_bridge.h:53). */
int fl_synchronize(fl_context *ctx);
/* Backend.GetVRAMUsage (device.go:159-161): bytes held by this context and
 * the device's total memory. */
int fl_vram_usage(fl_context *ctx, int64_t *allocated, int64_t *total);
/* The hipStream_t (as void*) every op of this context is enqueued on. */
int fl_get_stream(fl_context *ctx, void **stream);

/* ---- Buffers ----------------------------------------------------------- */
/* Cuda_Alloc (cuda_bridge.h:23).  The buffer is zero-filled, as
 * Backend.GetTensor requires (cpu_backend.go:147-156, device_test.go:98-112). */
int fl_alloc(fl_context *ctx, int64_t bytes, void **out);
/* fl_alloc without the zero fill, for the result tensors of the producing
 * ops (Linear, LinearActivation, Attention, Gather, Cast, Slice, and
 * NewTensor with data: device.go:5-117), which write them whole.  The
 * reference's Metal backend zero-fills those too (NewTensorWithType,
 * metal_darwin.go:100-125); this skips one write pass over every result.
 * Contents are undefined until written. */
int fl_alloc_uninit(fl_context *ctx, int64_t bytes, void **out);
/* Cuda_FreeBuffer (cuda_bridge.h:24); Backend.PutTensor (device.go:146).  The
 * buffer goes back to the context's cache without waiting for the device
 * (like the Metal pool, metal_darwin.go:151-274): a later fl_alloc may hand
 * it out again, and its work is ordered behind the earlier work on the
 * context stream.  Work on other streams that reads the buffer must finish
 * before the buffer is freed. */
int fl_free(fl_context *ctx, void *ptr);
/* The buffer cache's counters, like the Metal pool's metrics
 * (metal_darwin.go pool hits / misses / size / buffers): stats[0] hits,
 * [1] misses, [2] cached bytes, [3] cached buffers, [4] bytes of packed
 * weights kept by fl_linear / fl_gemm, [5] buffers in use. */
int fl_pool_stats(fl_context *ctx, int64_t *stats);
/* Returns every cached (free) buffer to the device (synchronises). */
int fl_pool_trim(fl_context *ctx);
/* Marks an fl_alloc buffer as written by code outside this library (drops
 * the packed copies fl_linear / fl_gemm keep of it). */
int fl_buffer_written(fl_context *ctx, const void *ptr);
/* Cuda_CopyToDevice (cuda_bridge.h:25-26); the host buffer may be reused on
 * return (copies up to 64 MiB go through pinned staging without waiting). */
int fl_copy_to_device(fl_context *ctx, void *dst, const void *src, int64_t bytes);
/* Cuda_CopyToHost (cuda_bridge.h:27); waits for prior work on the stream. */
int fl_copy_to_host(fl_context *ctx, void *dst, const void *src, int64_t bytes);
/* Tensor.Copy (device.go:31) between device buffers. */
int fl_copy_device(fl_context *ctx, void *dst, const void *src, int64_t bytes);
int fl_memset(fl_context *ctx, void *ptr, int value, int64_t bytes);
/* Tensor.CopyFromFloat32 (device.go:27): host fp32 -> device `dtype`. */
int fl_upload_f32(fl_context *ctx, void *dst, int dtype, const float *src, int64_t n,
                  int rounding);
/* Tensor.ToHost (device.go:24): device `dtype` -> host fp32 (synchronises). */
int fl_download_f32(fl_context *ctx, float *dst, const void *src, int dtype, int64_t n);

/* ---- Tensor ops (device.go:39-116) --------------------------------------- */
/* Tensor.Mul (device.go:39-42; cpu_backend.go:316-372):
 * C[m x n] = alpha * op(A) * op(B), op = transpose when trans_* != 0.
 * A is stored [m x k] (or [k x m] when trans_a), B [k x n] (or [n x k]). */
int fl_gemm(fl_context *ctx, int dtype, int trans_a, int trans_b, int m, int n, int k,
            float alpha, const void *a, int lda, const void *b, int ldb, void *c, int ldc);
/* Tensor.Linear / LinearActivation (device.go:75-81; cpu_backend.go:612-660):
 * out = act(x * W + bias).  x is [rows x in_cols] of x_dtype; W is
 * [in_cols x out_cols] (FL_W_IN_OUT) or [out_cols x in_cols] (FL_W_OUT_IN)
 * of w_dtype; bias is w_dtype [out_cols] or NULL; out is w_dtype (the
 * result follows the weight, metal_darwin.go:818-829: bert.go:253-258 keeps
 * an fp32 hidden state that fp16 weights read, bert.go:614-616).  For
 * FL_ACT_SWIGLU out has out_cols/2 columns: silu(first half) * second half
 * (cpu_backend.go:636-654). */
int fl_linear(fl_context *ctx, int x_dtype, const void *x, int rows, int in_cols, int w_dtype,
              const void *w, int w_layout, int out_cols, const void *bias, int act, int math,
              void *out);
/* Tensor.Add (device.go:45): t += other, n elements; other (other_dtype) is
 * converted to t's dtype (metal_darwin.go:603-619). */
int fl_add(fl_context *ctx, int dtype, void *t, int other_dtype, const void *other, int64_t n);
/* Tensor.AddScalar (device.go:48). */
int fl_add_scalar(fl_context *ctx, int dtype, void *t, int64_t n, float v);
/* Tensor.Scale (device.go:51). */
int fl_scale(fl_context *ctx, int dtype, void *t, int64_t n, float v);
/* Tensor.AddBias (device.go:54): bias [cols] broadcast over rows. */
int fl_add_bias(fl_context *ctx, int dtype, void *t, int rows, int cols, const void *bias);
/* Tensor.Softmax / Gelu / Tanh (device.go:57-59) in place; act is
 * FL_ACT_SOFTMAX (row-wise), FL_ACT_GELU or FL_ACT_TANH. */
int fl_activation(fl_context *ctx, int dtype, void *t, int rows, int cols, int act, int math);
/* Tensor.LayerNorm (device.go:62): in place; gamma/beta fp32 [cols]
 * (bert.go:278-280 keeps LayerNorm parameters in fp32). */
int fl_layernorm(fl_context *ctx, int dtype, void *t, int rows, int cols, const float *gamma,
                 const float *beta, float eps);
/* Tensor.AddLayerNorm (device.go:64-72): t = LayerNorm(t + residual), the
 * residual (res_dtype) converted to t's dtype on load: bert.go:813-824 adds
 * an fp16 branch to the fp32 hidden state. */
int fl_add_layernorm(fl_context *ctx, int dtype, void *t, int res_dtype, const void *residual,
                     int rows, int cols, const float *gamma, const float *beta, float eps);
/* Tensor.Gather (device.go:72): out[i] = table[idx[i]]; idx on the host. */
int fl_gather_rows(fl_context *ctx, int dtype, const void *table, int rows, int cols,
                   const int64_t *idx, int n, void *out);
/* Tensor.ApplyRoPE (device.go:91-93; cpu_backend.go:760-805): in place on
 * [batch*seq, heads*head_dim], position = row % seq, rotate-half pairs
 * (i, i + head_dim/2); the reference fixes base = 10000. */
int fl_rope(fl_context *ctx, int dtype, void *t, int batch, int seq, int heads, int head_dim,
            float base);
/* RoPE over packed variable-length sequences; positions restart at 0 for
 * each sequence (what bert.go:619-624 intends for ragged batches). */
int fl_rope_varlen(fl_context *ctx, int dtype, void *t, const int64_t *lengths, int nseq,
                   int heads, int head_dim, float base);
/* Tensor.Attention (device.go:83-88; cpu_backend.go:662-758):
 * out = softmax(scale * Q K^T) V per (batch item, head) over [batch*seq, hidden]. */
int fl_attention(fl_context *ctx, int dtype, const void *q, const void *k, const void *v,
                 void *out, int batch, int seq, int heads, int hidden, float scale, int math);
/* Tensor.AttentionVarLen (device.go:85-90; cpu_backend.go:66-132): per
 * sequence attention over packed rows; lengths on the host. */
int fl_attention_varlen(fl_context *ctx, int dtype, const void *q, const void *k,
                        const void *v, void *out, const int64_t *lengths, int nseq, int heads,
                        int hidden, float scale, int math);
/* Tensor.Cast (device.go:107-109): n elements, device side, round to nearest. */
int fl_cast(fl_context *ctx, const void *src, int src_dtype, void *dst, int dst_dtype,
            int64_t n);
/* Tensor.HasNaN (device.go:111-112; cpu_backend.go:845-863): *out = 1 if any
 * element is NaN or +-Inf (synchronises). */
int fl_has_nan(fl_context *ctx, const void *t, int dtype, int64_t n, int *out);
/* Tensor.Slice (device.go:34) of a column range: copy rows [r0, r1) x cols
 * [c0, c1) of a [rows x cols] tensor into a dense [(r1-r0) x (c1-c0)] buffer
 * (metal_darwin.go:522-541).  A slice of all columns is a view (see the
 * conventions above), not a call. */
int fl_slice(fl_context *ctx, int dtype, const void *src, int rows, int cols, int r0, int r1,
             int c0, int c1, void *dst);
/* Masked mean-pool (+ L2 normalise when l2 != 0) over packed sequences:
 * out[b] = mean of hidden rows of sequence b; out is device fp32 [nseq x cols].
 * Not in the reference (its output is the CLS pooler). */
int fl_mean_pool(fl_context *ctx, int dtype, const void *hidden, int cols,
                 const int64_t *lengths, int nseq, int l2, float *out);

/* No counterpart in the reference.  fl_mean_pool for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): same arguments and the same results, bit
 * for bit, but it calls no hipMalloc / hipFree / host-to-device copy.  The
 * sequence lengths travel in the kernel arguments; cu_seqlens and the partial
 * sums go to a static scratch array of FL_NOALLOC_PARTIAL_BYTES + 4 KiB that
 * each GPU the library runs on holds until the process ends.  Limits (else
 * FL_ERR_INVALID): nseq <= FL_NOALLOC_MAX_SEQS and
 * nseq * ceil(max(lengths) / 64) * cols * 4 <= FL_NOALLOC_PARTIAL_BYTES.
 * Every call on one GPU shares that GPU's array.  Calls run in the order
 * they are made: calls of one context are ordered on its stream, and a call
 * from another context's stream first waits for the previous call's kernels
 * (an event, no allocation).  Calls recorded under graph capture are not
 * ordered against other streams: graphs that contain this call and run on
 * one GPU at the same time race on the array. */
#define FL_NOALLOC_MAX_SEQS 512
#define FL_NOALLOC_PARTIAL_BYTES (16 << 20)
int fl_mean_pool_noalloc(fl_context *ctx, int dtype, const void *hidden, int cols,
                         const int64_t *lengths, int nseq, int l2, float *out);

/* ---- Model-level forward (BertModel.ForwardBatch, bert.go:149-169) ----- */
typedef struct {
  int32_t vocab_size;   /* BertConfig fields (bert.go:20-30) */
  int32_t hidden;
  int32_t layers;
  int32_t heads;
  int32_t intermediate;
  int32_t max_pos;
  int32_t activation;   /* FL_ACT_GELU or FL_ACT_SWIGLU */
  int32_t position;     /* FL_POS_ABSOLUTE or FL_POS_ROPE */
  float rope_base;      /* reference hard-codes 10000 (cpu_backend.go:790) */
  float ln_eps;         /* reference hard-codes 1e-7 (bert.go:281) */
  int32_t dtype;        /* compute dtype: FL_F32, FL_F16 or FL_BF16 */
  int32_t math;         /* FL_MATH_REFERENCE or FL_MATH_EXACT */
  int32_t pool;         /* FL_POOL_* */
  int32_t has_bias;     /* 0 for bias-free models (Nomic) */
} fl_model_config;

/* NewBertModelWithBackend (bert.go:94-104) without the random init: weights
 * are zero until set. */
int fl_model_create(fl_context *ctx, const fl_model_config *cfg, fl_model **out);
int fl_model_free(fl_model *model);
/* Weight upload in the reference layout (the order of loader.go:29-90,
 * named): "word_emb" [V,H], "pos_emb" [P,H], "type_emb" [2,H],
 * "emb_ln_g"/"emb_ln_b" [H]; per layer l: "q_w.l" "k_w.l" "v_w.l" "o_w.l"
 * [H,H], "q_b.l" "k_b.l" "v_b.l" "o_b.l" [H], "attn_ln_g.l" "attn_ln_b.l" [H],
 * "inter_w.l" [H, I or 2I], "inter_b.l", "out_w.l" [I,H], "out_b.l" [H],
 * "out_ln_g.l" "out_ln_b.l" [H]; "pool_w" [H,H], "pool_b" [H].  Host fp32;
 * the backend converts and repacks for its kernels. */
int fl_model_set_weight(fl_model *model, const char *name, const float *data, int64_t n);
/* Loader.LoadFromRawBinary (weights/loader.go:29-90): every tensor of the
 * model as little-endian float32 in the loader's fixed order, with the shapes
 * NewBertModel allocates (position table and bias vectors included even where
 * the model does not use them; a bias-free model requires them to be zero). */
int fl_model_load_raw(fl_model *model, const char *path);
/* Loader.LoadFromSafeTensors (weights/loader.go:155-237): F32 tensors by
 * HuggingFace BERT name; 2-D linear ".weight" tensors are [out, in] and are
 * transposed. */
int fl_model_load_safetensors(fl_model *model, const char *path);
/* ForwardBatch over flat host ids (sum(lengths)) and per-sequence lengths;
 * writes [nseq x hidden] fp32 to host `out` (synchronises). */
int fl_model_forward(fl_model *model, const int64_t *ids, const int64_t *lengths, int nseq,
                     float *out);
/* fl_model_forward with the pooled vectors delivered as out_dtype: FL_F32
 * (float [nseq x hidden]) or FL_F16 (IEEE half bits, uint16 [nseq x
 * hidden], converted on the device with round-to-nearest-even): the
 * fp16 transport of processOutput's Cast(Float16) + ExtractBytes
 * (embeddings.go:256-286), half the bytes over PCIe. */
int fl_model_forward_ex(fl_model *model, const int64_t *ids, const int64_t *lengths, int nseq,
                        int out_dtype, void *out);
/* Same over right-padded [nseq x max_len] ids with a 0/1 attention mask
 * (1 = token); padding never enters any computation. */
int fl_model_forward_padded(fl_model *model, const int64_t *ids, const int64_t *mask, int nseq,
                            int max_len, float *out);
/* Device-resident variant: d_ids int32 [sum(lengths)] already on the device,
 * lengths on the host, d_out device fp32 [nseq x hidden].  Asynchronous on the
 * context stream. */
int fl_model_forward_device(fl_model *model, const int32_t *d_ids, const int64_t *lengths,
                            int nseq, float *d_out);
/* runInferenceOnDevice's batching loop (embeddings.go:690-775) in one call:
 * sequences are taken in order into batches that end before the sequence
 * that would pass max_seqs sequences or max_tokens tokens (a batch always
 * holds at least one; the reference's Linux GPU defaults are 512 and 16384,
 * embeddings.go:84-131).  Consecutive batches of that plan are computed
 * together, in forwards of up to 65536 tokens (a larger batch alone): a
 * sequence's vector does not depend on the other sequences of its forward,
 * so every output bit is what one forward per batch gives.  Consecutive
 * forwards run on three streams at once, each carrying its forward's id
 * upload, kernels and vector download, replacing the reference's
 * double-buffered outputs (:766-775).
 * ids: flat host ids of all sequences (framing included, as in
 * fl_model_forward); out: host fp32 [nseq x hidden] in input order;
 * batch_nan (optional) int32 [nseq]: 1 where the sequence's batch output held
 * a NaN/Inf (the per-batch HasNaN check, :757-764); nbatches (optional): the
 * number of batches of the plan.  Returns when every output is on the host;
 * fl_model_status then reports the plan's last batch. */
int fl_model_embed(fl_model *model, const int64_t *ids, const int64_t *lengths, int nseq,
                   int max_seqs, int64_t max_tokens, float *out, int32_t *batch_nan,
                   int *nbatches);
/* fl_model_embed with the pooled vectors delivered as out_dtype (FL_F32 or
 * FL_F16, as in fl_model_forward_ex). */
int fl_model_embed_ex(fl_model *model, const int64_t *ids, const int64_t *lengths, int nseq,
                      int max_seqs, int64_t max_tokens, int out_dtype, void *out,
                      int32_t *batch_nan, int *nbatches);
/* Tensor.HasNaN on the pooled output of the previous forward (computed inside
 * the pooling kernel, embeddings.go:757-764) and whether any id was outside
 * [0, vocab) (such ids read row 0).  Synchronises. */
int fl_model_status(fl_model *model, int *nan_in_output, int *bad_ids);
/* Last hidden states [sum(lengths) x hidden] of the previous forward, as fp32
 * on the host.  After fl_model_embed: its plan's last forward (the batches
 * computed together last). */
int fl_model_last_hidden(fl_model *model, float *out, int64_t n);
/* Kernel timing with HIP events on the context stream.  While enabled every
 * kernel of the forward is bracketed by events; fl_model_profile_read
 * synchronises and returns, per kernel class, the accumulated milliseconds and
 * launch count since it was enabled.  Classes: 0 embed, 1 qkv_gemm,
 * 2 attention, 3 o_gemm, 4 add_layernorm, 5 ffn_up_gemm, 6 ffn_down_gemm,
 * 7 pool. */
#define FL_PROF_CLASSES 8
int fl_model_set_profiling(fl_model *model, int enabled);
int fl_model_profile_read(fl_model *model, double *ms, int64_t *count);

#ifdef __cplusplus
}
#endif
#endif /* FLETCHER_HIP_H */
