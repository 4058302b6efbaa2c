// kernels.hpp -- host-side launchers of the gfx950 kernels (internal).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/fletcher_hip.h"

namespace fl {

enum EpiKind : int {
  EPI_STORE = 0,   // out = acc + bias
  EPI_GELU = 1,    // out = gelu(acc + bias)
  EPI_TANH = 2,    // out = tanh(acc + bias)
  EPI_SWIGLU = 3,  // gate/up interleaved in 16-column blocks -> out = silu(g) * u
  EPI_ROPE = 4,    // rotate-half RoPE on columns [0, rope_cols), head_dim 64
};

// Row order of a packed [N, K] weight matrix (and of its fp32 bias): which
// packed row holds logical output column n.  Within each 64-row block the
// four-wave kernel's layouts put the columns an MFMA lane accumulates (4 rows
// of each of 4 16-row tiles) on adjacent outputs, so the epilogue produces 16
// bytes per lane:
//   PACK_LANE16       lane g holds outputs [16g, 16g+16) of the block
//   PACK_ROPE         lane g holds [8g, 8g+8) and [32+8g, 32+8g+8) of a
//                     64-wide head, i.e. both halves of its rotate-half pairs
//   PACK_SWIGLU_LANE  lane g holds gate and up of outputs [8g, 8g+8) of the
//                     block's 32 outputs (gate = column o, up = column N/2+o)
// PACK_SWIGLU16 is the 4-wave kernels' gate/up interleave in 16-row blocks.
enum PackLayout : int {
  PACK_PLAIN = 0,
  PACK_SWIGLU16 = 1,
  PACK_LANE16 = 2,
  PACK_ROPE = 3,
  PACK_SWIGLU_LANE = 4,
};
__host__ __device__ inline int packed_row(int n, int N, int layout) {
  switch (layout) {
    case PACK_SWIGLU16: {
      const int half = N / 2;
      return n < half ? (n / 16) * 32 + n % 16 : ((n - half) / 16) * 32 + 16 + (n - half) % 16;
    }
    case PACK_LANE16: {
      const int r = n % 64, g = r / 16, f = (r / 4) % 4, i = r % 4;
      return n - r + f * 16 + g * 4 + i;
    }
    case PACK_ROPE: {
      const int r = n % 64, r2 = r % 32, g = r2 / 8, f = (r2 / 4) % 2 + 2 * (r / 32), i = r % 4;
      return n - r + f * 16 + g * 4 + i;
    }
    case PACK_SWIGLU_LANE: {
      const int half = N / 2, up = n >= half, o = up ? n - half : n;
      const int ro = o % 32, g = ro / 8, f = 2 * ((ro / 4) % 2) + up, i = ro % 4;
      return (o / 32) * 64 + f * 16 + g * 4 + i;
    }
    default: return n;
  }
}

// Element offset of (packed row r, column k) in a packed [N, K] weight
// matrix.  The four-wave kernel's layouts (16-bit, N % 256 == 0) are
// stored tiled: block (r / 256, k / 32) is 256 rows x 32 columns, 16 KB,
// blocks ordered by row tile then K slice; inside a block, row r % 256 is 64
// bytes whose 16-byte chunk c sits in slot c ^ ((r % 256) >> 1 & 3).  That is
// the GEMMs' LDS image of a weight K slice, so each is one contiguous DMA.
// The other layouts are row-major.
__host__ __device__ inline size_t packed_offset(int n, int k, int N, int K, int layout) {
  const int r = packed_row(n, N, layout);
  if (layout < PACK_LANE16) return (size_t)r * K + k;
  const int rr = r % 256, slot = ((k % 32) / 8) ^ ((rr >> 1) & 3);
  return ((size_t)(r / 256) * (K / 32) + k / 32) * 8192 + rr * 32 + slot * 8 + k % 8;
}

struct GemmEpilogue {
  int kind = EPI_STORE;
  int math = 0;                    // MathMode for GELU / tanh / silu
  const float* bias = nullptr;     // fp32 [N] in packed row order, or null
  const float2* rope_cs = nullptr; // [max_pos][32] (cos, sin)
  const int* pos = nullptr;        // [M] position of each row in its sequence
  int rope_cols = 0;
  int layout = PACK_PLAIN;         // PackLayout of B and bias
  // Output columns [0, q_cols) are multiplied by q_scale last (the query
  // block of a fused QKV projection, pre-scaled for the flash kernel).  The
  // four-wave kernel's STORE epilogue multiplies; its RoPE epilogue rotates
  // those columns with rope_cs_q, the table times q_scale.  gemm_nt_supported
  // rejects q_cols elsewhere.
  int q_cols = 0;
  float q_scale = 1.0f;
  const float2* rope_cs_q = nullptr;
  // Tiled activations (four-wave kernel only, gemm_tiled_ok): out_tiled
  // writes the SwiGLU output C in the weights' tiled layout (tiled_act_offset)
  // with rows up to a multiple of 256; a_tiled reads A that way.  Rows past M
  // of the last tile hold copies of row M-1, so they can be read as operand
  // rows like any other.
  bool out_tiled = false;
  bool a_tiled = false;
  // C has rows up to the next multiple of 256: rows past M are written to
  // their own rows instead of row M-1.  Without it, the rows of A past M
  // must be copies of row M-1 (true of row-major A, which is read clamped,
  // and of a tiled output written by an out_tiled GEMM from such an A).
  bool c_padded = false;
  // The few-row kernel may take this GEMM (when its cost model says so).  It
  // never writes output rows past M, so a consumer that relies on the padding
  // rows of a tiled output being copies of row M-1 (a four-wave GEMM reading
  // it with a_tiled and without c_padded) needs this off.
  bool allow_small = true;
};

// Element offset of (row m, column k) of an activation matrix with K columns
// stored tiled: the layout of packed_offset for a four-wave weight matrix.
__host__ __device__ inline size_t tiled_act_offset(int64_t m, int k, int K) {
  const int rr = (int)(m % 256), slot = ((k % 32) / 8) ^ ((rr >> 1) & 3);
  return ((size_t)(m / 256) * (K / 32) + k / 32) * 8192 + rr * 32 + slot * 8 + k % 8;
}

// Whether the tiled-activation options can be used for this GEMM (the
// four-wave kernel takes it): 16-bit, a four-wave layout, K % 128 == 0,
// K >= 256; out_tiled only with the SwiGLU epilogue.
bool gemm_tiled_ok(int dtype, int N, int K, int epi_kind, int math, bool has_bias, bool out_tiled,
                   bool a_tiled, bool c_padded);

// The packing the persistent four-wave GEMM needs for this problem (16-bit,
// N % 256 == 0, K % 128 == 0, K >= 256, an epilogue it has), or -1 when that
// kernel does not take it (the caller then packs PACK_PLAIN / PACK_SWIGLU16
// for the older 4-wave kernels).
int gemm_w4_layout(int dtype, int N, int K, int epi_kind, int math, bool has_bias);

// The output width a model uses for a 16-bit projection of N outputs: N, or
// the next multiple of 256 when the four-wave kernel takes that width and N
// does not (STORE / GELU / tanh epilogues).  The padding rows of the packed
// weights and bias are zero, so the extra output columns hold zeros (or the
// activation of zero) and are never read.
int gemm_padded_width(int dtype, int N, int K, int epi_kind, int math, bool has_bias);

// C[M, N] = A[M, K] * B[N, K]^T with the epilogue.  MFMA path; requires
// N % 64 == 0, K % 64 (16-bit) or K % 32 (fp32) == 0 and 16-byte aligned rows,
// and B packed as epi.layout says.
bool gemm_nt_supported(int dtype, int M, int N, int K, const void* A, int lda, const void* B,
                       int ldb, const void* C, int ldc, const GemmEpilogue& epi);
hipError_t launch_gemm_nt(int dtype, const void* A, int lda, const void* B, int ldb, void* C,
                          int ldc, int M, int N, int K, const GemmEpilogue& epi,
                          hipStream_t stream);

// Any shape / transpose: C = alpha * op(A) op(B) (+ bias, activation).
hipError_t launch_gemm_generic(int dtype, int trans_a, int trans_b, int M, int N, int K,
                               float alpha, const void* A, int lda, const void* B, int ldb,
                               void* C, int ldc, const float* bias, int act, int math,
                               hipStream_t stream);

// Packed (row0 + n, k) = in[k, n] (dtype elements, packed_offset): [rows =
// K, cols = N] into rows [row0, row0 + N) of a packed [ntot, K] weight matrix
// (ntot 0: N).
hipError_t launch_transpose(int dtype, const void* in, int rows, int cols, void* out,
                            int layout, hipStream_t stream, int row0 = 0, int ntot = 0);
// Packed (n, :) = in[n, :] (packed_offset) for an [N, K] matrix with row
// stride ld.
hipError_t launch_pack_rows(int dtype, const void* in, int ld, int N, int K, void* out,
                            int layout, hipStream_t stream);
// out[packed_row(row0 + n)] = in[n] for an fp32 vector of N, the packed
// vector having ntot entries (0: N).
hipError_t launch_pack_vec_f32(const float* in, int N, float* out, int layout, hipStream_t stream,
                               int row0 = 0, int ntot = 0);

// ---- attention ------------------------------------------------------------
// One query block of one (sequence, head).  The sequence's first row and
// length ride in the item, so a workgroup needs a single dependent load
// (its item) before it can address Q, K and V.
struct AttnWork {
  int s0;      // first row of the sequence in the packed tensors
  int len;     // sequence length
  int head;    // head index
  int q0;      // first query row (relative to the sequence start)
};
// Flash attention (exact math, online softmax) for head_dim 32 or 64, 16-bit
// types.  q_prescaled (head_dim 64 only): Q already holds q * scale * log2(e)
// (GemmEpilogue::q_scale).  xcd_group_size: consecutive work items (the query
// blocks of one sequence and head) kept on one XCD, clamped to [1, 32].
// out_tiled_cols > 0 (head size 64): out is written in the tiled activation
// layout (tiled_act_offset) with that many columns instead of row-major.
hipError_t launch_attention_flash(int dtype, const void* q, const void* k, const void* v,
                                  int ldqkv, void* out, int ldo, const int* cu_seqlens,
                                  const AttnWork* work, int n_work, int head_dim, float scale,
                                  int waves, bool q_prescaled, int xcd_group_size,
                                  hipStream_t stream, int out_tiled_cols = 0);
// Two-pass attention (exact row max, then reference ExpFast or exp) for
// head_dim 64 fp32.
hipError_t launch_attention_f32(const float* q, const float* k, const float* v, int ldqkv,
                                float* out, int ldo, const int* cu_seqlens,
                                const AttnWork* work, int n_work, float scale, int math,
                                hipStream_t stream);
// Any head_dim / dtype: one thread per query row.
hipError_t launch_attention_generic(int dtype, const void* q, const void* k, const void* v,
                                    int ldqkv, void* out, int ldo, const int* cu_seqlens,
                                    int nseq, int max_len, int heads, int head_dim, float scale,
                                    int math, hipStream_t stream);

// ---- normalisation / embedding ---------------------------------------------
// t = LN(t [+ residual]) row-wise, fp32 statistics; gamma/beta fp32.
// t_tiled: t is stored tiled (tiled_act_offset; 16-bit, cols % 256 == 0,
// cols <= 1024), the residual row-major with row stride ld_res (0: cols).
hipError_t launch_layernorm(int dtype, void* t, const void* residual, int rows, int cols,
                            const float* gamma, const float* beta, float eps,
                            hipStream_t stream, bool t_tiled = false, int ld_res = 0);
// t = LN(t [+ residual]) over row-major [rows, cols] for the per-op ABI: the
// residual in its own storage type (res_dtype, converted on load); with
// `shadow` (fp32 t only) the result is also stored as shadow_dtype (16-bit)
// into shadow [rows, cols] in the same pass.
hipError_t launch_layernorm_mixed(int dtype, void* t, int res_dtype, const void* residual,
                                  int rows, int cols, const float* gamma, const float* beta,
                                  float eps, int shadow_dtype, void* shadow, hipStream_t stream);
// x[t] = LN(word[ids[t]] + pos[pos_ids[t]] (if pos) + type[0]).  Ids outside
// [0, vocab) read row 0 and set *bad_id (never an out-of-bounds read).
hipError_t launch_embed_ln(int dtype, const int* ids, const int* pos_ids, const void* word,
                           const void* pos_table, const void* type_table, int T, int H,
                           const float* gamma, const float* beta, float eps, int vocab,
                           int* bad_id, void* out, hipStream_t stream, bool out_tiled = false);

// ---- elementwise ------------------------------------------------------------
// t += o, o stored as odtype and converted to t's type on load.
hipError_t launch_add(int dtype, void* t, int odtype, const void* o, int64_t n, hipStream_t s);
hipError_t launch_affine(int dtype, void* t, int64_t n, float mul, float add, hipStream_t s);
hipError_t launch_add_bias(int dtype, void* t, int rows, int cols, const void* bias,
                           hipStream_t s);
hipError_t launch_activation(int dtype, void* t, int rows, int cols, int act, int math,
                             hipStream_t s);
hipError_t launch_cast(const void* src, int sdt, void* dst, int ddt, int64_t n, int truncate_ref,
                       hipStream_t s);
hipError_t launch_has_nan(const void* t, int dtype, int64_t n, int* flag, hipStream_t s);
// p[0 .. n) = v, as a kernel (graph-capture safe, unlike a memset node).
hipError_t launch_fill_i32(int* p, int n, int v, hipStream_t s);
// flags[r] = 1 if row r of fp32 t [rows x cols] holds a NaN or an infinity, else 0.
hipError_t launch_row_nonfinite(const float* t, int rows, int cols, int* flags, hipStream_t s);
hipError_t launch_gather(int dtype, const void* table, int cols, const int* idx, int n,
                         void* out, hipStream_t s);
hipError_t launch_slice(int dtype, const void* src, int cols, int r0, int r1, int c0, int c1,
                        void* dst, hipStream_t s);
// RoPE in place with positions pos[row] and a (cos, sin) table [max_pos][head_dim/2].
hipError_t launch_rope(int dtype, void* t, int rows, int heads, int head_dim, int ld,
                       const int* pos, const float2* cs, hipStream_t s);
// Masked mean-pool (+L2) over cu_seqlens into fp32 out [nseq x cols]; sets
// *nan_flag (if non-null) when any pooled value is NaN/Inf.  `partial` is
// scratch of nseq * ceil(max_len / rows_per_chunk) * cols floats.
hipError_t launch_mean_pool_staged(int dtype, const void* hidden, int cols, const int* cu_seqlens,
                                   int nseq, int max_len, int l2, float* partial, float* out,
                                   int* nan_flag, int rows_per_chunk, hipStream_t s,
                                   bool tiled = false);
// fl_mean_pool_noalloc: sequence lengths travel by value in the kernel
// arguments, cu_seqlens and the partial sums go to the static per-device
// scratch array (noalloc_scratch); rows_per_chunk is kNoAllocRowsPerChunk, as
// in fl_mean_pool.
constexpr int kNoAllocRowsPerChunk = 64;
struct NoAllocLengths {
  int n;
  int len[FL_NOALLOC_MAX_SEQS];
};
// Address of the current device's scratch array (`device` must be current);
// looked up once per device and kept.
hipError_t noalloc_scratch(int device, void** out);
// Calls on one device from different streams run in call order (each waits
// for the previous call's kernels when that call used another stream),
// except under graph capture.
hipError_t launch_mean_pool_noalloc(int dtype, const void* hidden, int cols,
                                    const NoAllocLengths& lengths, int max_len, int l2,
                                    float* out, int device, void* scratch_dev, hipStream_t s);
// out[r, c] = silu(in[r, c]) * in[r, inter + c] over an unfused [rows, 2*inter] product.
hipError_t launch_swiglu(int dtype, const void* in, int rows, int inter, void* out, int math,
                         hipStream_t s);
// Gathers the first row of each sequence as fp32 [nseq x cols].
hipError_t launch_gather_cls(int dtype, const void* hidden, int cols, const int* cu_seqlens,
                             int nseq, float* out, hipStream_t s, bool tiled = false);
// Row-major copy of a tiled [rows, cols] activation matrix (tiled_act_offset).
hipError_t launch_untile(int dtype, const void* in, int64_t rows, int cols, void* out,
                         hipStream_t s);

}  // namespace fl
