// norm.hip -- LayerNorm, residual+LayerNorm and the fused embedding kernel.
//
// LayerNorm follows cpu_backend.go:541-601: mean = sum/cols, variance =
// sum((x-mean)^2)/cols (two passes, here over registers), invStd =
// 1/float32(sqrt(float64(var+eps))), y = (x-mean)*invStd*gamma + beta, with
// fp32 statistics whatever the storage type.  AddLayerNorm
// (cpu_backend.go:603-610) adds the residual first.  One wave per row: a
// row of H = 768 is 12 values per lane held in registers, so every element is
// read once and written once.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace fl {

// Loads VEC consecutive elements starting at p as floats.
template <typename T, int VEC>
__device__ inline void load_vec(const T* p, float* out) {
  if constexpr (VEC == 8 && sizeof(T) == 2) {
    using V8 = T __attribute__((ext_vector_type(8)));
    V8 v = *(const V8*)p;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = to_f(v[i]);
  } else if constexpr (VEC == 4 && sizeof(T) == 2) {
    using V4 = T __attribute__((ext_vector_type(4)));
    V4 v = *(const V4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = to_f(v[i]);
  } else if constexpr (VEC == 4 && sizeof(T) == 4) {
    float4_t v = *(const float4_t*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = v[i];
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) out[i] = to_f(p[i]);
  }
}

// load_vec for data read once: 16-bit 8-vectors go out as non-temporal
// loads, which leave the caches to the data read again later (the residual
// stream the LayerNorm writes and the next kernels read).
template <typename T, int VEC>
__device__ inline void load_vec_once(const T* p, float* out) {
  if constexpr (VEC == 8 && sizeof(T) == 2) {
    using V8 = T __attribute__((ext_vector_type(8)));
    const V8 v = __builtin_nontemporal_load((const V8*)p);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = to_f(v[i]);
  } else {
    load_vec<T, VEC>(p, out);
  }
}

template <typename T, int VEC>
__device__ inline void store_vec(T* p, const float* in) {
  if constexpr (VEC == 8 && sizeof(T) == 2) {
    using V8 = T __attribute__((ext_vector_type(8)));
    V8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = from_f<T>(in[i]);
    *(V8*)p = v;
  } else if constexpr (VEC == 4 && sizeof(T) == 2) {
    using V4 = T __attribute__((ext_vector_type(4)));
    V4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = from_f<T>(in[i]);
    *(V4*)p = v;
  } else if constexpr (VEC == 4 && sizeof(T) == 4) {
    *(float4_t*)p = float4_t{in[0], in[1], in[2], in[3]};
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) p[i] = from_f<T>(in[i]);
  }
}

// Sum over the LPR consecutive lanes that share a row.
template <int LPR>
__device__ inline float group_sum(float v) {
#pragma unroll
  for (int o = LPR / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Normalises x[NCH][VEC] (this lane's share of one row, spread over LPR
// lanes; `valid` masks the tail) in place.
template <int NCH, int VEC, int LPR = 64>
__device__ inline void ln_core(float (&x)[NCH][VEC], const bool (&valid)[NCH], int cols,
                               const float* gamma, const float* beta, const int (&col0)[NCH],
                               float eps) {
#pragma clang fp contract(off)
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (valid[c])
#pragma unroll
      for (int i = 0; i < VEC; ++i) s += x[c][i];
  s = group_sum<LPR>(s);
  const float mean = s / (float)cols;
  float v = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (valid[c])
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float d = x[c][i] - mean;
        v += d * d;
      }
  v = group_sum<LPR>(v);
  const float var = v / (float)cols;
  const float inv = 1.0f / (float)sqrt((double)(var + eps));
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (valid[c])
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        x[c][i] = (x[c][i] - mean) * inv * gamma[col0[c] + i] + beta[col0[c] + i];
}

// R: the residual branch's storage type (converted on load, Tensor.Add's
// rule: the branch takes the receiver's type).  S: when it differs from T
// (an fp32 receiver), the normalised row is also stored as S into `shadow`,
// the 16-bit copy a following 16-bit Linear reads, in the same pass.
template <typename T, typename R, typename S, int NCH, int VEC>
__global__ void __launch_bounds__(256)
layernorm_kernel(T* t, const R* residual, int ldr, int rows, int cols, const float* gamma,
                 const float* beta, float eps, S* shadow) {
  constexpr bool SH = !std::is_same<S, T>::value;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  T* tr = t + (size_t)row * cols;
  const R* rr = residual ? residual + (size_t)row * ldr : nullptr;
  float x[NCH][VEC];
  bool valid[NCH];
  int col0[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    col0[c] = (lane + c * 64) * VEC;
    valid[c] = col0[c] < cols;
    if (valid[c]) {
      load_vec<T, VEC>(tr + col0[c], x[c]);
      if (rr) {
        float r[VEC];
        load_vec<R, VEC>(rr + col0[c], r);
#pragma unroll
        for (int i = 0; i < VEC; ++i) x[c][i] = x[c][i] + r[i];
      }
    }
  }
  ln_core<NCH, VEC>(x, valid, cols, gamma, beta, col0, eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (valid[c]) {
      store_vec<T, VEC>(tr + col0[c], x[c]);
      if constexpr (SH) store_vec<S, VEC>(shadow + (size_t)row * cols + col0[c], x[c]);
    }
}

// 16-byte vectors, LPR lanes per row (64 / LPR rows per wave): for H = 768
// in 16 bits, half a wave per row and three 16-byte loads per lane and
// tensor, so twice the rows per wave are in flight.
// TT: t is stored tiled (tiled_act_offset), 16-byte vectors never straddle
// a tiled chunk; the two rows of a wave are adjacent, so each load of the
// wave covers whole 128-byte lines of the tiled blocks.
template <typename T, typename R, typename S, int LPR, int NCH, int VEC, bool TT>
__global__ void __launch_bounds__(256)
layernorm_rows_kernel(T* t, const R* residual, int ldr, int rows, int cols, const float* gamma,
                      const float* beta, float eps, S* shadow) {
  constexpr bool SH = !std::is_same<S, T>::value;
  constexpr int RPW = 64 / LPR;
  const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + ((threadIdx.x & 63) / LPR);
  const int lane = threadIdx.x % LPR;
  if (row >= rows) return;
  const R* rr = residual ? residual + (size_t)row * ldr : nullptr;
  float x[NCH][VEC];
  bool valid[NCH];
  int col0[NCH];
  auto tp = [&](int col) -> T* {
    return TT ? t + tiled_act_offset(row, col, cols) : t + (size_t)row * cols + col;
  };
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    col0[c] = (lane + c * LPR) * VEC;
    valid[c] = col0[c] < cols;
    if (valid[c]) load_vec<T, VEC>(tp(col0[c]), x[c]);
  }
  if (rr) {
    // The residual branch (a GEMM output) is dead after this kernel.
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (valid[c]) {
        float r[VEC];
        load_vec_once<R, VEC>(rr + col0[c], r);
#pragma unroll
        for (int i = 0; i < VEC; ++i) x[c][i] = x[c][i] + r[i];
      }
  }
  ln_core<NCH, VEC, LPR>(x, valid, cols, gamma, beta, col0, eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (valid[c]) {
      store_vec<T, VEC>(tp(col0[c]), x[c]);
      if constexpr (SH) store_vec<S, VEC>(shadow + (size_t)row * cols + col0[c], x[c]);
    }
}

template <typename T, typename R, typename S, int LPR, int NCH, int VEC>
static hipError_t ln_rows_launch(void* t, const void* res, int ldr, int rows, int cols,
                                 const float* g, const float* b, float eps, hipStream_t s,
                                 bool tiled, void* shadow) {
  constexpr int rows_per_block = 4 * (64 / LPR);
  const dim3 grid((rows + rows_per_block - 1) / rows_per_block);
  if constexpr (std::is_same<R, T>::value && std::is_same<S, T>::value) {
    if (tiled) {
      hipLaunchKernelGGL((layernorm_rows_kernel<T, R, S, LPR, NCH, VEC, true>), grid, dim3(256),
                         0, s, (T*)t, (const R*)res, ldr, rows, cols, g, b, eps, (S*)shadow);
      return hipGetLastError();
    }
  } else {
    if (tiled) return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((layernorm_rows_kernel<T, R, S, LPR, NCH, VEC, false>), grid, dim3(256), 0,
                     s, (T*)t, (const R*)res, ldr, rows, cols, g, b, eps, (S*)shadow);
  return hipGetLastError();
}

template <typename T, typename R, typename S, int NCH, int VEC>
static hipError_t ln_launch(void* t, const void* res, int ldr, int rows, int cols, const float* g,
                            const float* b, float eps, hipStream_t s, void* shadow) {
  hipLaunchKernelGGL((layernorm_kernel<T, R, S, NCH, VEC>), dim3((rows + 3) / 4), dim3(256), 0,
                     s, (T*)t, (const R*)res, ldr, rows, cols, g, b, eps, (S*)shadow);
  return hipGetLastError();
}

// ldr: row stride of the residual (elements).
template <typename T, typename R, typename S>
static hipError_t ln_typed(void* t, const void* res, int ldr, int rows, int cols,
                           const float* g, const float* b, float eps, hipStream_t s, bool tiled,
                           void* shadow) {
  constexpr int V16 = 16 / sizeof(T);  // elements per 16-byte vector
  // Every operand's vectors aligned: V16 elements of T, of R and of S.
  auto aligned = [&](size_t vec) {
    return (((uintptr_t)t | (uintptr_t)res | (uintptr_t)shadow) % 16 == 0) &&
           ((size_t)ldr * sizeof(R)) % (vec * sizeof(R)) == 0 &&
           (uintptr_t)res % (vec * sizeof(R)) == 0 && (uintptr_t)shadow % (vec * sizeof(S)) == 0;
  };
  const bool a16 = aligned(V16);
  if (cols % (32 * V16) == 0 && cols <= 4 * 32 * V16 && a16) {
    switch (cols / (32 * V16)) {
      case 1: return ln_rows_launch<T, R, S, 32, 1, V16>(t, res, ldr, rows, cols, g, b, eps, s, tiled, shadow);
      case 2: return ln_rows_launch<T, R, S, 32, 2, V16>(t, res, ldr, rows, cols, g, b, eps, s, tiled, shadow);
      case 3: return ln_rows_launch<T, R, S, 32, 3, V16>(t, res, ldr, rows, cols, g, b, eps, s, tiled, shadow);
      case 4: return ln_rows_launch<T, R, S, 32, 4, V16>(t, res, ldr, rows, cols, g, b, eps, s, tiled, shadow);
    }
  }
  // Widths of 3 x 16 vectors (384 in 16 bits: MiniLM): 16 lanes per row.
  if (sizeof(T) == 2 && !tiled && cols == 3 * 16 * V16 && a16)
    return ln_rows_launch<T, R, S, 16, 3, V16>(t, res, ldr, rows, cols, g, b, eps, s, false,
                                               shadow);
  if (tiled) return hipErrorInvalidValue;
  if (cols % 4 == 0 && ((uintptr_t)t % (4 * sizeof(T))) == 0 &&
      ((uintptr_t)shadow % (4 * sizeof(S))) == 0 && ((uintptr_t)res % (4 * sizeof(R))) == 0 &&
      ((size_t)ldr % 4) == 0) {
    const int nch = (cols / 4 + 63) / 64;
    if (nch <= 1) return ln_launch<T, R, S, 1, 4>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
    if (nch <= 2) return ln_launch<T, R, S, 2, 4>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
    if (nch <= 3) return ln_launch<T, R, S, 3, 4>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
    if (nch <= 4) return ln_launch<T, R, S, 4, 4>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
    if (nch <= 8) return ln_launch<T, R, S, 8, 4>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
    if (nch <= 16) return ln_launch<T, R, S, 16, 4>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
    return hipErrorInvalidValue;
  }
  const int nch = (cols + 63) / 64;
  if (nch <= 2) return ln_launch<T, R, S, 2, 1>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
  if (nch <= 8) return ln_launch<T, R, S, 8, 1>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
  if (nch <= 32) return ln_launch<T, R, S, 32, 1>(t, res, ldr, rows, cols, g, b, eps, s, shadow);
  return hipErrorInvalidValue;
}

hipError_t launch_layernorm(int dtype, void* t, const void* residual, int rows, int cols,
                            const float* gamma, const float* beta, float eps,
                            hipStream_t stream, bool t_tiled, int ld_res) {
  if (rows <= 0) return hipSuccess;
  if (t_tiled && (dtype == F32 || cols % 256)) return hipErrorInvalidValue;
  if (ld_res <= 0) ld_res = cols;
  if (ld_res < cols) return hipErrorInvalidValue;
  switch (dtype) {
    case F32:
      return ln_typed<float, float, float>(t, residual, ld_res, rows, cols, gamma, beta, eps,
                                           stream, false, nullptr);
    case F16:
      return ln_typed<_Float16, _Float16, _Float16>(t, residual, ld_res, rows, cols, gamma, beta,
                                                    eps, stream, t_tiled, nullptr);
    case BF16:
      return ln_typed<__bf16, __bf16, __bf16>(t, residual, ld_res, rows, cols, gamma, beta, eps,
                                              stream, t_tiled, nullptr);
  }
  return hipErrorInvalidValue;
}

template <typename T, typename R>
static hipError_t ln_mixed_shadow(void* t, const void* res, int rows, int cols, const float* g,
                                  const float* b, float eps, hipStream_t s, int sdtype,
                                  void* shadow) {
  if (!shadow) return ln_typed<T, R, T>(t, res, cols, rows, cols, g, b, eps, s, false, nullptr);
  if constexpr (std::is_same<T, float>::value) {
    if (sdtype == F16)
      return ln_typed<T, R, _Float16>(t, res, cols, rows, cols, g, b, eps, s, false, shadow);
    if (sdtype == BF16)
      return ln_typed<T, R, __bf16>(t, res, cols, rows, cols, g, b, eps, s, false, shadow);
  }
  return hipErrorInvalidValue;
}

template <typename T>
static hipError_t ln_mixed_res(void* t, int rdtype, const void* res, int rows, int cols,
                               const float* g, const float* b, float eps, hipStream_t s,
                               int sdtype, void* shadow) {
  if (!res) rdtype = Elem<T>::dtype;
  switch (rdtype) {
    case F32: return ln_mixed_shadow<T, float>(t, res, rows, cols, g, b, eps, s, sdtype, shadow);
    case F16:
      return ln_mixed_shadow<T, _Float16>(t, res, rows, cols, g, b, eps, s, sdtype, shadow);
    case BF16:
      return ln_mixed_shadow<T, __bf16>(t, res, rows, cols, g, b, eps, s, sdtype, shadow);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_layernorm_mixed(int dtype, void* t, int res_dtype, const void* residual,
                                  int rows, int cols, const float* gamma, const float* beta,
                                  float eps, int shadow_dtype, void* shadow, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (shadow && dtype != F32) return hipErrorInvalidValue;
  switch (dtype) {
    case F32:
      return ln_mixed_res<float>(t, res_dtype, residual, rows, cols, gamma, beta, eps, stream,
                                 shadow_dtype, shadow);
    case F16:
      return ln_mixed_res<_Float16>(t, res_dtype, residual, rows, cols, gamma, beta, eps, stream,
                                    shadow_dtype, nullptr);
    case BF16:
      return ln_mixed_res<__bf16>(t, res_dtype, residual, rows, cols, gamma, beta, eps, stream,
                                  shadow_dtype, nullptr);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Fused embedding (BertEmbeddings.ForwardBatch, bert.go:215-261):
// x = (word[id] + pos[p]) + type[0], then LayerNorm, one write.
// ---------------------------------------------------------------------------
template <typename T, int NCH, int VEC, bool OT>
__global__ void __launch_bounds__(256)
embed_ln_kernel(const int* ids, const int* pos_ids, const T* word, const T* pos_table,
                const T* type_table, int rows, int cols, const float* gamma, const float* beta,
                float eps, int vocab, int* bad_id, T* out) {
#pragma clang fp contract(off)
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  int id = ids[row];
  if (id < 0 || id >= vocab) {
    if (lane == 0) atomicOr(bad_id, 1);
    id = 0;
  }
  const T* wr = word + (size_t)id * cols;
  const T* pr = pos_table ? pos_table + (size_t)pos_ids[row] * cols : nullptr;
  float x[NCH][VEC];
  bool valid[NCH];
  int col0[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    col0[c] = (lane + c * 64) * VEC;
    valid[c] = col0[c] < cols;
    if (valid[c]) {
      load_vec<T, VEC>(wr + col0[c], x[c]);
      float y[VEC];
      if (pr) {
        load_vec<T, VEC>(pr + col0[c], y);
#pragma unroll
        for (int i = 0; i < VEC; ++i) x[c][i] = x[c][i] + y[i];
      }
      load_vec<T, VEC>(type_table + col0[c], y);
#pragma unroll
      for (int i = 0; i < VEC; ++i) x[c][i] = x[c][i] + y[i];
    }
  }
  ln_core<NCH, VEC>(x, valid, cols, gamma, beta, col0, eps);
  // OT: tiled output (tiled_act_offset); VEC elements never straddle a chunk.
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (valid[c])
      store_vec<T, VEC>(OT ? out + tiled_act_offset(row, col0[c], cols)
                           : out + (size_t)row * cols + col0[c],
                        x[c]);
}

// The same with 16-byte vectors and LPR lanes per row (64 / LPR rows per
// wave), for 16-bit widths of 32*8 .. 4*32*8: the rows of a wave are
// adjacent, so with the tiled output each store of the wave writes whole
// 128-byte lines (two rows' 64-byte pieces of a K slice) instead of halves.
template <typename T, int LPR, int NCH, bool OT>
__global__ void __launch_bounds__(256)
embed_rows_kernel(const int* ids, const int* pos_ids, const T* word, const T* pos_table,
                  const T* type_table, int rows, int cols, const float* gamma,
                  const float* beta, float eps, int vocab, int* bad_id, T* out) {
#pragma clang fp contract(off)
  constexpr int VEC = 8, RPW = 64 / LPR;
  const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + ((threadIdx.x & 63) / LPR);
  const int lane = threadIdx.x % LPR;
  if (row >= rows) return;
  int id = ids[row];
  if (id < 0 || id >= vocab) {
    if (lane == 0) atomicOr(bad_id, 1);
    id = 0;
  }
  const T* wr = word + (size_t)id * cols;
  const T* pr = pos_table ? pos_table + (size_t)pos_ids[row] * cols : nullptr;
  float x[NCH][VEC];
  bool valid[NCH];
  int col0[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    col0[c] = (lane + c * LPR) * VEC;
    valid[c] = col0[c] < cols;
    if (valid[c]) {
      load_vec<T, VEC>(wr + col0[c], x[c]);
      float y[VEC];
      if (pr) {
        load_vec<T, VEC>(pr + col0[c], y);
#pragma unroll
        for (int i = 0; i < VEC; ++i) x[c][i] = x[c][i] + y[i];
      }
      load_vec<T, VEC>(type_table + col0[c], y);
#pragma unroll
      for (int i = 0; i < VEC; ++i) x[c][i] = x[c][i] + y[i];
    }
  }
  ln_core<NCH, VEC, LPR>(x, valid, cols, gamma, beta, col0, eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (valid[c])
      store_vec<T, VEC>(OT ? out + tiled_act_offset(row, col0[c], cols)
                           : out + (size_t)row * cols + col0[c],
                        x[c]);
}

struct EmbArgs {
  const int* ids;
  const int* pos_ids;
  const void* word;
  const void* pos_table;
  const void* type_table;
  int T, H;
  const float* g;
  const float* b;
  float eps;
  int vocab;
  int* bad_id;
  void* out;
  bool out_tiled;
};

template <typename T, int NCH, int VEC>
static hipError_t emb_launch(const EmbArgs& a, hipStream_t s) {
  if (a.out_tiled)
    hipLaunchKernelGGL((embed_ln_kernel<T, NCH, VEC, true>), dim3((a.T + 3) / 4), dim3(256), 0, s,
                       a.ids, a.pos_ids, (const T*)a.word, (const T*)a.pos_table,
                       (const T*)a.type_table, a.T, a.H, a.g, a.b, a.eps, a.vocab, a.bad_id,
                       (T*)a.out);
  else
    hipLaunchKernelGGL((embed_ln_kernel<T, NCH, VEC, false>), dim3((a.T + 3) / 4), dim3(256), 0,
                       s, a.ids, a.pos_ids, (const T*)a.word, (const T*)a.pos_table,
                       (const T*)a.type_table, a.T, a.H, a.g, a.b, a.eps, a.vocab, a.bad_id,
                       (T*)a.out);
  return hipGetLastError();
}

template <typename T, int NCH>
static hipError_t emb_rows_launch(const EmbArgs& a, hipStream_t s) {
  constexpr int rows_per_block = 4 * (64 / 32);
  const dim3 grid((a.T + rows_per_block - 1) / rows_per_block);
  if (a.out_tiled)
    hipLaunchKernelGGL((embed_rows_kernel<T, 32, NCH, true>), grid, dim3(256), 0, s, a.ids,
                       a.pos_ids, (const T*)a.word, (const T*)a.pos_table,
                       (const T*)a.type_table, a.T, a.H, a.g, a.b, a.eps, a.vocab, a.bad_id,
                       (T*)a.out);
  else
    hipLaunchKernelGGL((embed_rows_kernel<T, 32, NCH, false>), grid, dim3(256), 0, s, a.ids,
                       a.pos_ids, (const T*)a.word, (const T*)a.pos_table,
                       (const T*)a.type_table, a.T, a.H, a.g, a.b, a.eps, a.vocab, a.bad_id,
                       (T*)a.out);
  return hipGetLastError();
}

template <typename T>
static hipError_t emb_typed(const EmbArgs& a, hipStream_t s) {
  // 16-bit rows of 256 .. 1024 elements: 32 lanes per row, 16-byte vectors.
  if (sizeof(T) == 2 && a.H % 256 == 0 && a.H <= 1024) {
    switch (a.H / 256) {
      case 1: return emb_rows_launch<T, 1>(a, s);
      case 2: return emb_rows_launch<T, 2>(a, s);
      case 3: return emb_rows_launch<T, 3>(a, s);
      case 4: return emb_rows_launch<T, 4>(a, s);
    }
  }
  if (a.H % 4 == 0) {
    const int nch = (a.H / 4 + 63) / 64;
    if (nch <= 1) return emb_launch<T, 1, 4>(a, s);
    if (nch <= 3) return emb_launch<T, 3, 4>(a, s);
    if (nch <= 4) return emb_launch<T, 4, 4>(a, s);
    if (nch <= 8) return emb_launch<T, 8, 4>(a, s);
    if (nch <= 16) return emb_launch<T, 16, 4>(a, s);
    return hipErrorInvalidValue;
  }
  const int nch = (a.H + 63) / 64;
  if (nch <= 8) return emb_launch<T, 8, 1>(a, s);
  if (nch <= 32) return emb_launch<T, 32, 1>(a, s);
  return hipErrorInvalidValue;
}

hipError_t launch_embed_ln(int dtype, const int* ids, const int* pos_ids, const void* word,
                           const void* pos_table, const void* type_table, int T_, int H,
                           const float* gamma, const float* beta, float eps, int vocab,
                           int* bad_id, void* out, hipStream_t stream, bool out_tiled) {
  if (T_ <= 0) return hipSuccess;
  if (out_tiled && (dtype == F32 || H % 256)) return hipErrorInvalidValue;
  const EmbArgs a{ids, pos_ids, word, pos_table, type_table, T_, H, gamma, beta, eps, vocab,
                  bad_id, out, out_tiled};
  switch (dtype) {
    case F32: return emb_typed<float>(a, stream);
    case F16: return emb_typed<_Float16>(a, stream);
    case BF16: return emb_typed<__bf16>(a, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace fl
