// elementwise.hip -- memory-bound Tensor ops (device.go:44-116) and pooling.
//
// Add / Scale / AddScalar / AddBias / Gelu / Tanh / Softmax / Cast / HasNaN /
// Gather / Slice / ApplyRoPE, plus the masked mean-pool (+L2) and CLS gather
// that turn last hidden states into one vector per sequence.
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"

namespace fl {

static inline dim3 grid_for(int64_t n, int per_block = 256 * 4) {
  int64_t g = (n + per_block - 1) / per_block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return dim3((unsigned)g);
}

#define FL_GRID_STRIDE(i, n) \
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < (n); i += (int64_t)gridDim.x * blockDim.x)

// t += o: the other operand takes the receiver's type (Tensor.Add,
// metal_darwin.go:603-619), converted on load.
template <typename T, typename O>
__global__ void add_kernel(T* t, const O* o, int64_t n) {
#pragma clang fp contract(off)
  FL_GRID_STRIDE(i, n) t[i] = from_f<T>(to_f(t[i]) + to_f(from_f<T>(to_f(o[i]))));
}

template <typename T>
__global__ void affine_kernel(T* t, int64_t n, float mul, float add) {
#pragma clang fp contract(off)
  FL_GRID_STRIDE(i, n) {
    float v = to_f(t[i]);
    if (mul != 1.0f) v = v * mul;
    if (add != 0.0f) v = v + add;
    t[i] = from_f<T>(v);
  }
}

template <typename T>
__global__ void add_bias_kernel(T* t, int rows, int cols, const T* bias) {
#pragma clang fp contract(off)
  const int64_t n = (int64_t)rows * cols;
  FL_GRID_STRIDE(i, n) t[i] = from_f<T>(to_f(t[i]) + to_f(bias[i % cols]));
}

template <typename T, int ACT, int MATH>
__global__ void act_kernel(T* t, int64_t n) {
  FL_GRID_STRIDE(i, n) {
    const float v = to_f(t[i]);
    t[i] = from_f<T>(ACT == ACT_GELU ? gelu_m<MATH>(v) : tanh_m<MATH>(v));
  }
}

// Row softmax, one wave per row.  MATH_REFERENCE is SoftmaxFast
// (simd.go:78-100): ExpFast(v - max), sum, times 1/sum.
template <typename T, int MATH>
__global__ void __launch_bounds__(256) softmax_kernel(T* t, int rows, int cols) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  T* r = t + (size_t)row * cols;
  float mx = -INFINITY;
  for (int j = lane; j < cols; j += 64) mx = fmaxf(mx, to_f(r[j]));
  mx = wave_max(mx);
  float s = 0.f;
  for (int j = lane; j < cols; j += 64) {
    const float v = to_f(r[j]);
    s += MATH == MATH_REFERENCE ? exp_fast_ref(v - mx) : expf(v - mx);
  }
  s = wave_sum(s);
  const float inv = 1.0f / s;
  for (int j = lane; j < cols; j += 64) {
    const float v = to_f(r[j]);
    const float e = MATH == MATH_REFERENCE ? exp_fast_ref(v - mx) : expf(v - mx);
    r[j] = from_f<T>(e * inv);
  }
}

// SwiGLU over an unfused [rows, 2I] product (cpu_backend.go:636-654).
template <typename T, int MATH>
__global__ void swiglu_kernel(const T* in, int rows, int inter, T* out) {
  const int64_t n = (int64_t)rows * inter;
  FL_GRID_STRIDE(i, n) {
    const int64_t r = i / inter, c = i % inter;
    const float g = to_f(in[r * 2 * inter + c]);
    const float u = to_f(in[r * 2 * inter + inter + c]);
    out[i] = from_f<T>(silu_m<MATH>(g) * u);
  }
}

// Float32ToFloat16 of utils.go:13-72 (truncating; flush below 2^-14; clamp).
__device__ inline uint16_t f32_to_f16_ref(float f) {
  const uint32_t bits = __float_as_uint(f);
  if (isnan(f)) return 0x7E00;
  if (isinf(f)) return f > 0 ? 0x7C00 : 0xFC00;
  if (f > 65504.0f) f = 65504.0f;
  else if (f < -65504.0f) f = -65504.0f;
  const float a = fabsf(f);
  if (a < 6.10351562e-5f && a > 0.f) return f < 0 ? 0x8000 : 0x0000;
  const uint32_t b = __float_as_uint(f);
  (void)bits;
  const uint32_t sign = (b >> 16) & 0x8000u;
  const int e = (int)((b >> 23) & 0xFF) - 127 + 15;
  const uint32_t frac = (b >> 13) & 0x3FFu;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7BFFu);
  if (e <= 0) return (uint16_t)sign;
  return (uint16_t)(sign | ((uint32_t)e << 10) | frac);
}

template <typename S, typename D>
__global__ void cast_kernel(const S* src, D* dst, int64_t n) {
  FL_GRID_STRIDE(i, n) dst[i] = from_f<D>(to_f(src[i]));
}

__global__ void cast_f32_f16_ref_kernel(const float* src, uint16_t* dst, int64_t n) {
  FL_GRID_STRIDE(i, n) dst[i] = f32_to_f16_ref(src[i]);
}

template <typename T>
__global__ void has_nan_kernel(const T* t, int64_t n, int* flag) {
  bool bad = false;
  FL_GRID_STRIDE(i, n) {
    const float v = to_f(t[i]);
    bad |= !isfinite(v);
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(flag, 1);
}

// p[i] = v for i < n (a fill kernel: a captured graph replays it reliably,
// where memset nodes have given wrong results on replays after the first).
__global__ void fill_i32_kernel(int* p, int n, int v) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

// One wave per row of an fp32 [rows x cols] matrix: flags[r] = 1 if row r
// holds a NaN or an infinity, else 0 (every row's flag is written).
__global__ void row_nonfinite_kernel(const float* t, int rows, int cols, int* flags) {
  const int r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (r >= rows) return;  // uniform per wave
  const float* row = t + (size_t)r * cols;
  bool bad = false;
  for (int c = threadIdx.x & 63; c < cols; c += 64) bad |= !isfinite(row[c]);
  const bool any = __any(bad);
  if ((threadIdx.x & 63) == 0) flags[r] = any ? 1 : 0;
}

template <typename T>
__global__ void gather_kernel(const T* table, int cols, const int* idx, int n, T* out) {
  const int64_t total = (int64_t)n * cols;
  FL_GRID_STRIDE(i, total) {
    const int64_t r = i / cols, c = i % cols;
    out[i] = table[(size_t)idx[r] * cols + c];
  }
}

template <typename T>
__global__ void slice_kernel(const T* src, int cols, int r0, int c0, int rows_out, int cols_out,
                             T* dst) {
  const int64_t total = (int64_t)rows_out * cols_out;
  FL_GRID_STRIDE(i, total) {
    const int64_t r = i / cols_out, c = i % cols_out;
    dst[i] = src[(size_t)(r0 + r) * cols + c0 + c];
  }
}

// RoPE (cpu_backend.go:760-805): pairs (i, i + d/2) of each head rotated by
// the (cos, sin) of theta = pos * base^(-2i/d), table computed in float64.
template <typename T>
__global__ void rope_kernel(T* t, int rows, int heads, int hd, int ld, const int* pos,
                            const float2* cs) {
#pragma clang fp contract(off)
  const int half = hd / 2;
  const int64_t total = (int64_t)rows * heads * half;
  FL_GRID_STRIDE(i, total) {
    const int64_t r = i / ((int64_t)heads * half);
    const int rem = (int)(i % ((int64_t)heads * half));
    const int h = rem / half, j = rem % half;
    T* x = t + (size_t)r * ld + h * hd;
    const float2 c = cs[(size_t)pos[r] * half + j];
    const float x1 = to_f(x[j]), x2 = to_f(x[j + half]);
    x[j] = from_f<T>(x1 * c.x - x2 * c.y);
    x[j + half] = from_f<T>(x1 * c.y + x2 * c.x);
  }
}

// The same for 16-bit tensors with 16-byte aligned rows and half % 8 == 0:
// one work item = 8 consecutive pairs (j, j + half) of one head of one row,
// two 16-byte loads and stores of the tensor and four of the table, with
// the arithmetic of rope_kernel.
template <typename T>
__global__ void __launch_bounds__(256)
rope_vec_kernel(T* t, int rows, int heads, int hd, int ld, const int* pos, const float2* cs) {
#pragma clang fp contract(off)
  using V8 = T __attribute__((ext_vector_type(8)));
  const int half = hd / 2, cph = half / 8;  // 8-pair chunks per head
  const int per_row = heads * cph;
  const int64_t total = (int64_t)rows * per_row;
  FL_GRID_STRIDE(i, total) {
    const int r = (int)(i / per_row);
    const int rem = (int)(i - (int64_t)r * per_row);
    const int h = rem / cph, j0 = (rem - h * cph) * 8;
    T* x = t + (size_t)r * ld + h * hd + j0;
    const float4_t* c4 = (const float4_t*)(cs + (size_t)pos[r] * half + j0);
    const V8 a = *(const V8*)x, b = *(const V8*)(x + half);
    V8 oa, ob;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4_t c = c4[q];  // (cos, sin) of pairs j0 + 2q, j0 + 2q + 1
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float x1 = to_f(a[2 * q + e]), x2 = to_f(b[2 * q + e]);
        const float co = c[2 * e], si = c[2 * e + 1];
        oa[2 * q + e] = from_f<T>(x1 * co - x2 * si);
        ob[2 * q + e] = from_f<T>(x1 * si + x2 * co);
      }
    }
    *(V8*)x = oa;
    *(V8*)(x + half) = ob;
  }
}

// Masked mean-pool, stage 1: per (sequence, row chunk) column sums into
// part[seq][chunk][cols] (deterministic, no atomics).
template <typename T>
__global__ void __launch_bounds__(256)
pool_partial_kernel(const T* hidden, int cols, const int* cu, int rows_per_chunk, int max_chunks,
                    float* part, bool tiled) {
  const int seq = blockIdx.y, chunk = blockIdx.x;
  const int s0 = cu[seq], L = cu[seq + 1] - s0;
  const int r0 = chunk * rows_per_chunk;
  float* dst = part + ((size_t)seq * max_chunks + chunk) * cols;
  const int r1 = min(L, r0 + rows_per_chunk);
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    float acc = 0.f;
    for (int r = r0; r < r1; ++r)
      acc += to_f(hidden[tiled ? tiled_act_offset(s0 + r, c, cols) : (size_t)(s0 + r) * cols + c]);
    dst[c] = acc;
  }
}

// Stage 1 with 16-byte loads: the workgroup's RL x CV work items are (row
// lane, 16-byte column vector); row lane l sums rows r0 + l, r0 + l + RL, ...
// of its vector, and the RL partial sums are added in a fixed order through
// LDS (deterministic).  red holds RL x cols floats.
template <typename T>
__global__ void __launch_bounds__(256)
pool_partial_vec_kernel(const T* hidden, int cols, const int* cu, int rows_per_chunk,
                        int max_chunks, int RL, float* part, bool tiled) {
  constexpr int VE = 16 / (int)sizeof(T);
  using V = T __attribute__((ext_vector_type(VE)));
  extern __shared__ float red[];
  const int seq = blockIdx.y, chunk = blockIdx.x;
  const int s0 = cu[seq], L = cu[seq + 1] - s0;
  const int r0 = chunk * rows_per_chunk;
  const int r1 = min(L, r0 + rows_per_chunk);
  const int CV = cols / VE;
  for (int it = threadIdx.x; it < RL * CV; it += blockDim.x) {
    const int rl = it / CV, c = (it % CV) * VE;
    float acc[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) acc[i] = 0.f;
#pragma unroll 4
    for (int r = r0 + rl; r < r1; r += RL) {
      const size_t off = tiled ? tiled_act_offset(s0 + r, c, cols) : (size_t)(s0 + r) * cols + c;
      const V v = *(const V*)(hidden + off);
#pragma unroll
      for (int i = 0; i < VE; ++i) acc[i] += to_f(v[i]);
    }
#pragma unroll
    for (int i = 0; i < VE; ++i) red[rl * cols + c + i] = acc[i];
  }
  __syncthreads();
  float* dst = part + ((size_t)seq * max_chunks + chunk) * cols;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    float sum = 0.f;
    for (int l = 0; l < RL; ++l) sum += red[l * cols + c];
    dst[c] = sum;
  }
}

// Stage 2: sum chunks, divide by L, optional L2 normalisation, NaN flag.
__global__ void __launch_bounds__(256)
pool_final_kernel(const float* part, int cols, const int* cu, int rows_per_chunk, int max_chunks,
                  int l2, float* out, int* nan_flag) {
  __shared__ float red[4];
  const int seq = blockIdx.x;
  const int L = cu[seq + 1] - cu[seq];
  const int nchunks = (L + rows_per_chunk - 1) / rows_per_chunk;
  float* orow = out + (size_t)seq * cols;
  float ss = 0.f;
  bool bad = false;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    float acc = 0.f;
    for (int k = 0; k < nchunks; ++k) acc += part[((size_t)seq * max_chunks + k) * cols + c];
    const float m = acc / (float)L;
    orow[c] = m;
    ss += m * m;
  }
  if (l2) {
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const int nw = blockDim.x >> 6;
    float tot = 0.f;
    for (int w = 0; w < nw; ++w) tot += red[w];
    const float inv = 1.0f / fmaxf(sqrtf(tot), 1e-12f);
    for (int c = threadIdx.x; c < cols; c += blockDim.x) {
      const float v = orow[c] * inv;
      orow[c] = v;
      bad |= !isfinite(v);
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += blockDim.x) bad |= !isfinite(orow[c]);
  }
  if (nan_flag && __any(bad) && (threadIdx.x & 63) == 0) atomicOr(nan_flag, 1);
}

template <typename T>
__global__ void gather_cls_kernel(const T* hidden, int cols, const int* cu, int nseq,
                                  float* out, bool tiled) {
  const int64_t n = (int64_t)nseq * cols;
  FL_GRID_STRIDE(i, n) {
    const int s = (int)(i / cols), c = (int)(i % cols);
    out[i] = to_f(hidden[tiled ? tiled_act_offset(cu[s], c, cols) : (size_t)cu[s] * cols + c]);
  }
}

// Row-major copy of a tiled activation matrix, one 16-byte chunk per thread.
template <typename T>
__global__ void untile_kernel(const T* in, int64_t rows, int cols, T* out) {
  constexpr int E = 16 / sizeof(T);
  const int64_t n = rows * (cols / E);
  FL_GRID_STRIDE(i, n) {
    const int64_t r = i / (cols / E);
    const int c = (int)(i % (cols / E)) * E;
    *(u32x4_t*)(out + r * cols + c) = *(const u32x4_t*)(in + tiled_act_offset(r, c, cols));
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
#define FL_DISPATCH(dtype, T, ...)              \
  switch (dtype) {                              \
    case F32: {                                 \
      using T = float;                          \
      __VA_ARGS__;                              \
      break;                                    \
    }                                           \
    case F16: {                                 \
      using T = _Float16;                       \
      __VA_ARGS__;                              \
      break;                                    \
    }                                           \
    case BF16: {                                \
      using T = __bf16;                         \
      __VA_ARGS__;                              \
      break;                                    \
    }                                           \
    default: return hipErrorInvalidValue;       \
  }

hipError_t launch_add(int dtype, void* t, int odtype, const void* o, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  FL_DISPATCH(dtype, T, FL_DISPATCH(odtype, O, hipLaunchKernelGGL((add_kernel<T, O>), grid_for(n),
                                                                  dim3(256), 0, s, (T*)t,
                                                                  (const O*)o, n)));
  return hipGetLastError();
}

hipError_t launch_affine(int dtype, void* t, int64_t n, float mul, float add, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  FL_DISPATCH(dtype, T, hipLaunchKernelGGL(affine_kernel<T>, grid_for(n), dim3(256), 0, s, (T*)t,
                                           n, mul, add));
  return hipGetLastError();
}

hipError_t launch_add_bias(int dtype, void* t, int rows, int cols, const void* bias,
                           hipStream_t s) {
  const int64_t n = (int64_t)rows * cols;
  if (n <= 0) return hipSuccess;
  FL_DISPATCH(dtype, T, hipLaunchKernelGGL(add_bias_kernel<T>, grid_for(n), dim3(256), 0, s,
                                           (T*)t, rows, cols, (const T*)bias));
  return hipGetLastError();
}

hipError_t launch_activation(int dtype, void* t, int rows, int cols, int act, int math,
                             hipStream_t s) {
  const int64_t n = (int64_t)rows * cols;
  if (n <= 0) return hipSuccess;
  const bool ref = math == MATH_REFERENCE;
  if (act == ACT_SOFTMAX) {
    dim3 g((rows + 3) / 4);
    FL_DISPATCH(dtype, T,
                if (ref) hipLaunchKernelGGL((softmax_kernel<T, MATH_REFERENCE>), g, dim3(256), 0,
                                            s, (T*)t, rows, cols);
                else hipLaunchKernelGGL((softmax_kernel<T, MATH_EXACT>), g, dim3(256), 0, s,
                                        (T*)t, rows, cols));
  } else if (act == ACT_GELU) {
    FL_DISPATCH(dtype, T,
                if (ref) hipLaunchKernelGGL((act_kernel<T, ACT_GELU, MATH_REFERENCE>), grid_for(n),
                                            dim3(256), 0, s, (T*)t, n);
                else hipLaunchKernelGGL((act_kernel<T, ACT_GELU, MATH_EXACT>), grid_for(n),
                                        dim3(256), 0, s, (T*)t, n));
  } else if (act == ACT_TANH) {
    FL_DISPATCH(dtype, T,
                if (ref) hipLaunchKernelGGL((act_kernel<T, ACT_TANH, MATH_REFERENCE>), grid_for(n),
                                            dim3(256), 0, s, (T*)t, n);
                else hipLaunchKernelGGL((act_kernel<T, ACT_TANH, MATH_EXACT>), grid_for(n),
                                        dim3(256), 0, s, (T*)t, n));
  } else if (act != ACT_IDENTITY) {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_swiglu(int dtype, const void* in, int rows, int inter, void* out, int math,
                         hipStream_t s) {
  const int64_t n = (int64_t)rows * inter;
  if (n <= 0) return hipSuccess;
  FL_DISPATCH(dtype, T,
              if (math == MATH_REFERENCE) hipLaunchKernelGGL((swiglu_kernel<T, MATH_REFERENCE>),
                                                             grid_for(n), dim3(256), 0, s,
                                                             (const T*)in, rows, inter, (T*)out);
              else hipLaunchKernelGGL((swiglu_kernel<T, MATH_EXACT>), grid_for(n), dim3(256), 0,
                                      s, (const T*)in, rows, inter, (T*)out));
  return hipGetLastError();
}

hipError_t launch_cast(const void* src, int sdt, void* dst, int ddt, int64_t n, int truncate_ref,
                       hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if (truncate_ref) {
    if (sdt != F32 || ddt != F16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(cast_f32_f16_ref_kernel, grid_for(n), dim3(256), 0, s, (const float*)src,
                       (uint16_t*)dst, n);
    return hipGetLastError();
  }
  FL_DISPATCH(sdt, S, FL_DISPATCH(ddt, D, hipLaunchKernelGGL((cast_kernel<S, D>), grid_for(n),
                                                             dim3(256), 0, s, (const S*)src,
                                                             (D*)dst, n)));
  return hipGetLastError();
}

hipError_t launch_has_nan(const void* t, int dtype, int64_t n, int* flag, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  FL_DISPATCH(dtype, T, hipLaunchKernelGGL(has_nan_kernel<T>, grid_for(n), dim3(256), 0, s,
                                           (const T*)t, n, flag));
  return hipGetLastError();
}

hipError_t launch_fill_i32(int* p, int n, int v, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_i32_kernel, dim3((n + 255) / 256 < 64 ? (n + 255) / 256 : 64), dim3(256),
                     0, s, p, n, v);
  return hipGetLastError();
}

hipError_t launch_row_nonfinite(const float* t, int rows, int cols, int* flags, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(row_nonfinite_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, t, rows, cols,
                     flags);
  return hipGetLastError();
}

hipError_t launch_gather(int dtype, const void* table, int cols, const int* idx, int n,
                         void* out, hipStream_t s) {
  const int64_t total = (int64_t)n * cols;
  if (total <= 0) return hipSuccess;
  FL_DISPATCH(dtype, T, hipLaunchKernelGGL(gather_kernel<T>, grid_for(total), dim3(256), 0, s,
                                           (const T*)table, cols, idx, n, (T*)out));
  return hipGetLastError();
}

hipError_t launch_slice(int dtype, const void* src, int cols, int r0, int r1, int c0, int c1,
                        void* dst, hipStream_t s) {
  const int ro = r1 - r0, co = c1 - c0;
  const int64_t total = (int64_t)ro * co;
  if (total <= 0) return hipSuccess;
  FL_DISPATCH(dtype, T, hipLaunchKernelGGL(slice_kernel<T>, grid_for(total), dim3(256), 0, s,
                                           (const T*)src, cols, r0, c0, ro, co, (T*)dst));
  return hipGetLastError();
}

hipError_t launch_rope(int dtype, void* t, int rows, int heads, int head_dim, int ld,
                       const int* pos, const float2* cs, hipStream_t s) {
  const int64_t total = (int64_t)rows * heads * (head_dim / 2);
  if (total <= 0) return hipSuccess;
  if (dtype != F32 && (head_dim / 2) % 8 == 0 && ld % 8 == 0 && ((uintptr_t)t & 15) == 0 &&
      (int64_t)rows * heads * (head_dim / 16) < INT64_C(1) << 31) {
    const int64_t items = total / 8;
    if (dtype == F16)
      hipLaunchKernelGGL(rope_vec_kernel<_Float16>, grid_for(items, 256 * 2), dim3(256), 0, s,
                         (_Float16*)t, rows, heads, head_dim, ld, pos, cs);
    else
      hipLaunchKernelGGL(rope_vec_kernel<__bf16>, grid_for(items, 256 * 2), dim3(256), 0, s,
                         (__bf16*)t, rows, heads, head_dim, ld, pos, cs);
    return hipGetLastError();
  }
  FL_DISPATCH(dtype, T, hipLaunchKernelGGL(rope_kernel<T>, grid_for(total), dim3(256), 0, s,
                                           (T*)t, rows, heads, head_dim, ld, pos, cs));
  return hipGetLastError();
}

hipError_t launch_mean_pool_staged(int dtype, const void* hidden, int cols, const int* cu_seqlens,
                                   int nseq, int max_len, int l2, float* partial, float* out,
                                   int* nan_flag, int rows_per_chunk, hipStream_t s,
                                   bool tiled) {
  if (nseq <= 0) return hipSuccess;
  if (tiled && (dtype == F32 || cols % 32)) return hipErrorInvalidValue;
  const int max_chunks = (max_len + rows_per_chunk - 1) / rows_per_chunk;
  dim3 g1(max_chunks, nseq);
  const int ve = dtype == F32 ? 4 : 8;  // elements per 16-byte vector
  const int cv = cols / ve;
  const int rl = cv > 0 ? std::max(1, 256 / cv) : 1;
  const size_t lds = (size_t)rl * cols * sizeof(float);
  if (cols % ve == 0 && ((uintptr_t)hidden & 15) == 0 && lds <= 32768) {
    FL_DISPATCH(dtype, T, hipLaunchKernelGGL(pool_partial_vec_kernel<T>, g1, dim3(256), lds, s,
                                             (const T*)hidden, cols, cu_seqlens, rows_per_chunk,
                                             max_chunks, rl, partial, tiled));
  } else {
    const int threads = cols >= 256 ? 256 : 64;
    FL_DISPATCH(dtype, T, hipLaunchKernelGGL(pool_partial_kernel<T>, g1, dim3(threads), 0, s,
                                             (const T*)hidden, cols, cu_seqlens, rows_per_chunk,
                                             max_chunks, partial, tiled));
  }
  hipLaunchKernelGGL(pool_final_kernel, dim3(nseq), dim3(256), 0, s, partial, cols, cu_seqlens,
                     rows_per_chunk, max_chunks, l2, out, nan_flag);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Allocation-free mean pool (fl_mean_pool_noalloc).  Its cu_seqlens and
// partial sums live in `scratch`, a static array every GPU the library runs on
// holds until the process ends: cu_seqlens in the first kNoAllocCuBytes, the
// partial sums after them.  Host code never passes `scratch` itself (in host
// code the name is a stand-in, not a device address): noalloc_scratch()
// returns the address of the current device's copy, looked up once per device
// with hipGetSymbolAddress.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocCuBytes = 4096;
static_assert((FL_NOALLOC_MAX_SEQS + 1) * 4 <= (int)kNoAllocCuBytes, "cu_seqlens region");
static __device__ __align__(256) char scratch[kNoAllocCuBytes + FL_NOALLOC_PARTIAL_BYTES];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];
// Per device: an event recorded after the last call's kernels and the stream
// they ran on.  A call from another stream (another context on the same GPU)
// waits for that event first, so calls of several contexts one after the
// other do not overwrite each other's cu_seqlens and partial sums.
static hipEvent_t g_scratch_done[kMaxDevices];
static hipStream_t g_scratch_stream[kMaxDevices];

hipError_t noalloc_scratch(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    // Each GPU holds its own copy of the array at its own address; the
    // caller has made `device` current.
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device) return hipErrorInvalidDevice;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    // The ordering event (no device memory), made here with the address.
    e = hipEventCreateWithFlags(&g_scratch_done[device], hipEventDisableTiming);
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return hipSuccess;
}

// The array's address on `device` (set up by noalloc_scratch) must be what
// scratch_dev is: the launch below orders this call after the device's
// previous call when that one ran on another stream.
static hipError_t noalloc_order_begin(int device, hipStream_t s, bool* ordered) {
  *ordered = false;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) return e;
  // Under graph capture the call is recorded, not run: its order against
  // other streams is the caller's to set.
  if (cap != hipStreamCaptureStatusNone) return hipSuccess;
  if (g_scratch_stream[device] && g_scratch_stream[device] != s) {
    e = hipStreamWaitEvent(s, g_scratch_done[device], 0);
    if (e != hipSuccess) return e;
  }
  *ordered = true;
  return hipSuccess;
}

static hipError_t noalloc_order_end(int device, hipStream_t s) {
  hipError_t e = hipEventRecord(g_scratch_done[device], s);
  if (e != hipSuccess) return e;
  g_scratch_stream[device] = s;
  return hipSuccess;
}

// cu[0] = 0, cu[i + 1] = cu[i] + len[i] (one thread; at most 512 sequences).
__global__ void cu_from_lengths_kernel(NoAllocLengths a, int* cu) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int s = 0;
  cu[0] = 0;
  for (int i = 0; i < a.n; ++i) {
    s += a.len[i];
    cu[i + 1] = s;
  }
}

hipError_t launch_mean_pool_noalloc(int dtype, const void* hidden, int cols,
                                    const NoAllocLengths& lengths, int max_len, int l2,
                                    float* out, int device, void* scratch_dev, hipStream_t s) {
  if (lengths.n <= 0) return hipSuccess;
  if (!scratch_dev || device < 0 || device >= kMaxDevices) return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[device] != scratch_dev) return hipErrorInvalidValue;
  bool ordered = false;
  hipError_t e = noalloc_order_begin(device, s, &ordered);
  if (e != hipSuccess) return e;
  int* cu = (int*)scratch_dev;
  float* partial = (float*)((char*)scratch_dev + kNoAllocCuBytes);
  hipLaunchKernelGGL(cu_from_lengths_kernel, dim3(1), dim3(64), 0, s, lengths, cu);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // The same kernels as fl_mean_pool, so the results are identical bit for bit.
  e = launch_mean_pool_staged(dtype, hidden, cols, cu, lengths.n, max_len, l2, partial, out,
                              nullptr, kNoAllocRowsPerChunk, s, false);
  if (e != hipSuccess || !ordered) return e;
  return noalloc_order_end(device, s);
}

hipError_t launch_gather_cls(int dtype, const void* hidden, int cols, const int* cu_seqlens,
                             int nseq, float* out, hipStream_t s, bool tiled) {
  const int64_t total = (int64_t)nseq * cols;
  if (total <= 0) return hipSuccess;
  if (tiled && (dtype == F32 || cols % 32)) return hipErrorInvalidValue;
  FL_DISPATCH(dtype, T, hipLaunchKernelGGL(gather_cls_kernel<T>, grid_for(total), dim3(256), 0, s,
                                           (const T*)hidden, cols, cu_seqlens, nseq, out, tiled));
  return hipGetLastError();
}

hipError_t launch_untile(int dtype, const void* in, int64_t rows, int cols, void* out,
                         hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (dtype == F32 || cols % 32 || (((uintptr_t)in | (uintptr_t)out) & 15))
    return hipErrorInvalidValue;
  const int64_t total = rows * (cols / 8);
  FL_DISPATCH(dtype, T, hipLaunchKernelGGL(untile_kernel<T>, grid_for(total), dim3(256), 0, s,
                                           (const T*)in, rows, cols, (T*)out));
  return hipGetLastError();
}

}  // namespace fl
