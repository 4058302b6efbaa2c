// common.hpp -- shared types, numerics and launch helpers for the gfx950
// encoder-forward kernels.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

namespace fl {

// Storage types (device.go:119-124 numbers Float32 = 0, Float16 = 1; BF16 is
// an addition of this backend).
enum DType : int { F32 = 0, F16 = 1, BF16 = 2 };
// device.go:126-134
enum Act : int { ACT_IDENTITY = 0, ACT_GELU = 1, ACT_TANH = 2, ACT_SOFTMAX = 3, ACT_SWIGLU = 4 };
// MATH_REFERENCE evaluates the reference CPU formulas (simd.go ExpFast /
// TanhFast); MATH_EXACT uses hardware exp2 and an accurate tanh.
enum MathMode : int { MATH_REFERENCE = 0, MATH_EXACT = 1 };

inline size_t dtype_size(int dt) { return dt == F32 ? 4 : 2; }

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Element conversion
// ---------------------------------------------------------------------------
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int dtype = F32;
  __device__ static inline float to_f(float v) { return v; }
  __device__ static inline float from_f(float v) { return v; }
};
template <> struct Elem<_Float16> {
  static constexpr int dtype = F16;
  __device__ static inline float to_f(_Float16 v) { return (float)v; }
  __device__ static inline _Float16 from_f(float v) { return (_Float16)v; }
};
template <> struct Elem<__bf16> {
  static constexpr int dtype = BF16;
  __device__ static inline float to_f(__bf16 v) { return (float)v; }
  __device__ static inline __bf16 from_f(float v) { return (__bf16)v; }
};

template <typename T> __device__ inline float to_f(T v) { return Elem<T>::to_f(v); }
template <typename T> __device__ inline T from_f(float v) { return Elem<T>::from_f(v); }

// ---------------------------------------------------------------------------
// Reference numerics (internal/simd/simd.go), evaluated one rounded float32
// operation at a time so the device matches the CPU path's formulas.
// ---------------------------------------------------------------------------

// simd.go:7-46 ExpFast: clamp at +-88, t = x*log2e, k = trunc(t) then k--
// for t < 0, f = t - k, cubic in f, times 2^k.
__device__ inline float exp_fast_ref(float x) {
#pragma clang fp contract(off)
  if (x > 88.0f) return 1e38f;
  if (x < -88.0f) return 0.0f;
  float t = x * 1.442695f;
  int k = (int)t;
  if (t < 0.0f) k--;
  float f = t - (float)k;
  float p = 1.0f + f * (0.6931472f + f * (0.2402265f + f * 0.0555041f));
  return p * ldexpf(1.0f, k);
}

// A float32 product that is never fused into a following add: the reference
// scales scores (sgemm alpha) and subtracts the row max as two rounded
// operations, and ExpFast's floor step turns a fused residue below zero into a
// 0.56% jump, so the rounding must match.
__device__ inline float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

// simd.go:49-64 TanhFast.
__device__ inline float tanh_fast_ref(float x) {
#pragma clang fp contract(off)
  if (x > 4.0f) return 1.0f;
  if (x < -4.0f) return -1.0f;
  float x2 = x * x;
  return x * (27.0f + x2) / (27.0f + 9.0f * x2);
}

// simd.go:66-76 GeluFast (tanh-form GELU through TanhFast).
__device__ inline float gelu_ref(float x) {
#pragma clang fp contract(off)
  return 0.5f * x * (1.0f + tanh_fast_ref(0.7978846f * (x + 0.044715f * x * x * x)));
}

__device__ inline float tanh_exact(float x) { return tanhf(x); }

// 0.5 x (1 + tanh(y)) = x / (1 + exp(-2y)), y = sqrt(2/pi) (x + 0.044715 x^3):
// with -2y log2(e) = x (k1 + k2 x^2) it is five VALU operations and two
// transcendentals (exp2, reciprocal).  Large |x| saturate to x and -0.
__device__ inline float gelu_exact(float x) {
  constexpr float k1 = -2.0f * 0.7978845608f * 1.4426950409f;
  constexpr float k2 = k1 * 0.044715f;
  const float q = x * __builtin_fmaf(x * x, k2, k1);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(q));
}

template <int MATH> __device__ inline float gelu_m(float x) {
  if constexpr (MATH == MATH_REFERENCE) return gelu_ref(x);
  else return gelu_exact(x);
}
template <int MATH> __device__ inline float tanh_m(float x) {
  if constexpr (MATH == MATH_REFERENCE) return tanh_fast_ref(x);
  else return tanh_exact(x);
}
// cpu_backend.go:649 swish: x / (1 + float32(exp(float64(-x)))).
template <int MATH> __device__ inline float silu_m(float x) {
  if constexpr (MATH == MATH_REFERENCE) {
#pragma clang fp contract(off)
    return x / (1.0f + (float)exp(-(double)x));
  } else {
    // Hardware reciprocal (1 ulp): exp(-x) = inf gives -0, exp(-x) = 0 gives x.
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
  }
}

// ---------------------------------------------------------------------------
// Wave helpers (wave64)
// ---------------------------------------------------------------------------
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Remaps a linear workgroup id so that ids handed out to one XCD (the
// hardware deals workgroups round-robin over the 8 XCDs) become a contiguous
// range of logical tiles, keeping neighbouring tiles in one L2.
__device__ inline int xcd_remap(int bid, int nwg) {
  constexpr int kXcd = 8;
  int per = nwg / kXcd;
  if (per == 0) return bid;
  int full = per * kXcd;
  if (bid >= full) return bid;
  return (bid % kXcd) * per + bid / kXcd;
}

// Regroups a linear workgroup id so that every XCD receives runs of C
// consecutive logical ids: within each window of 8*C dispatches (C rounds
// over the 8 XCDs), XCD x gets logical ids [x*C, x*C + C).  The global order
// is kept at window granularity; ids past the last full window map to
// themselves.
__device__ inline int xcd_group(int bid, int nwg, int C) {
  constexpr int kXcd = 8;
  const int win = kXcd * C;
  if (bid >= (nwg / win) * win) return bid;
  const int r = bid % win;
  return bid - r + (r % kXcd) * C + r / kXcd;
}

}  // namespace fl

#define FL_HIP_CHECK(expr)                                   \
  do {                                                       \
    hipError_t _e = (expr);                                  \
    if (_e != hipSuccess) return ::fl::hip_fail(_e, #expr);  \
  } while (0)
