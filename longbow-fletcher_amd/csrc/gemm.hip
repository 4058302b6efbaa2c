// gemm.hip -- MFMA GEMMs for gfx950 with fused epilogues.
//
// Backs Tensor.Mul / Linear / LinearActivation (cpu_backend.go:316-372,
// 612-660) and the encoder's projections (bert.go:610-824).  Layout:
// activations A[M, K] row-major (tokens x features), weights B[N, K]
// row-major (output features x input features, i.e. the reference's [in,out]
// matrix packed transposed at load time).
//
// The weight tile is the MFMA "A" operand and the token tile the "B"
// operand, so each lane of a 16x16 accumulator holds 4 consecutive output
// features of one token: stores are 8/16-byte vectors and the RoPE pair
// (j, j+32) and the SwiGLU (gate, up) pair land in the same lane.
#include <algorithm>
#include <climits>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace fl {

// Tuning constants, chosen by measurement on MI355X.
// Row blocks per group of the persistent tile order (an XCD's workgroups
// share a group's activation rows in L2).  Outputs of at most
// kGroupNarrowN column tiles go column-fastest instead (groups of one row
// block): an XCD's 32 workgroups then take about 11 whole row blocks per
// round, where groups of 8 row blocks x 3 column tiles split a third of the
// blocks between rounds and fetch them twice (Nomic at 131072 tokens:
// FFN-down 1458 -> 1099 MB per launch, O 370 -> 280 MB; times unchanged).
constexpr int kGroupM = 8;
constexpr int kGroupNarrowN = 4;
// Four-wave kernel: the next tile's first K step runs inside the epilogue.
constexpr bool kW4Fuse = true;
// Four-wave kernel, STORE epilogue: a partial last round of tiles runs as
// half-width tiles on twice as many CUs, for K up to kW4HalfMaxK (BERT-base
// at 32768 tokens: O 0.052 -> 0.050 ms, QKV 0.116 -> 0.112; at K = 3072,
// FFN-down, no gain: a half tile loads the whole tile's activations).
constexpr bool kW4Half = true;
constexpr int kW4HalfMaxK = 1024;
// Direct-LDS 16-bit GEMM (plain layouts): K step, LDS stages (48 KB, two
// workgroups per CU) and chunk swizzle (row >> 1) & 3.
constexpr int kLdsBK = 32, kLdsStages = 2, kLdsSwz = 1;

// Register-level K steps and accumulator reads of gemm_w4_kernel.
#include "gemm_w4.inc"

template <typename T> struct Mfma;
template <> struct Mfma<_Float16> {
  static constexpr int EPC = 8;  // elements per 16-byte fragment
  __device__ static inline void mma(float4_t& c, const u32x4_t& a, const u32x4_t& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                               __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<__bf16> {
  static constexpr int EPC = 8;
  __device__ static inline void mma(float4_t& c, const u32x4_t& a, const u32x4_t& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<float> {
  static constexpr int EPC = 4;
  // Four k=4 steps; lane group g supplies k = 4g + j at step j for both
  // operands, so the sum covers the 16 k values of the fragment.
  __device__ static inline void mma(float4_t& c, const u32x4_t& a, const u32x4_t& b) {
    const float4_t af = __builtin_bit_cast(float4_t, a);
    const float4_t bf = __builtin_bit_cast(float4_t, b);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[0], bf[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[1], bf[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[2], bf[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[3], bf[3], c, 0, 0, 0);
  }
};

struct GemmParams {
  const void* A;
  const void* B;
  void* C;
  int lda, ldb, ldc;
  int M, N, K;
  GemmEpilogue epi;
};

template <typename T>
__device__ inline void store4(T* dst, float4_t v) {
  if constexpr (sizeof(T) == 4) {
    *(float4_t*)dst = v;
  } else if constexpr (Elem<T>::dtype == F16) {
    half4_t h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    *(half4_t*)dst = h;
  } else {
    bf16x4_t h = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
    *(bf16x4_t*)dst = h;
  }
}

template <int EPI, int MATH>
__device__ inline float4_t act4(float4_t v) {
  if constexpr (EPI == EPI_GELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = gelu_m<MATH>(v[i]);
  } else if constexpr (EPI == EPI_TANH) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = tanh_m<MATH>(v[i]);
  }
  return v;
}

// BM x BN output tile per workgroup of WM x WN waves, K streamed in BK
// slices through double-buffered LDS (rows padded by one 16-byte fragment so
// the 16 lanes reading one fragment column hit distinct banks).
template <typename T, int BM, int BN, int BK, int WM, int WN, int EPI, int MATH>
__global__ void __launch_bounds__(WM* WN * 64) gemm_nt_kernel(GemmParams p) {
  constexpr int NT = WM * WN * 64;
  constexpr int EPC = Mfma<T>::EPC;
  constexpr int LS = BK + EPC;  // LDS row stride (elements)
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, FN = WTN / 16;
  constexpr int CPR = BK / EPC;
  constexpr int A_PER = BM * CPR / NT, B_PER = BN * CPR / NT;
  constexpr int KSTEP = 4 * EPC;
  static_assert(BM * CPR % NT == 0 && BN * CPR % NT == 0, "tile/thread mismatch");
  static_assert(BK % KSTEP == 0 && WTM % 16 == 0 && WTN % 16 == 0, "bad tile");
  static_assert(EPI != EPI_SWIGLU || FN % 2 == 0, "SwiGLU needs gate/up tile pairs");
  static_assert(EPI != EPI_ROPE || WTN % 64 == 0, "RoPE needs whole 64-wide heads per wave");

  __shared__ __attribute__((aligned(16))) T smem[2 * (BM + BN) * LS];
  T* As = smem;
  T* Bs = smem + 2 * BM * LS;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // Tile order: XCD-contiguous, then groups of 8 row-tiles sweeping all
  // column tiles so concurrently resident tiles share A and B in L2.
  const int num_m = (p.M + BM - 1) / BM, num_n = p.N / BN;
  const int L = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * num_n;
  const int g = L / per_group;
  const int first_m = g * GROUP_M;
  const int gsize = min(num_m - first_m, GROUP_M);
  const int r = L - g * per_group;
  const int m0 = (first_m + r % gsize) * BM;
  const int n0 = (r / gsize) * BN;

  const T* A = (const T*)p.A;
  const T* B = (const T*)p.B;
  const int M = p.M;

  u32x4_t ra[A_PER], rb[B_PER];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int c = tid + i * NT, row = c / CPR, col = (c % CPR) * EPC;
      const int gm = m0 + row;
      if (gm < M) ra[i] = *(const u32x4_t*)(A + (size_t)gm * p.lda + k0 + col);
      else ra[i] = u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = tid + i * NT, row = c / CPR, col = (c % CPR) * EPC;
      rb[i] = *(const u32x4_t*)(B + (size_t)(n0 + row) * p.ldb + k0 + col);
    }
  };
  auto lstore = [&](int buf) {
    T* as = As + buf * BM * LS;
    T* bs = Bs + buf * BN * LS;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int c = tid + i * NT, row = c / CPR, col = (c % CPR) * EPC;
      *(u32x4_t*)(as + row * LS + col) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = tid + i * NT, row = c / CPR, col = (c % CPR) * EPC;
      *(u32x4_t*)(bs + row * LS + col) = rb[i];
    }
  };

  float4_t acc[FN][TM];
#pragma unroll
  for (int f = 0; f < FN; ++f)
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[f][t] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = p.K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
    const T* as = As + cur * BM * LS + (wm * WTM + (lane & 15)) * LS;
    const T* bs = Bs + cur * BN * LS + (wn * WTN + (lane & 15)) * LS;
#pragma unroll
    for (int ks = 0; ks < BK / KSTEP; ++ks) {
      const int col = ks * KSTEP + (lane >> 4) * EPC;
      u32x4_t fa[TM], fb[FN];
#pragma unroll
      for (int t = 0; t < TM; ++t) fa[t] = *(const u32x4_t*)(as + t * 16 * LS + col);
#pragma unroll
      for (int f = 0; f < FN; ++f) fb[f] = *(const u32x4_t*)(bs + f * 16 * LS + col);
#pragma unroll
      for (int f = 0; f < FN; ++f)
#pragma unroll
        for (int t = 0; t < TM; ++t) Mfma<T>::mma(acc[f][t], fb[f], fa[t]);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  T* C = (T*)p.C;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int nbase = n0 + wn * WTN;
  const float* bias = p.epi.bias;
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int m = m0 + wm * WTM + t * 16 + lrow;
    if (m >= M) continue;
    T* crow = C + (size_t)m * p.ldc;
    if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
      for (int j = 0; j < FN / 2; ++j) {
        const int ng = nbase + 2 * j * 16 + lgrp * 4;
        float4_t gt = acc[2 * j][t], up = acc[2 * j + 1][t];
        if (bias) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            gt[i] += bias[ng + i];
            up[i] += bias[ng + 16 + i];
          }
        }
        float4_t o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = silu_m<MATH>(gt[i]) * up[i];
        store4<T>(crow + nbase / 2 + j * 16 + lgrp * 4, o);
      }
    } else if constexpr (EPI == EPI_ROPE) {
      const int ps = p.epi.pos[m];
      const float2* cs = p.epi.rope_cs + (size_t)ps * 32;
#pragma unroll
      for (int h = 0; h < FN / 4; ++h) {
        const int hb = nbase + h * 64;
        float4_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[q] = acc[h * 4 + q][t];
          if (bias) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[q][i] += bias[hb + q * 16 + lgrp * 4 + i];
          }
        }
        if (hb < p.epi.rope_cols) {
#pragma clang fp contract(off)
#pragma unroll
          for (int q = 0; q < 2; ++q) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float2 c = cs[q * 16 + lgrp * 4 + i];
              const float x1 = v[q][i], x2 = v[q + 2][i];
              v[q][i] = x1 * c.x - x2 * c.y;
              v[q + 2][i] = x1 * c.y + x2 * c.x;
            }
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) store4<T>(crow + hb + q * 16 + lgrp * 4, v[q]);
      }
    } else {
#pragma unroll
      for (int f = 0; f < FN; ++f) {
        const int n = nbase + f * 16 + lgrp * 4;
        float4_t v = acc[f][t];
        if (bias) {
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] += bias[n + i];
        }
        store4<T>(crow + n, act4<EPI, MATH>(v));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 16-bit GEMM with direct global->LDS loads (global_load_lds_dwordx4).
// Each wave instruction writes 64 lanes x 16 B = 1 KB contiguously in lane
// order, so the LDS layout is chosen through the source address each lane
// fetches: rows of BK = 64 halfs (128 B) unpadded, 16-byte chunk c of row r
// stored at position c ^ swz(r) so the 16 rows of an MFMA fragment read land
// in distinct banks.  Two statically distinct LDS stages let the compiler see
// that reads of one stage do not alias the DMA into the other; one barrier
// per K step.  Token rows past M are clamped to row M-1 (read, never stored).
// ---------------------------------------------------------------------------
template <int SWZ_SHIFT, int CPR>
__device__ inline int lds_swz(int row) { return (row >> SWZ_SHIFT) & (CPR - 1); }

template <typename T, int BM, int BN, int BK, int WM, int WN, int EPI, int MATH, int SWZ_SHIFT,
          int STAGES>
__global__ void __launch_bounds__(WM* WN * 64) gemm_lds_kernel(GemmParams p) {
  constexpr int NW = WM * WN;
  constexpr int ROWB = BK * 2;                // bytes per LDS row
  constexpr int CPR = BK / 8;                 // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;               // rows per 1 KB wave load
  static_assert(BK == 32 || BK == 64, "BK 32 or 64");
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, FN = WTN / 16;
  constexpr int A_INS = BM / RPI / NW, B_INS = BN / RPI / NW;  // 1 KB wave loads per stage
  static_assert(BM % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "tile/wave mismatch");
  static_assert(EPI != EPI_SWIGLU || FN % 2 == 0, "SwiGLU needs gate/up tile pairs");
  static_assert(EPI != EPI_ROPE || WTN % 64 == 0, "RoPE needs whole 64-wide heads per wave");
  static_assert(STAGES == 2 || STAGES == 3, "2 or 3 LDS stages");
  __shared__ __attribute__((aligned(1024))) char lds0[(BM + BN) * ROWB];
  __shared__ __attribute__((aligned(1024))) char lds1[(BM + BN) * ROWB];
  __shared__ __attribute__((aligned(1024))) char lds2[STAGES == 3 ? (BM + BN) * ROWB : 16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int num_m = (p.M + BM - 1) / BM, num_n = p.N / BN;
  const int L = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * num_n;
  const int g = L / per_group;
  const int first_m = g * GROUP_M;
  const int gsize = min(num_m - first_m, GROUP_M);
  const int r = L - g * per_group;
  const int m0 = (first_m + r % gsize) * BM;
  const int n0 = (r / gsize) * BN;
  const int M = p.M;

  // Per-lane 32-bit byte offsets from wave-uniform tile bases, so the loads
  // use the scalar-base + vector-offset form (one VGPR each).
  const char* abase = (const char*)p.A + (size_t)m0 * p.lda * sizeof(T);
  const char* bbase = (const char*)p.B + (size_t)n0 * p.ldb * sizeof(T);
  uint32_t aoff[A_INS], boff[B_INS];
#pragma unroll
  for (int i = 0; i < A_INS; ++i) {
    const int row = (wave * A_INS + i) * RPI + lane / CPR;
    const int c = (lane % CPR) ^ lds_swz<SWZ_SHIFT, CPR>(row);
    const int rr = min(row, M - 1 - m0);
    aoff[i] = (uint32_t)(rr * p.lda + c * 8) * (uint32_t)sizeof(T);
  }
#pragma unroll
  for (int i = 0; i < B_INS; ++i) {
    const int row = (wave * B_INS + i) * RPI + lane / CPR;
    const int c = (lane % CPR) ^ lds_swz<SWZ_SHIFT, CPR>(row);
    boff[i] = (uint32_t)(row * p.ldb + c * 8) * (uint32_t)sizeof(T);
  }
  auto issue = [&](char* stage, int k0) {
    const char* ak = abase + (size_t)k0 * sizeof(T);
    const char* bk = bbase + (size_t)k0 * sizeof(T);
#pragma unroll
    for (int i = 0; i < A_INS; ++i)
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(ak + aoff[i]),
          (__attribute__((address_space(3))) void*)(stage + (wave * A_INS + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < B_INS; ++i)
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(bk + boff[i]),
          (__attribute__((address_space(3))) void*)(stage + BM * ROWB + (wave * B_INS + i) * 1024),
          16, 0, 0);
  };

  // Fragment read offsets: row = base + t*16 + (lane & 15); swz depends on lane only.
  const int fr = lane & 15, fg = lane >> 4;
  const int swz = lds_swz<SWZ_SHIFT, CPR>(fr);
  const int a_row0 = (wm * WTM + fr) * ROWB;
  const int b_row0 = BM * ROWB + (wn * WTN + fr) * ROWB;

  float4_t acc[FN][TM];
#pragma unroll
  for (int f = 0; f < FN; ++f)
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[f][t] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const char* stage) {
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      const int co = ((ks * 4 + fg) ^ swz) << 4;
      u32x4_t fa[TM], fb[FN];
#pragma unroll
      for (int t = 0; t < TM; ++t) fa[t] = *(const u32x4_t*)(stage + a_row0 + t * 16 * ROWB + co);
#pragma unroll
      for (int f = 0; f < FN; ++f) fb[f] = *(const u32x4_t*)(stage + b_row0 + f * 16 * ROWB + co);
#pragma unroll
      for (int f = 0; f < FN; ++f)
#pragma unroll
        for (int t = 0; t < TM; ++t) Mfma<T>::mma(acc[f][t], fb[f], fa[t]);
      // Keep one K substep's fragments live at a time.
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // K is a multiple of STAGES*BK (checked on the host), so stages rotate
  // without a mid-loop exit (which would make every accumulator a loop-exit
  // value).  Loads of the last iterations re-fetch tile 0 into an idle stage
  // (in bounds, never read) to keep the wait counts uniform.  vmcnt counts
  // in issue order: waiting for <= one stage of loads outstanding means the
  // oldest stage has landed.
  const int nk = p.K / BK;
  auto kclamp = [&](int k) { return (k < nk ? k : 0) * BK; };
  if constexpr (STAGES == 2) {
    issue(lds0, 0);
    for (int kt = 0; kt < nk; kt += 2) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      issue(lds1, kclamp(kt + 1));
      compute(lds0);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      issue(lds0, kclamp(kt + 2));
      compute(lds1);
    }
  } else {
    constexpr int PER = A_INS + B_INS;  // loads per stage per wave
    static_assert(PER <= 63, "vmcnt range");
    issue(lds0, 0);
    issue(lds1, kclamp(1));
    for (int kt = 0; kt < nk; kt += 3) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER) : "memory");
      __syncthreads();
      issue(lds2, kclamp(kt + 2));
      compute(lds0);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER) : "memory");
      __syncthreads();
      issue(lds0, kclamp(kt + 3));
      compute(lds1);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER) : "memory");
      __syncthreads();
      issue(lds1, kclamp(kt + 4));
      compute(lds2);
    }
  }
  // No DMA may still target this workgroup's LDS when it exits.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  T* C = (T*)p.C;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int nbase = n0 + wn * WTN;
  const float* bias = p.epi.bias;
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int m = m0 + wm * WTM + t * 16 + lrow;
    if (m >= M) continue;
    T* crow = C + (size_t)m * p.ldc;
    if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
      for (int j = 0; j < FN / 2; ++j) {
        const int ng = nbase + 2 * j * 16 + lgrp * 4;
        float4_t gt = acc[2 * j][t], up = acc[2 * j + 1][t];
        if (bias) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            gt[i] += bias[ng + i];
            up[i] += bias[ng + 16 + i];
          }
        }
        float4_t o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = silu_m<MATH>(gt[i]) * up[i];
        store4<T>(crow + nbase / 2 + j * 16 + lgrp * 4, o);
      }
    } else if constexpr (EPI == EPI_ROPE) {
      const int ps = p.epi.pos[m];
      const float2* cs = p.epi.rope_cs + (size_t)ps * 32;
#pragma unroll
      for (int h = 0; h < FN / 4; ++h) {
        const int hb = nbase + h * 64;
        float4_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[q] = acc[h * 4 + q][t];
          if (bias) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[q][i] += bias[hb + q * 16 + lgrp * 4 + i];
          }
        }
        if (hb < p.epi.rope_cols) {
#pragma clang fp contract(off)
#pragma unroll
          for (int q = 0; q < 2; ++q) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float2 c = cs[q * 16 + lgrp * 4 + i];
              const float x1 = v[q][i], x2 = v[q + 2][i];
              v[q][i] = x1 * c.x - x2 * c.y;
              v[q + 2][i] = x1 * c.y + x2 * c.x;
            }
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) store4<T>(crow + hb + q * 16 + lgrp * 4, v[q]);
      }
    } else {
#pragma unroll
      for (int f = 0; f < FN; ++f) {
        const int n = nbase + f * 16 + lgrp * 4;
        float4_t v = acc[f][t];
        if (bias) {
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] += bias[n + i];
        }
        store4<T>(crow + n, act4<EPI, MATH>(v));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Four-wave kernel epilogue math.  B (and the bias) are packed so that the 16
// values a lane holds for one row block are adjacent outputs (PackLayout), so
// each lane produces 16 contiguous bytes at a time.  The bias is read in
// packed order.
// ---------------------------------------------------------------------------
// One 16x16x32 MFMA with 16-bit operands given as raw 16-byte fragments.
template <typename T> struct MfmaFrag;
template <> struct MfmaFrag<_Float16> {
  __device__ static inline void mma(float4_t& c, const u32x4_t& a, const u32x4_t& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                               __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  }
};
template <> struct MfmaFrag<__bf16> {
  __device__ static inline void mma(float4_t& c, const u32x4_t& a, const u32x4_t& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};

template <typename T>
__device__ inline u32x4_t pack8(float4_t a, float4_t b) {
  if constexpr (Elem<T>::dtype == F16) {
    half8_t h = {(_Float16)a[0], (_Float16)a[1], (_Float16)a[2], (_Float16)a[3],
                 (_Float16)b[0], (_Float16)b[1], (_Float16)b[2], (_Float16)b[3]};
    return __builtin_bit_cast(u32x4_t, h);
  } else {
    bf16x8_t h = {(__bf16)a[0], (__bf16)a[1], (__bf16)a[2], (__bf16)a[3],
                  (__bf16)b[0], (__bf16)b[1], (__bf16)b[2], (__bf16)b[3]};
    return __builtin_bit_cast(u32x4_t, h);
  }
}

// One 16-row block of a 64-feature group: v[f] is accumulator tile f of the
// group for the lane's token row; nbase is the group's first (packed) output
// column.  bias_at(f) gives the bias of tile f (added when BIAS), rope_at(k)
// the (cos, sin) float4 k of the row's position in the group's RoPE table
// (asked for every group; ignored past rope_cols).  The results go out
// through put(col, a, b): eight outputs of the lane's row starting at output
// column col.  ROT = false: the RoPE layout's columns without the rotation
// (a group wholly past rope_cols; rope_at is not called).
template <typename T, int EPI, int MATH, bool BIAS, bool ROT = true, typename BiasAt,
          typename RopeAt, typename Put>
__device__ __attribute__((always_inline)) inline void w4_epilogue_block(
    const GemmParams& p, float4_t (&v)[4], int nbase, int lane, BiasAt&& bias_at,
    RopeAt&& rope_at, Put&& put) {
  const int g = lane >> 4;
  if constexpr (BIAS) {
#pragma unroll
    for (int f = 0; f < 4; ++f) v[f] += bias_at(f);
  }
  if constexpr (EPI == EPI_SWIGLU) {
    // PACK_SWIGLU_LANE: tiles 2h / 2h+1 are gate / up of outputs 8g+4h+i.
    float4_t o[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[h][i] = silu_m<MATH>(v[2 * h][i]) * v[2 * h + 1][i];
    }
    put(nbase / 2 + g * 8, o[0], o[1]);
  } else if constexpr (EPI == EPI_ROPE) {
    // PACK_ROPE: tiles 0 / 1 hold dims 8g+i / 8g+4+i of the head, tiles
    // 2 / 3 their rotate-half partners 32+8g+i / 32+8g+4+i.  Heads past
    // rope_cols rotate by the identity (cos 1, sin 0), which leaves them
    // unchanged; the code stays free of branches.
    const bool rot = nbase < p.epi.rope_cols;
#pragma unroll
    for (int f = 0; f < 2 && ROT; ++f) {
#pragma clang fp contract(off)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float4_t c = rope_at(f * 2 + h);  // (cos, sin) of dims 8g + 4f + 2h, +1
        c = rot ? c : float4_t{1.f, 0.f, 1.f, 0.f};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int i = 2 * h + e;
          const float x1 = v[f][i], x2 = v[f + 2][i];
          const float co = c[2 * e], si = c[2 * e + 1];
          v[f][i] = x1 * co - x2 * si;
          v[f + 2][i] = x1 * si + x2 * co;
        }
      }
    }
    put(nbase + g * 8, v[0], v[1]);
    put(nbase + 32 + g * 8, v[2], v[3]);
  } else {
    // PACK_LANE16: tile f holds outputs 16g+4f+i.
#pragma unroll
    for (int f = 0; f < 4; ++f) v[f] = act4<EPI, MATH>(v[f]);
    if (nbase < p.epi.q_cols) {
#pragma unroll
      for (int f = 0; f < 4; ++f) v[f] *= p.epi.q_scale;
    }
    put(nbase + g * 16, v[0], v[1]);
    put(nbase + g * 16 + 8, v[2], v[3]);
  }
}

// 16-byte chunk swizzle of an LDS row: the 16 rows of one fragment read
// land on distinct banks (64-byte rows: pairs of rows share a 128-byte bank
// line; 128-byte rows: one row per bank line).
template <int CPR>
__device__ inline int w4_swz(int row) {
  if constexpr (CPR == 4) return (row >> 1) & 3;
  else return (row & 7) ^ ((row >> 3) & 1);
}

// ---------------------------------------------------------------------------
// Four-wave 16-bit GEMM: 256x256 tiles, one wave per SIMD, each wave owning a
// 128x128 output block (64 accumulator tiles in AGPRs), NS LDS stages of
// 32-deep K slices of weights packed tiled (packed_offset).  Against 128x64
// wave tiles (eight waves, two per SIMD) this reads a third fewer bytes from
// LDS per MFMA; the price is that nothing hides the epilogue.
//
// A K step is written out as volatile asm: 64 MFMAs, interleaved with the 16
// LDS fragment reads of the next step (into the other register set) and the
// wave's 8 DMA loads of step s+NS-1, in a fixed order the compiler cannot
// rearrange.  The step ends with the DMA wait for step s+2, the fragment
// wait and one barrier.
//
// Step s reads stage (s+1)%NS and loads stage (s+NS-1)%NS = (s-1)%NS, which
// was last read in step s-2, before the barrier that ended it.  At the end of
// step s each wave waits until its own loads of step s+2 have landed; after
// the barrier every wave's have.
// ---------------------------------------------------------------------------
// f(integral_constant<int, i>) for i = 0 .. N-1, unrolled.
template <int N, int I = 0, typename F>
__device__ __attribute__((always_inline)) inline void w4_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    w4_for<N, I + 1>(f);
  }
}

// The K-step blocks set m0 (the LDS address of DMA loads) themselves; the
// compiler emits no m0 use of its own in this kernel.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One 1 KB DMA load outside the K-step blocks (prologue): 64 lanes x 16
// bytes from gsrc + voff into LDS at lds_dst.
__device__ __attribute__((always_inline)) inline void w4_dma(uint32_t lds_dst, uint32_t voff,
                                                             const void* gsrc) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2" ::"s"(lds_dst),
      "v"(voff), "s"(gsrc)
      : "memory", "m0");
}

template <typename T, int EPI, int MATH, int NS>
__global__ void __launch_bounds__(256) gemm_w4_kernel(GemmParams p, int ntiles, int nhalf) {
  constexpr int BM = 256, BN = 256, BK = 32, ROWB = 64;
  constexpr int STAGE = (BM + BN) * ROWB;     // 32 KB
  constexpr int NLD = 8;                      // 1 KB loads per wave per step
  const int GROUP_M = p.N / BN <= kGroupNarrowN ? 1 : kGroupM;
  constexpr bool F16T = Elem<T>::dtype == F16;
  static_assert(NS == 4, "the K loop runs in groups of four steps, one per stage");
  // NS stages, then an 8 KB epilogue staging area per wave.
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE + 4 * 8192];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  const int G = (int)gridDim.x;
  const int me = xcd_remap((int)blockIdx.x, G);
  // Tiles ntiles .. ntiles + nhalf - 1 (STORE only) run as two 256x128
  // halves each, on workgroups 0 .. 2 * nhalf - 1 after their full tiles
  // (the host makes that the last, partial round): half tile me & 1 of tile
  // ntiles + me / 2, both halves on one XCD.  A half tile loads the whole
  // tile's K slices like a full one (the same DMA, waits and LDS layout), so
  // the pipeline runs on across tiles unchanged; only its MFMAs, fragment
  // reads (feature blocks 0-3 of its 128 weight rows) and epilogue are
  // half-width.
  constexpr bool HALF = EPI == EPI_STORE && MATH == MATH_EXACT;
  const int my_full = me < ntiles ? (ntiles - 1 - me) / G + 1 : 0;
  const bool has_half = HALF && me < 2 * nhalf;
  const int my_tiles = my_full + (has_half ? 1 : 0);
  if (my_tiles == 0) return;
  const bool chunked = (ntiles % G == 0) && (G % 8 == 0);
  const int per = G / 8;
  const int num_m = (p.M + BM - 1) / BM, num_n = p.N / BN;
  const int per_group = GROUP_M * num_n;
  // Tile i of this workgroup: its 256x256 block and half (-1: the whole tile).
  auto coords = [&](int i, int& m0, int& n0, int& hf) __attribute__((always_inline)) {
    const bool h = has_half && i == my_full;
    hf = h ? (me & 1) : -1;
    const int L = h ? ntiles + (me >> 1)
                    : chunked ? (me / per) * (my_full * per) + i * per + (me % per) : i * G + me;
    const int g = L / per_group;
    const int first_m = g * GROUP_M;
    const int gsize = min(num_m - first_m, GROUP_M);
    const int r = L - g * per_group;
    m0 = (first_m + r % gsize) * BM;
    n0 = (r / gsize) * BN;
  };
  const int nk = p.K / BK;

  // Fragment reads: A block t is rows 128*wm + 16t + (lane & 15), B block f
  // rows 128*wn + 16f + (lane & 15), 16-byte k chunk lane >> 4 (swizzled).
  const int fr = lane & 15, fg = lane >> 4;
  const uint32_t co = (uint32_t)((fg ^ w4_swz<4>(fr)) << 4);
  const uint32_t rdA = lds0 + (uint32_t)((wm * 128 + fr) * ROWB) + co;
  const uint32_t rdB = lds0 + (uint32_t)(BM * ROWB + (wn * 128 + fr) * ROWB) + co;
  // Half tiles: weight rows 128 * half + 64 * wn + 16f + (lane & 15), f < 4.
  const uint32_t rdBh = lds0 + (uint32_t)(BM * ROWB + (wn * 64 + fr) * ROWB) + co;
  const uint32_t dma0 = lds0 + (uint32_t)wave * 4096;

  // DMA geometry: wave w loads activation rows [64w, 64w+64) (loads 0-3) and
  // weight rows [64w, 64w+64) (loads 4-7) of each stage, 16 rows x 64 bytes
  // per load; lane l writes 16-byte chunk l%4 of row l/4, holding global
  // chunk (l%4) ^ swz(row).  Activation rows past M re-read row M-1.  The
  // weights are stored tiled (tiled_offset), so their loads are contiguous.
  const int lrow = lane >> 2, lcol = lane & 3;
  uint32_t off[NLD];
  const char* ka = nullptr;  // DMA cursor: token / weight base of the next K slice to load
  const char* kb = nullptr;
  constexpr size_t KB_STEP = (size_t)BN * BK * sizeof(T);  // one tiled weight block
  const bool a_tiled = p.epi.a_tiled;
  const size_t KA_STEP = a_tiled ? (size_t)BM * BK * sizeof(T) : BK * sizeof(T);
  uint32_t rdBn = rdB;  // weight fragment base of the tile load_tile was given
  auto load_tile = [&](int ti) __attribute__((always_inline)) {
    int m0, n0, hf;
    coords(ti, m0, n0, hf);
    rdBn = hf < 0 ? rdB : rdBh + (uint32_t)(hf * 128 * ROWB);
    ka = a_tiled ? (const char*)p.A + (size_t)(m0 / BM) * nk * KA_STEP
                 : (const char*)p.A + (size_t)m0 * p.lda * sizeof(T);
    kb = (const char*)p.B + (size_t)(n0 / BN) * nk * KB_STEP;
    const int lim = p.M - 1 - m0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wave * 64 + j * 16 + lrow;
      const int c = lcol ^ w4_swz<4>(row);
      off[j] = a_tiled ? (uint32_t)((wave * 4 + j) * 1024 + lane * 16)
                       : (uint32_t)(min(row, lim) * p.lda + c * 8) * (uint32_t)sizeof(T);
      off[4 + j] = (uint32_t)((wave * 4 + j) * 1024 + lane * 16);
    }
  };

  // DMA of the cursor's step into stage st, then advance the cursor.
  auto load_step = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NLD; ++j)
      w4_dma(dma0 + st * STAGE + (j < 4 ? j * 1024 : BM * ROWB + (j - 4) * 1024), off[j],
             j < 4 ? ka : kb);
    ka += KA_STEP;
    kb += KB_STEP;
  };

  // Prologue: steps 0 .. 3 into stages 0 .. 3; wait for steps 0 and 1;
  // fragments of step 0 into register set 0.
  load_tile(0);
  uint32_t rdBc = rdBn;  // weight fragment base of the tile being multiplied
  if constexpr (EPI == EPI_ROPE) {
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) load_step(s);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NLD) : "memory");
  } else {
#pragma unroll
    for (int s = 0; s < NS; ++s) load_step(s);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * NLD) : "memory");
  }
  asm volatile(FL_W4_READ_0 ::"v"(rdA), "v"(rdBc) : "memory", FL_W4_CLOBBER_V);

  // K step j of a group of four (global step s = j mod 4, since every tile
  // has a multiple of four steps): register set j % 2, reads stage (j+1)%4,
  // loads the cursor's step into stage (j+3)%4, then advances the cursor.
  // It first waits (vmcnt VM) until its own loads of step s+1 have landed.
  // A tile's first step (Z) loads nothing: its slice, step 3, went out
  // before the previous tile's epilogue, so that the next two steps' waits
  // can let the epilogue's stores stay outstanding.
  // H: a half tile's step (32 MFMAs, 12 fragment reads, the same loads).
  // rdb: the weight fragment base of the tile whose next step is read (the
  // next tile's in a tile's last step).
  auto kstep = [&](auto jc, auto zero, auto vmc, auto hc, uint32_t rdb)
                   __attribute__((always_inline)) {
    constexpr int J = decltype(jc)::value;
    constexpr int Z = decltype(zero)::value;  // 0 accumulate, 1 zero without DMA, 2 zero with DMA
    constexpr int VM = decltype(vmc)::value;
    constexpr bool H = decltype(hc)::value;
    constexpr uint32_t RD = ((J + 1) % NS) * STAGE, DM = ((J + NS - 1) % NS) * STAGE;
#define FL_W4_ARGS                                                                          \
  ::"v"(rdA + RD), "v"(rdb + RD), "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]),        \
      "v"(off[4]), "v"(off[5]), "v"(off[6]), "v"(off[7]), "s"(dma0 + DM), "s"(ka), "s"(kb),  \
      "n"(VM)                                                                              \
  : "memory", "m0", "scc", FL_W4_CLOBBER_V, FL_W4_CLOBBER_A
#define FL_W4_HCASE(j, z)                                                                   \
  if constexpr (J % 2 == j && Z == z) {                                                    \
    if constexpr (F16T) asm volatile(FL_W4_HSTEP_F16_##j##_##z FL_W4_ARGS);                 \
    else asm volatile(FL_W4_HSTEP_BF16_##j##_##z FL_W4_ARGS);                               \
  }
    if constexpr (H) {
      FL_W4_HCASE(0, 0) FL_W4_HCASE(0, 1) FL_W4_HCASE(0, 2)
      FL_W4_HCASE(1, 0) FL_W4_HCASE(1, 1) FL_W4_HCASE(1, 2)
    } else if constexpr (F16T) {
      if constexpr (J % 2 == 0 && Z == 0) asm volatile(FL_W4_STEP_F16_0_0 FL_W4_ARGS);
      if constexpr (J % 2 == 0 && Z == 1) asm volatile(FL_W4_STEP_F16_0_1 FL_W4_ARGS);
      if constexpr (J % 2 == 0 && Z == 2) asm volatile(FL_W4_STEP_F16_0_2 FL_W4_ARGS);
      if constexpr (J % 2 == 1 && Z == 0) asm volatile(FL_W4_STEP_F16_1_0 FL_W4_ARGS);
      if constexpr (J % 2 == 1 && Z == 1) asm volatile(FL_W4_STEP_F16_1_1 FL_W4_ARGS);
      if constexpr (J % 2 == 1 && Z == 2) asm volatile(FL_W4_STEP_F16_1_2 FL_W4_ARGS);
    } else {
      if constexpr (J % 2 == 0 && Z == 0) asm volatile(FL_W4_STEP_BF16_0_0 FL_W4_ARGS);
      if constexpr (J % 2 == 0 && Z == 1) asm volatile(FL_W4_STEP_BF16_0_1 FL_W4_ARGS);
      if constexpr (J % 2 == 0 && Z == 2) asm volatile(FL_W4_STEP_BF16_0_2 FL_W4_ARGS);
      if constexpr (J % 2 == 1 && Z == 0) asm volatile(FL_W4_STEP_BF16_1_0 FL_W4_ARGS);
      if constexpr (J % 2 == 1 && Z == 1) asm volatile(FL_W4_STEP_BF16_1_1 FL_W4_ARGS);
      if constexpr (J % 2 == 1 && Z == 2) asm volatile(FL_W4_STEP_BF16_1_2 FL_W4_ARGS);
    }
#undef FL_W4_HCASE
#undef FL_W4_ARGS
    if constexpr (Z != 1) {
      ka += KA_STEP;
      kb += KB_STEP;
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  // FUSE: the next tile's first K step (accumulating into 0, no DMA) runs
  // inside this tile's epilogue, each of its MFMAs right after the four
  // accumulator reads of the tile it restarts, so the MFMAs execute while the
  // reads and the epilogue's math issue.  fused_read(t, h, v) returns the
  // accumulators of row block t, feature group h (v[f] = tile 8(4h+f) + t).
  constexpr bool FUSE = kW4Fuse && EPI != EPI_ROPE;
  auto fused_read = [&](auto tc, auto hc, float4_t (&v)[4]) __attribute__((always_inline)) {
    constexpr int TB = decltype(tc)::value, HB = decltype(hc)::value;
    constexpr uint32_t RD1 = (1 % NS) * STAGE;
    float x[16];
#define FL_W4_FUSED_ASM(name)                                                               \
  asm volatile(name                                                                         \
               : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]), \
                 "=&v"(x[6]), "=&v"(x[7]), "=&v"(x[8]), "=&v"(x[9]), "=&v"(x[10]),           \
                 "=&v"(x[11]), "=&v"(x[12]), "=&v"(x[13]), "=&v"(x[14]), "=&v"(x[15])        \
               : "v"(rdA + RD1), "v"(rdBn + RD1)                                           \
               : "memory", FL_W4_CLOBBER_V, FL_W4_CLOBBER_A)
#define FL_W4_FUSED_CASE(t, h)                                                              \
  if constexpr (TB == t && HB == h) {                                                       \
    if constexpr (F16T) FL_W4_FUSED_ASM(FL_W4_FUSED_F16_##t##_##h);                         \
    else FL_W4_FUSED_ASM(FL_W4_FUSED_BF16_##t##_##h);                                       \
  }
    FL_W4_FUSED_CASE(0, 0) FL_W4_FUSED_CASE(0, 1) FL_W4_FUSED_CASE(1, 0) FL_W4_FUSED_CASE(1, 1)
    FL_W4_FUSED_CASE(2, 0) FL_W4_FUSED_CASE(2, 1) FL_W4_FUSED_CASE(3, 0) FL_W4_FUSED_CASE(3, 1)
    FL_W4_FUSED_CASE(4, 0) FL_W4_FUSED_CASE(4, 1) FL_W4_FUSED_CASE(5, 0) FL_W4_FUSED_CASE(5, 1)
    FL_W4_FUSED_CASE(6, 0) FL_W4_FUSED_CASE(6, 1) FL_W4_FUSED_CASE(7, 0) FL_W4_FUSED_CASE(7, 1)
#undef FL_W4_FUSED_CASE
#undef FL_W4_FUSED_ASM
#pragma unroll
    for (int f = 0; f < 4; ++f) v[f] = float4_t{x[4 * f], x[4 * f + 1], x[4 * f + 2], x[4 * f + 3]};
  };

  // Epilogue: accumulator tiles come out four at a time (one 16-row block
  // of one 64-feature group), so the compiler's registers stay below v128.
  // Each 16-row block of the wave's outputs (RB bytes per row) is assembled
  // row-major in the wave's LDS staging area (16-byte chunk c of row r in
  // slot c ^ (r % CPRW)) and stored from there as whole rows: every store
  // instruction writes 64/CPRW rows of RB contiguous bytes, where the
  // accumulator layout alone would scatter 16-byte pieces over 16 rows.
  // A unit is one 16-row block of the wave's outputs (both feature groups).
  constexpr int RB = EPI == EPI_SWIGLU ? 128 : 256, CPRW = RB / 16;
  constexpr int NUNITS = 8, RD = 2;
  // Loads of the epilogue (bias, positions) are issued before its first
  // store: the memory counter completes in issue order, so a wait for a
  // load issued after a store would also wait for the store.  RoPE tables
  // (the same table and rows for both heads of the wave: gemm_w4_ok) are
  // fetched RD units ahead, so that the stores a table load queues behind
  // have had RD units of time to complete.
  // (The bias test is hoisted out of the epilogue so that its code has no
  // data-dependent branches around loads: the compiler's wait counts stay
  // exact only on straight-line code.)
  auto epilogue_hb = [&](int ti, auto hbc) __attribute__((always_inline)) {
    constexpr bool HB = decltype(hbc)::value;
    int m0, n0, hf;
    coords(ti, m0, n0, hf);
    int ln = lane;
    asm volatile("" : "+v"(ln));
    // The last MFMAs' results must be written before they are read.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    const int r = ln & 15, g = ln >> 4;
    const int mrow = m0 + wm * 128 + r;
    const int cbase = n0 + wn * 128;  // the wave's first packed feature
    char* stg = lds + NS * STAGE + wave * 8192;
    const int mlast = p.epi.c_padded ? INT_MAX : p.M - 1;
    float4_t bv[2][4];
    if constexpr (HB) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int f = 0; f < 4; ++f)
          bv[h][f] = *(const float4_t*)(p.epi.bias + cbase + h * 64 + f * 16 + g * 4);
    }
    int pos[8];
    float4_t cs[RD + 1][4];  // [unit % (RD + 1)][k]
    if constexpr (EPI == EPI_ROPE) {
#pragma unroll
      for (int t = 0; t < 8; ++t) pos[t] = p.epi.pos[min(mrow + t * 16, p.M - 1)];
    }
    const float2* table = cbase < p.epi.q_cols ? p.epi.rope_cs_q : p.epi.rope_cs;
    auto fetch_cs = [&](auto uc) __attribute__((always_inline)) {
      constexpr int u = decltype(uc)::value;
      if constexpr (EPI == EPI_ROPE && u < NUNITS) {
        // Loaded for every tile (in bounds; unused past rope_cols).
        const float4_t* src = (const float4_t*)(table + (size_t)pos[u] * 32 + g * 8);
#pragma unroll
        for (int k = 0; k < 4; ++k) cs[u % (RD + 1)][k] = src[k];
      }
    };
    // Unit u is assembled in an LDS buffer of 4 KB (ubuf) and stored from
    // there.  STORE / SwiGLU: buffer u % 2, stored while unit u+1 is
    // computed, so the LDS round trip of one overlaps the other's math.
    // RoPE: six buffers (the staging area and this wave's 8 KB of stages 0
    // and 3, both free during the epilogue); units 0-5 are computed before
    // the first store, so every table load is issued ahead of every store.
    const int col0 = EPI == EPI_SWIGLU ? cbase / 2 : cbase;
    auto ubuf = [&](int u) __attribute__((always_inline)) -> char* {
      if constexpr (EPI != EPI_ROPE) return stg + (u & 1) * 4096;
      const int b = u < 6 ? u : u - 6;
      char* base = b < 2 ? stg : lds + (b < 4 ? 0 : 3) * STAGE + wave * 8192;
      return base + (b & 1) * 4096;
    };
    // rotc = false (RoPE kernel, a wave wholly past rope_cols): two staging
    // buffers and no tables, as for STORE.
    auto compute_unit = [&](auto uc, auto rotc) __attribute__((always_inline)) {
      constexpr int u = decltype(uc)::value;
      constexpr int t = u;
      constexpr bool ROT = decltype(rotc)::value;
      char* buf = ROT ? ubuf(u) : stg + (u & 1) * 4096;
      if constexpr (ROT) fetch_cs(std::integral_constant<int, u + RD>{});
      auto put = [&](int col, float4_t a, float4_t b) __attribute__((always_inline)) {
        const int c = (col - col0) >> 3;
        *(u32x4_t*)(buf + r * RB + ((c ^ (r % CPRW)) << 4)) = pack8<T>(a, b);
      };
      auto block = [&](auto hc) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value;
        float4_t v[4];
        if constexpr (FUSE && ROT) {
          fused_read(std::integral_constant<int, t>{}, hc, v);
        } else {
          v[0] = W4Acc<(4 * h + 0) * 8 + t>::read();
          v[1] = W4Acc<(4 * h + 1) * 8 + t>::read();
          v[2] = W4Acc<(4 * h + 2) * 8 + t>::read();
          v[3] = W4Acc<(4 * h + 3) * 8 + t>::read();
        }
        w4_epilogue_block<T, EPI, MATH, HB, ROT>(
            p, v, cbase + h * 64, ln, [&](int f) { return bv[h][f]; },
            [&](int k) { return cs[u % (RD + 1)][k]; }, put);
      };
      block(I0{});
      block(I1{});
    };
    // The QKV (RoPE) and SwiGLU outputs are written as non-temporal stores:
    // at the encoder's sizes they are larger than the caches and the next
    // kernel reads them from the start, so the cached copies would only
    // evict data read again sooner (measured: QKV GEMM -3%, attention -4%,
    // FFN-up -1.4%).
    constexpr bool NTS = EPI == EPI_ROPE || EPI == EPI_SWIGLU;
    auto put16 = [&](T* dst, u32x4_t val) __attribute__((always_inline)) {
      if constexpr (NTS) __builtin_nontemporal_store(val, (u32x4_t*)dst);
      else *(u32x4_t*)dst = val;
    };
    auto store_unit = [&](auto uc, auto rotc) __attribute__((always_inline)) {
      constexpr int u = decltype(uc)::value;
      constexpr int t = u;
      const char* buf = decltype(rotc)::value ? ubuf(u) : stg + (u & 1) * 4096;
      if constexpr (EPI == EPI_SWIGLU) {
        if (p.epi.out_tiled) {
          // Tiled output: the unit's 16 rows of each 32-column K slice are one
          // contiguous 1 KB block; lane l writes row l/4, slot l%4 of it.  Rows
          // past M hold row M-1's outputs: they fill the tile's last rows.
          const int rr = ln >> 2, slot = ln & 3;
          const int trow = wm * 128 + t * 16;  // first row of the unit in its 256-row tile
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            const int cc = kk * 4 + (slot ^ ((rr >> 1) & 3));
            const u32x4_t val = *(const u32x4_t*)(buf + rr * RB + ((cc ^ (rr % CPRW)) << 4));
            const size_t blk = (size_t)(m0 / 256) * (p.ldc / 32) + col0 / 32 + kk;
            put16((T*)p.C + blk * 8192 + trow * 32 + ln * 8, val);
          }
          return;
        }
      }
      const int c = ln % CPRW;
#pragma unroll
      for (int k = 0; k < CPRW / 4; ++k) {
        const int rr = ln / CPRW + k * (64 / CPRW);
        const u32x4_t val = *(const u32x4_t*)(buf + rr * RB + ((c ^ (rr % CPRW)) << 4));
        // Rows past M go to their own padding rows (c_padded), or else hold
        // row M-1's outputs (computed from its inputs) and are stored there
        // again: the same bytes.  Either way, no branch.
        const int m = min(m0 + wm * 128 + t * 16 + rr, mlast);
        put16((T*)p.C + (size_t)m * p.ldc + col0 + c * 8, val);
      }
    };
    if constexpr (EPI == EPI_ROPE) {
      // Every wave has read stage 0 (the next tile's first fragments).
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    if (EPI == EPI_ROPE && cbase >= p.epi.rope_cols) {
      // V columns: the STORE schedule (the same EST stores, no table loads).
      using NR = std::false_type;
      auto unit = [&](auto uc) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value;
        compute_unit(uc, NR{});
        if constexpr (u > 0) store_unit(std::integral_constant<int, u - 1>{}, NR{});
        __builtin_amdgcn_sched_barrier(0);
      };
      w4_for<NUNITS>([&](auto uc) __attribute__((always_inline)) { unit(uc); });
      store_unit(std::integral_constant<int, NUNITS - 1>{}, NR{});
    } else if constexpr (EPI == EPI_ROPE) {
      w4_for<RD>([&](auto uc) __attribute__((always_inline)) { fetch_cs(uc); });
      w4_for<6>([&](auto uc) __attribute__((always_inline)) {
        compute_unit(uc, std::true_type{});
        __builtin_amdgcn_sched_barrier(0);
      });
      store_unit(std::integral_constant<int, 0>{}, std::true_type{});
      compute_unit(std::integral_constant<int, 6>{}, std::true_type{});
      store_unit(std::integral_constant<int, 1>{}, std::true_type{});
      compute_unit(std::integral_constant<int, 7>{}, std::true_type{});
      w4_for<6>([&](auto uc) __attribute__((always_inline)) {
        store_unit(std::integral_constant<int, decltype(uc)::value + 2>{}, std::true_type{});
      });
    } else {
      auto unit = [&](auto uc) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value;
        compute_unit(uc, std::true_type{});
        if constexpr (u > 0) store_unit(std::integral_constant<int, u - 1>{}, std::true_type{});
        __builtin_amdgcn_sched_barrier(0);
      };
      w4_for<RD>([&](auto uc) __attribute__((always_inline)) { fetch_cs(uc); });
      w4_for<NUNITS>([&](auto uc) __attribute__((always_inline)) { unit(uc); });
      store_unit(std::integral_constant<int, NUNITS - 1>{}, std::true_type{});
    }
    asm volatile("" ::: "memory");
  };
  auto epilogue = [&](int ti) __attribute__((always_inline)) {
    if (EPI != EPI_ROPE && p.epi.bias) epilogue_hb(ti, std::true_type{});
    else epilogue_hb(ti, std::false_type{});
  };

  // Half tile (STORE, always a workgroup's last tile): the STORE epilogue
  // over the wave's 128 x 64 block, accumulator tiles 8f + t, f < 4.  Unit t
  // (16 rows of 128 bytes) is assembled in LDS buffer t % 2 and stored as
  // whole rows while unit t+1 is computed.
  auto epilogue_half = [&](int ti, auto hbc) __attribute__((always_inline)) {
    constexpr bool HB = decltype(hbc)::value;
    constexpr int HRB = 128, HCP = HRB / 16;
    int m0, n0, hf;
    coords(ti, m0, n0, hf);
    int ln = lane;
    asm volatile("" : "+v"(ln));
    // The last MFMAs' results must be written before they are read.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    const int r = ln & 15, g = ln >> 4;
    const int cbase = n0 + hf * 128 + wn * 64;  // the wave's first packed feature
    char* stg = lds + NS * STAGE + wave * 8192;
    const int mlast = p.epi.c_padded ? INT_MAX : p.M - 1;
    float4_t bv[4];
    if constexpr (HB) {
#pragma unroll
      for (int f = 0; f < 4; ++f) bv[f] = *(const float4_t*)(p.epi.bias + cbase + f * 16 + g * 4);
    }
    auto compute_unit = [&](auto uc) __attribute__((always_inline)) {
      constexpr int t = decltype(uc)::value;
      char* buf = stg + (t & 1) * 2048;
      auto put = [&](int col, float4_t a, float4_t b) __attribute__((always_inline)) {
        const int c = (col - cbase) >> 3;
        *(u32x4_t*)(buf + r * HRB + ((c ^ (r % HCP)) << 4)) = pack8<T>(a, b);
      };
      float4_t v[4];
      v[0] = W4Acc<0 * 8 + t>::read();
      v[1] = W4Acc<1 * 8 + t>::read();
      v[2] = W4Acc<2 * 8 + t>::read();
      v[3] = W4Acc<3 * 8 + t>::read();
      w4_epilogue_block<T, EPI, MATH, HB>(
          p, v, cbase, ln, [&](int f) { return bv[f]; },
          [&](int) { return float4_t{0.f, 0.f, 0.f, 0.f}; }, put);
    };
    auto store_unit = [&](auto uc) __attribute__((always_inline)) {
      constexpr int t = decltype(uc)::value;
      const char* buf = stg + (t & 1) * 2048;
      const int c = ln % HCP;
#pragma unroll
      for (int k = 0; k < HCP / 4; ++k) {
        const int rr = ln / HCP + k * (64 / HCP);
        const u32x4_t val = *(const u32x4_t*)(buf + rr * HRB + ((c ^ (rr % HCP)) << 4));
        const int m = min(m0 + wm * 128 + t * 16 + rr, mlast);
        *(u32x4_t*)((T*)p.C + (size_t)m * p.ldc + cbase + c * 8) = val;
      }
    };
    w4_for<8>([&](auto uc) __attribute__((always_inline)) {
      constexpr int u = decltype(uc)::value;
      compute_unit(uc);
      if constexpr (u > 0) store_unit(std::integral_constant<int, u - 1>{});
      __builtin_amdgcn_sched_barrier(0);
    });
    store_unit(std::integral_constant<int, 7>{});
    asm volatile("" ::: "memory");
  };

  // Per tile: group 0 (its first step multiplies into zero), groups 1 ..
  // G-2, and the last group, whose steps 1-3 load the next tile's steps 0-2
  // (past the last tile: its steps again, in bounds and never read).  Then
  // step 3 of the next tile goes into stage 3 (free since step 2 of this
  // group) ahead of the epilogue.
  //
  // Wait counts: every wave's memory operations complete in issue order.
  // The epilogue issues exactly EST stores (no loads once its stores start
  // but RoPE's, which only add to the count), so in the next tile step 1
  // (needing step 2) and step 2 (needing step 3) find at least EST + 8
  // operations issued after the loads they need.  Everything else waits
  // with 8 outstanding: the one step loaded since.
  constexpr int EST = EPI == EPI_SWIGLU ? 16 : 32;
  using VM8 = std::integral_constant<int, NLD>;
  using VME = std::integral_constant<int, NLD + EST>;
  using VM63 = std::integral_constant<int, 63>;
  // RoPE keeps stage 3 free for its epilogue: the next tile's first step
  // loads its step 3 itself, and its step 2 then waits for the stores.
  constexpr bool PRE3 = EPI != EPI_ROPE;
  using Z0 = std::integral_constant<int, 0>;
  using ZF = std::integral_constant<int, PRE3 ? 1 : 2>;
  using VM2 = std::conditional_t<PRE3, VME, VM8>;
  const int G4 = nk / 4;
  // Tile ti, full (hc false) or half.  Its last step reads the first
  // fragments of the next tile (rdBn, set by load_tile); with FUSE, a full
  // tile's epilogue runs the next tile's first step (a whole-width step
  // also for a half tile: the extra accumulators are never read).
  auto tile = [&](int ti, auto hc) __attribute__((always_inline)) {
    using H = decltype(hc);
    // With FUSE, every tile but the first had its first step in the
    // previous epilogue.
    if (!FUSE || ti == 0) kstep(I0{}, ZF{}, VM63{}, H{}, rdBc);
    if (ti == 0) {
      kstep(I1{}, Z0{}, VM8{}, H{}, rdBc);
      kstep(I2{}, Z0{}, VM8{}, H{}, rdBc);
    } else {
      kstep(I1{}, Z0{}, VME{}, H{}, rdBc);
      kstep(I2{}, Z0{}, VM2{}, H{}, rdBc);
    }
    kstep(I3{}, Z0{}, VM8{}, H{}, rdBc);
    for (int g = 1; g < G4 - 1; ++g) {
      kstep(I0{}, Z0{}, VM8{}, H{}, rdBc);
      kstep(I1{}, Z0{}, VM8{}, H{}, rdBc);
      kstep(I2{}, Z0{}, VM8{}, H{}, rdBc);
      kstep(I3{}, Z0{}, VM8{}, H{}, rdBc);
    }
    kstep(I0{}, Z0{}, VM8{}, H{}, rdBc);
    load_tile(ti + 1 < my_tiles ? ti + 1 : ti);
    kstep(I1{}, Z0{}, VM8{}, H{}, rdBc);
    kstep(I2{}, Z0{}, VM8{}, H{}, rdBc);
    kstep(I3{}, Z0{}, VM8{}, H{}, rdBn);
    // Steps 0 and 1 of the next tile have landed (step 1 is read in its
    // first step); step 3 goes out before the stores.
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NLD) : "memory");
    if constexpr (PRE3) load_step(3);
    if constexpr (H::value) {
      if (p.epi.bias) epilogue_half(ti, std::true_type{});
      else epilogue_half(ti, std::false_type{});
    } else {
      epilogue(ti);
    }
    rdBc = rdBn;
  };
  for (int ti = 0; ti < my_full; ++ti) tile(ti, std::false_type{});
  if constexpr (HALF) {
    if (has_half) tile(my_full, std::true_type{});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
#pragma clang diagnostic pop

// ---------------------------------------------------------------------------
// Tile configurations of the older 4-wave kernels, which take what the
// persistent four-wave kernel does not (fp32, tanh and reference-formula
// epilogues, N % 256 != 0, K % 128 != 0): 16-bit 256x128 tiles of 4 waves x
// (128x64); fp32 128x64 tiles of 2 waves.
// ---------------------------------------------------------------------------
struct Cfg256x128 { static constexpr int BM = 256, BN = 128, BK = 64, WM = 2, WN = 2; };
struct CfgF32 { static constexpr int BM = 128, BN = 64, BK = 32, WM = 2, WN = 1; };

template <typename T, typename C, int EPI, int MATH>
static hipError_t launch_lds(const GemmParams& p, hipStream_t s) {
  const int num_m = (p.M + C::BM - 1) / C::BM;
  const int num_n = p.N / C::BN;
  dim3 grid(num_m * num_n), block(C::WM * C::WN * 64);
  hipLaunchKernelGGL(
      (gemm_lds_kernel<T, C::BM, C::BN, kLdsBK, C::WM, C::WN, EPI, MATH, kLdsSwz,
                       kLdsStages>),
      grid, block, 0, s, p);
  return hipGetLastError();
}

static int cu_count() {
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!counts[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

// Epilogues the four-wave kernel is built for.  The others (tanh, the
// reference-formula GELU and SiLU) need more registers than it leaves next to
// its accumulators and take the older 4-wave kernels; so does RoPE with a
// bias.
constexpr bool w4_epilogue_ok(int epi, int math) {
  return epi == EPI_STORE || epi == EPI_ROPE ||
         (math == MATH_EXACT && (epi == EPI_SWIGLU || epi == EPI_GELU));
}

// Workgroups of a persistent launch over ntiles tiles: the fewest that take
// the same number of rounds of tiles as one per CU (a multiple of 8 where
// that stays within the CUs, for the XCD-chunked tile order).  The kernel
// takes as long as with one workgroup per CU, and the CUs it leaves free run
// other streams' work (fl_model_embed runs two batches at once).
static int persistent_grid(int ntiles) {
  const int cus = cu_count();
  if (ntiles <= 0) return 1;
  const int rounds = (ntiles + cus - 1) / cus;
  int grid = (ntiles + rounds - 1) / rounds;
  const int g8 = (grid + 7) / 8 * 8;
  if (g8 <= cus && (ntiles + g8 - 1) / g8 == rounds) grid = g8;
  return grid;
}

// ---------------------------------------------------------------------------
// Few-row form of the four-wave GEMM.  With a single 256-row block the
// four-wave kernel runs N / 256 tiles, each walking the whole K on one CU
// (FFN-down at 16 tokens: 3 workgroups, 96 K steps).  Here a workgroup owns
// one epilogue unit, 16 rows x 64 packed features: wave w multiplies feature
// block w (16 features) over the whole K with the same 16x16x32 MFMA, the
// same operand roles (weights as the first operand) and the same K order
// starting from zero, so every accumulator holds the bits the four-wave
// kernel's does; the unit then goes through the same epilogue math
// (w4_epilogue_block).  Outputs are therefore identical, and a sequence's
// vector still does not depend on the batch around it.  Fragments come
// straight from global memory (weights tiled, activations tiled or
// row-major), PF K steps ahead in registers.  Rows past M are computed from
// rows M-1 (row-major A) or the padding rows (tiled A) and not stored.
// ---------------------------------------------------------------------------
template <typename T, int EPI, int MATH, bool HB>
__global__ void __launch_bounds__(256) gemm_small_kernel(GemmParams p) {
  constexpr int PF = 16;  // K steps in flight per wave
  __shared__ float4_t accs[4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nbase = blockIdx.x * 64;      // the unit's first packed feature
  const int m0 = blockIdx.y * 16;         // the unit's first row
  const int fr = lane & 15, fg = lane >> 4;
  const int nk = p.K / 32;
  const T* W = (const T*)p.B;
  const T* A = (const T*)p.A;
  const int n = nbase + wave * 16 + fr;   // this lane's packed feature (weight row)
  const int m = m0 + fr;                  // this lane's row
  const int ma = p.epi.a_tiled ? m : min(m, p.M - 1);
  // Packed row n of the tiled weights: the tiled activation layout over K.
  auto wptr = [&](int s) __attribute__((always_inline)) {
    return (const u32x4_t*)(W + tiled_act_offset(n, s * 32 + fg * 8, p.K));
  };
  auto aptr = [&](int s) __attribute__((always_inline)) {
    const int k = s * 32 + fg * 8;
    return (const u32x4_t*)(A + (p.epi.a_tiled ? tiled_act_offset(ma, k, p.K)
                                               : (size_t)ma * p.lda + k));
  };
  u32x4_t wf[PF], af[PF];
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    const int s = min(j, nk - 1);
    wf[j] = *wptr(s);
    af[j] = *aptr(s);
  }
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  int s0 = 0;
  for (; s0 + PF <= nk; s0 += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      MfmaFrag<T>::mma(acc, wf[j], af[j]);
      // The step PF ahead (clamped: loads past the end repeat the last step
      // and are never used), issued without a branch so the waits stay exact.
      const int s = min(s0 + PF + j, nk - 1);
      wf[j] = *wptr(s);
      af[j] = *aptr(s);
    }
  }
  // The last nk % PF steps (a multiple of 4: K % 128 == 0) sit in slots
  // 0 .. nk % PF - 1.
#pragma unroll
  for (int q = 0; q < PF / 4 - 1; ++q) {
    if (s0 + 4 * q + 4 > nk) break;
#pragma unroll
    for (int j = 4 * q; j < 4 * q + 4; ++j) MfmaFrag<T>::mma(acc, wf[j], af[j]);
  }
  accs[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  float4_t v[4] = {accs[0][lane], accs[1][lane], accs[2][lane], accs[3][lane]};
  const int r = lane & 15, g = lane >> 4;
  const int row = m0 + r;
  float4_t bv[4];
  if constexpr (HB) {
#pragma unroll
    for (int f = 0; f < 4; ++f) bv[f] = *(const float4_t*)(p.epi.bias + nbase + f * 16 + g * 4);
  }
  float4_t cs[4];
  if constexpr (EPI == EPI_ROPE) {
    const float2* table = nbase < p.epi.q_cols ? p.epi.rope_cs_q : p.epi.rope_cs;
    const int pos = p.epi.pos[min(row, p.M - 1)];
    const float4_t* src = (const float4_t*)(table + (size_t)pos * 32 + g * 8);
#pragma unroll
    for (int k = 0; k < 4; ++k) cs[k] = src[k];
  }
  auto put = [&](int col, float4_t a, float4_t b) __attribute__((always_inline)) {
    if (row >= p.M) return;
    T* dst = (T*)p.C + (EPI == EPI_SWIGLU && p.epi.out_tiled ? tiled_act_offset(row, col, p.ldc)
                                                             : (size_t)row * p.ldc + col);
    *(u32x4_t*)dst = pack8<T>(a, b);
  };
  auto bias_at = [&](int f) { return bv[f]; };
  auto rope_at = [&](int k) { return cs[k]; };
  if (EPI == EPI_ROPE && nbase >= p.epi.rope_cols)
    w4_epilogue_block<T, EPI, MATH, HB, false>(p, v, nbase, lane, bias_at, rope_at, put);
  else
    w4_epilogue_block<T, EPI, MATH, HB, true>(p, v, nbase, lane, bias_at, rope_at, put);
}

// The four-wave kernel's K loop runs in groups of four steps with at least
// two groups per tile; its RoPE epilogue gives both 64-feature heads of a
// wave the same table and rotation.
static bool gemm_w4_shape_ok(int K) { return K % 128 == 0 && K >= 256; }
static bool gemm_w4_ok(const GemmParams& p) {
  if (!gemm_w4_shape_ok(p.K)) return false;
  if (p.epi.kind == EPI_ROPE && (p.epi.q_cols % 128 || p.epi.rope_cols % 128)) return false;
  return true;
}

template <typename T, int EPI, int MATH>
static hipError_t launch_w4(const GemmParams& p, hipStream_t s) {
  const int ntiles = ((p.M + 255) / 256) * (p.N / 256);
  // STORE: a partial last round on at most half the CUs runs as half tiles,
  // two per tile, on twice as many (the kernel's nhalf).  The full rounds
  // take every CU (full is a multiple of the CU count), so each workgroup
  // has the same number of full tiles and 2 * rest <= grid.
  const int cus = cu_count();
  const int rest = ntiles % cus;
  if (EPI == EPI_STORE && MATH == MATH_EXACT && kW4Half && p.K <= kW4HalfMaxK && rest > 0 &&
      2 * rest <= cus) {
    const int full = ntiles - rest;
    const int grid = full > 0 ? persistent_grid(full) : 2 * rest;
    hipLaunchKernelGGL((gemm_w4_kernel<T, EPI, MATH, 4>), dim3(grid), dim3(256), 0, s, p, full,
                       rest);
    return hipGetLastError();
  }
  const int grid = persistent_grid(ntiles);
  hipLaunchKernelGGL((gemm_w4_kernel<T, EPI, MATH, 4>), dim3(grid), dim3(256), 0, s,
                     p, ntiles, 0);
  return hipGetLastError();
}

// Whether the few-row kernel beats the four-wave kernel on this GEMM, from
// per-launch times measured on single-sequence forwards of 128-1024 tokens
// (Nomic and BERT-base projections): the four-wave kernel takes ~0.55 us per
// K step and ~10 us more per round of tiles, whatever the rows; the few-row
// kernel ~9 us plus 0.25 ns per (unit, K step) with tiled activations,
// 0.6 ns with row-major ones (16 rows x 16 bytes at the row pitch per load).
// At 512 tokens that sends FFN-down (96 K steps, 3 column tiles) and O to the
// few-row kernel and keeps FFN-up (96 units per 16 rows) on the four-wave one.
static bool gemm_small_better(const GemmParams& p) {
  if (p.M > 4096 || !p.epi.allow_small) return false;
  const double nk = p.K / 32;
  const double units = (double)((p.M + 15) / 16) * (p.N / 64);
  const double small_us = units * nk * (p.epi.a_tiled ? 0.25e-3 : 0.6e-3) + 9.0;
  const int cus = cu_count();
  const int ntiles = ((p.M + 255) / 256) * (p.N / 256);
  const double w4_us = ((ntiles + cus - 1) / cus) * (0.55 * nk + 10.0);
  return small_us < w4_us;
}

template <typename T, int EPI, int MATH>
static hipError_t launch_small(const GemmParams& p, hipStream_t s) {
  const dim3 grid(p.N / 64, (p.M + 15) / 16);
  if (EPI != EPI_ROPE && p.epi.bias)
    hipLaunchKernelGGL((gemm_small_kernel<T, EPI, MATH, true>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_small_kernel<T, EPI, MATH, false>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, typename C, int EPI, int MATH>
static hipError_t launch_cfg(const GemmParams& p, hipStream_t s) {
  const int num_m = (p.M + C::BM - 1) / C::BM;
  const int num_n = p.N / C::BN;
  dim3 grid(num_m * num_n), block(C::WM * C::WN * 64);
  hipLaunchKernelGGL((gemm_nt_kernel<T, C::BM, C::BN, C::BK, C::WM, C::WN, EPI, MATH>), grid,
                     block, 0, s, p);
  return hipGetLastError();
}

template <typename T, int EPI, int MATH>
static hipError_t launch_pick(const GemmParams& p, hipStream_t s) {
  if constexpr (sizeof(T) == 4) {
    return launch_cfg<T, CfgF32, EPI, MATH>(p, s);
  } else {
    // B packed for the four-wave kernel (gemm_w4_layout) goes there; only the
    // epilogues and shapes it was built for reach this point with such a
    // layout (gemm_nt_supported).
    if (p.epi.layout >= PACK_LANE16) {
      if constexpr (w4_epilogue_ok(EPI, MATH)) {
        if (gemm_w4_ok(p)) {
          if (gemm_small_better(p)) return launch_small<T, EPI, MATH>(p, s);
          return launch_w4<T, EPI, MATH>(p, s);
        }
      }
      return hipErrorInvalidValue;
    }
    if (p.K % (kLdsBK * kLdsStages) == 0) return launch_lds<T, Cfg256x128, EPI, MATH>(p, s);
    return launch_cfg<T, Cfg256x128, EPI, MATH>(p, s);
  }
}

template <typename T>
static hipError_t launch_typed(const GemmParams& p, hipStream_t s) {
  const bool ref = p.epi.math == MATH_REFERENCE;
  switch (p.epi.kind) {
    case EPI_STORE: return launch_pick<T, EPI_STORE, MATH_EXACT>(p, s);
    case EPI_ROPE: return launch_pick<T, EPI_ROPE, MATH_EXACT>(p, s);
    case EPI_GELU:
      return ref ? launch_pick<T, EPI_GELU, MATH_REFERENCE>(p, s)
                 : launch_pick<T, EPI_GELU, MATH_EXACT>(p, s);
    case EPI_TANH:
      return ref ? launch_pick<T, EPI_TANH, MATH_REFERENCE>(p, s)
                 : launch_pick<T, EPI_TANH, MATH_EXACT>(p, s);
    case EPI_SWIGLU:
      return ref ? launch_pick<T, EPI_SWIGLU, MATH_REFERENCE>(p, s)
                 : launch_pick<T, EPI_SWIGLU, MATH_EXACT>(p, s);
  }
  return hipErrorInvalidValue;
}

template <typename T>
static bool cfg_ok(int N, int K) {
  if constexpr (sizeof(T) == 4) return N % CfgF32::BN == 0 && K % CfgF32::BK == 0;
  else return N % Cfg256x128::BN == 0 && K % Cfg256x128::BK == 0;
}

int gemm_w4_layout(int dtype, int N, int K, int epi_kind, int math, bool has_bias) {
  if (dtype != F16 && dtype != BF16) return -1;
  if (N <= 0 || N % 256 || !gemm_w4_shape_ok(K)) return -1;
  if (!w4_epilogue_ok(epi_kind, math)) return -1;
  if (epi_kind == EPI_ROPE) return has_bias ? -1 : PACK_ROPE;
  return epi_kind == EPI_SWIGLU ? PACK_SWIGLU_LANE : PACK_LANE16;
}

int gemm_padded_width(int dtype, int N, int K, int epi_kind, int math, bool has_bias) {
  if (N <= 0 || N % 256 == 0 || epi_kind == EPI_SWIGLU || epi_kind == EPI_ROPE) return N;
  const int np = (N + 255) / 256 * 256;
  return gemm_w4_layout(dtype, np, K, epi_kind, math, has_bias) >= 0 ? np : N;
}

bool gemm_tiled_ok(int dtype, int N, int K, int epi_kind, int math, bool has_bias, bool out_tiled,
                   bool a_tiled, bool c_padded) {
  if (!out_tiled && !a_tiled && !c_padded) return true;
  if (gemm_w4_layout(dtype, N, K, epi_kind, math, has_bias) < 0) return false;
  if (out_tiled && (epi_kind != EPI_SWIGLU || (N / 2) % 32)) return false;
  return true;
}

bool gemm_nt_supported(int dtype, int M, int N, int K, const void* A, int lda, const void* B,
                       int ldb, const void* C, int ldc, const GemmEpilogue& epi) {
  if (M <= 0 || N <= 0 || K <= 0) return false;
  if (!gemm_tiled_ok(dtype, N, K, epi.kind, epi.math, epi.bias != nullptr, epi.out_tiled,
                     epi.a_tiled, epi.c_padded))
    return false;
  if (epi.layout >= PACK_LANE16) {
    if (gemm_w4_layout(dtype, N, K, epi.kind, epi.math, epi.bias != nullptr) != epi.layout)
      return false;
    if (lda % 8 || ldb % 8 || ldc % 8) return false;
    if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C | (uintptr_t)epi.bias) & 15) return false;
    // The RoPE epilogue gives both 64-feature heads of a wave the same table
    // and rotation: its column bounds are multiples of 128.
    if (epi.kind == EPI_ROPE && (epi.rope_cols % 128 || !epi.pos || !epi.rope_cs)) return false;
    if (epi.q_cols && (epi.q_cols % 64 || (epi.kind != EPI_STORE && epi.kind != EPI_ROPE)))
      return false;
    if (epi.q_cols && epi.kind == EPI_ROPE &&
        (epi.q_cols % 128 || !epi.rope_cs_q || epi.q_cols > epi.rope_cols))
      return false;
    return true;
  }
  if (epi.q_cols) return false;  // only the four-wave epilogues scale a query block
  if (epi.layout != (epi.kind == EPI_SWIGLU ? PACK_SWIGLU16 : PACK_PLAIN)) return false;
  const int esz = dtype == F32 ? 4 : 2;
  const int epc = 16 / esz;
  bool shape = dtype == F32 ? cfg_ok<float>(N, K)
                            : (dtype == F16 ? cfg_ok<_Float16>(N, K) : cfg_ok<__bf16>(N, K));
  if (!shape) return false;
  if (lda % epc || ldb % epc || ldc % 4) return false;
  if (((uintptr_t)A | (uintptr_t)B) & 15) return false;
  if ((uintptr_t)C & (4 * esz - 1)) return false;
  if ((uintptr_t)epi.bias & 15) return false;
  if (epi.kind == EPI_SWIGLU && (N % 32)) return false;
  if (epi.kind == EPI_ROPE && (epi.rope_cols % 64 || !epi.pos || !epi.rope_cs)) return false;
  return true;
}

hipError_t launch_gemm_nt(int dtype, const void* A, int lda, const void* B, int ldb, void* C,
                          int ldc, int M, int N, int K, const GemmEpilogue& epi,
                          hipStream_t stream) {
  GemmParams p{A, B, C, lda, ldb, ldc, M, N, K, epi};
  switch (dtype) {
    case F16: return launch_typed<_Float16>(p, stream);
    case BF16: return launch_typed<__bf16>(p, stream);
    case F32: return launch_typed<float>(p, stream);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Generic GEMM (any shape, transposes, alpha): 16x16 LDS tiles on the VALU.
// Used for odd shapes of the per-op API; fp32 accumulation.
// ---------------------------------------------------------------------------
template <typename T, int MATH>
__global__ void __launch_bounds__(256)
gemm_generic_kernel(int ta, int tb, int M, int N, int K, float alpha, const T* A, int lda,
                    const T* B, int ldb, T* C, int ldc, const float* bias, int act) {
  __shared__ float sa[16][17], sb[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
  float acc = 0.f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    {
      const int ar = blockIdx.y * 16 + ty, ak = k0 + tx;
      float v = 0.f;
      if (ar < M && ak < K) v = to_f(ta ? A[(size_t)ak * lda + ar] : A[(size_t)ar * lda + ak]);
      sa[ty][tx] = v;
      const int bk = k0 + ty, bc = blockIdx.x * 16 + tx;
      float w = 0.f;
      if (bk < K && bc < N) w = to_f(tb ? B[(size_t)bc * ldb + bk] : B[(size_t)bk * ldb + bc]);
      sb[ty][tx] = w;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) acc += sa[ty][kk] * sb[kk][tx];
    __syncthreads();
  }
  if (row < M && col < N) {
    float v = alpha * acc;
    if (bias) v += bias[col];
    if (act == ACT_GELU) v = gelu_m<MATH>(v);
    else if (act == ACT_TANH) v = tanh_m<MATH>(v);
    C[(size_t)row * ldc + col] = from_f<T>(v);
  }
}

template <typename T>
static hipError_t gen_typed(int ta, int tb, int M, int N, int K, float alpha, const void* A,
                            int lda, const void* B, int ldb, void* C, int ldc, const float* bias,
                            int act, int math, hipStream_t s) {
  dim3 grid((N + 15) / 16, (M + 15) / 16), block(256);
  if (math == MATH_REFERENCE)
    hipLaunchKernelGGL((gemm_generic_kernel<T, MATH_REFERENCE>), grid, block, 0, s, ta, tb, M,
                       N, K, alpha, (const T*)A, lda, (const T*)B, ldb, (T*)C, ldc, bias, act);
  else
    hipLaunchKernelGGL((gemm_generic_kernel<T, MATH_EXACT>), grid, block, 0, s, ta, tb, M, N, K,
                       alpha, (const T*)A, lda, (const T*)B, ldb, (T*)C, ldc, bias, act);
  return hipGetLastError();
}

hipError_t launch_gemm_generic(int dtype, int trans_a, int trans_b, int M, int N, int K,
                               float alpha, const void* A, int lda, const void* B, int ldb,
                               void* C, int ldc, const float* bias, int act, int math,
                               hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  switch (dtype) {
    case F32:
      return gen_typed<float>(trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, C, ldc, bias,
                              act, math, s);
    case F16:
      return gen_typed<_Float16>(trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, C, ldc, bias,
                                 act, math, s);
    case BF16:
      return gen_typed<__bf16>(trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, C, ldc, bias,
                               act, math, s);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Weight packing: out[n][k] = in[k][n]; with SwiGLU interleave the [gate|up]
// output columns are reordered into 16-column blocks g0 u0 g1 u1 ...
// Column n of the input becomes row row0 + n of a packed matrix of ntot rows
// (one part of a fused QKV matrix, or a matrix with zero padding rows).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void transpose_kernel(const T* in, int rows, int cols, T* out, int layout, int row0,
                                 int ntot) {
  __shared__ T tile[32][33];
  const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int j = ty; j < 32; j += 8) {
    const int r = by + j, c = bx + tx;
    if (r < rows && c < cols) tile[j][tx] = in[(size_t)r * cols + c];
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    const int n = bx + j, k = by + tx;  // output row n (input column), column k
    if (n < cols && k < rows) out[packed_offset(row0 + n, k, ntot, rows, layout)] = tile[tx][j];
  }
}

// Packed row n of an [N, K] matrix, one row per block of 64 threads x 16 B
// (8 elements of 16-bit types, 4 of fp32: a 16-byte chunk never straddles
// a tiled 16-byte slot).
__global__ void pack_rows_kernel(const char* in, size_t ld_bytes, int N, int K, int esz,
                                 char* out, int layout) {
  const int n = blockIdx.x;
  const char* src = in + (size_t)n * ld_bytes;
  const int epc = 16 / esz;
  for (int k = threadIdx.x * epc; k < K; k += 64 * epc)
    *(u32x4_t*)(out + packed_offset(n, k, N, K, layout) * esz) =
        *(const u32x4_t*)(src + (size_t)k * esz);
}

__global__ void pack_vec_kernel(const float* in, int N, float* out, int layout, int row0,
                                int ntot) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n < N) out[packed_row(row0 + n, ntot, layout)] = in[n];
}

hipError_t launch_pack_rows(int dtype, const void* in, int ld, int N, int K, void* out,
                            int layout, hipStream_t s) {
  const size_t esz = dtype == F32 ? 4 : 2;
  if (((uintptr_t)in | (uintptr_t)out | (ld * esz) | (K * esz)) & 15) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_rows_kernel, dim3(N), dim3(64), 0, s, (const char*)in, ld * esz, N, K,
                     (int)esz, (char*)out, layout);
  return hipGetLastError();
}

hipError_t launch_pack_vec_f32(const float* in, int N, float* out, int layout, hipStream_t s,
                               int row0, int ntot) {
  if (ntot <= 0) ntot = N;
  if (row0 < 0 || row0 + N > ntot) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_vec_kernel, dim3((N + 255) / 256), dim3(256), 0, s, in, N, out, layout,
                     row0, ntot);
  return hipGetLastError();
}

hipError_t launch_transpose(int dtype, const void* in, int rows, int cols, void* out,
                            int layout, hipStream_t s, int row0, int ntot) {
  if (ntot <= 0) ntot = cols;
  if (row0 < 0 || row0 + cols > ntot) return hipErrorInvalidValue;
  dim3 grid((cols + 31) / 32, (rows + 31) / 32), block(256);
  switch (dtype) {
    case F32:
      hipLaunchKernelGGL(transpose_kernel<float>, grid, block, 0, s, (const float*)in, rows, cols,
                         (float*)out, layout, row0, ntot);
      break;
    case F16:
      hipLaunchKernelGGL(transpose_kernel<_Float16>, grid, block, 0, s, (const _Float16*)in,
                         rows, cols, (_Float16*)out, layout, row0, ntot);
      break;
    case BF16:
      hipLaunchKernelGGL(transpose_kernel<__bf16>, grid, block, 0, s, (const __bf16*)in, rows,
                         cols, (__bf16*)out, layout, row0, ntot);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace fl
