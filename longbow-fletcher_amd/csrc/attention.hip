// attention.hip -- scaled dot-product attention for gfx950.
//
// Backs Tensor.Attention / AttentionVarLen (cpu_backend.go:662-758, 66-132)
// and the encoder's self-attention (bert.go:610-728).  Inputs are packed rows
// [T, ld] with head h in columns [h*d, (h+1)*d) (cpu_backend.go:706-718);
// sequences are given by cu_seqlens, so a uniform batch and a ragged batch
// take the same path and padding never enters the arithmetic.
//
// Flash kernel (16-bit, exact math): computed transposed, S^T = K Q^T and
// O^T = V^T P^T, so the probabilities leave the first MFMA already in the
// operand layout of the second one (no cross-lane shuffle of P).  K and V
// tiles go global -> LDS by DMA, row-major with an XOR chunk swizzle; the
// V^T operand is read with the gfx950 transposing LDS load.  A query
// column's scores of a key tile live in the 4 lanes {q, q+16, q+32, q+48};
// its row max is two permlane swaps and its row sum comes out of an extra
// MFMA against a ones operand; with Q pre-scaled, the offset by the running
// max rides in the score MFMA's accumulator, so the softmax costs one exp2,
// half a max and half a pack per score.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace fl {

struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int ld;   // row stride of q/k/v (elements)
  int ldo;  // row stride of out
  const int* cu;
  const AttnWork* work;
  float scale;
  int group;  // consecutive work items per XCD (query blocks of one sequence-head)
  // > 0: the output is stored in the tiled activation layout
  // (tiled_act_offset) with this many columns, for a GEMM that reads it as a
  // tiled operand; ldo is then unused.
  int out_tiled_cols;
};

template <typename T> struct AttnMfma;
template <> struct AttnMfma<_Float16> {
  static constexpr uint32_t kOnes = 0x3C003C00u;  // two fp16 1.0
  __device__ static inline void mma(float4_t& c, const u32x4_t& a, const u32x4_t& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                               __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float a, float b) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 h = {(_Float16)a, (_Float16)b};  // v_cvt_pk_f16_f32 (RNE)
    return __builtin_bit_cast(uint32_t, h);
  }
};
template <> struct AttnMfma<__bf16> {
  static constexpr uint32_t kOnes = 0x3F803F80u;  // two bf16 1.0
  __device__ static inline void mma(float4_t& c, const u32x4_t& a, const u32x4_t& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float a, float b) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 h = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32 (RNE)
    return __builtin_bit_cast(uint32_t, h);
  }
};

typedef __attribute__((address_space(3))) char lds_char;

// Max over the lanes {l, l^16, l^32, l^48} (v_permlane16/32_swap: each swap
// returns the value pair of a lane and its xor-16 / xor-32 partner).
__device__ inline float quad_max(float v) {
  const uint32_t x = __builtin_bit_cast(uint32_t, v);
  const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  v = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
  const uint32_t y = __builtin_bit_cast(uint32_t, v);
  const auto b = __builtin_amdgcn_permlane32_swap(y, y, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One 1 KB DMA load: 64 lanes x 16 bytes from gsrc + voff into LDS at lds_dst
// (m0); gsrc and lds_dst are wave-uniform.  The flash kernel's own code never
// uses m0.
__device__ __attribute__((always_inline)) inline void attn_dma(uint32_t lds_dst, uint32_t voff,
                                                               const void* gsrc) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2" ::"s"(lds_dst),
      "v"(voff), "s"(gsrc)
      : "memory", "m0");
}
#pragma clang diagnostic pop

// One workgroup = WAVES waves x 32 query rows of one (sequence, head); key /
// value tiles of 64 rows are double-buffered in LDS.  A tile is 64 rows of
// D * 2 bytes (CH = D / 8 chunks of 16 bytes); chunk c of row r sits at
// chunk c ^ (r % CH).  Head sizes 64 (BERT-base, Nomic) and 32 (MiniLM).
//
// Scores are kept relative to a running row maximum m in the exp2 domain:
// x = s * scale * log2(e) - m, p = exp2(x).  PRE: Q arrives multiplied by
// scale * log2(e) (the encoder's QKV epilogue does it), so the first score
// MFMA starts from the accumulator -m and produces x directly; otherwise x
// takes one FMA per score.
// The four-wave form asks for four waves per SIMD (at most 128 VGPRs): with
// only the block size to go by, the register allocator may pick 130.
template <typename T, int D, int WAVES, bool PRE>
__global__ void __launch_bounds__(WAVES * 64)
    __attribute__((amdgpu_waves_per_eu(WAVES == 4 ? 4 : 1))) attn_flash_kernel(AttnParams p) {
  static_assert(D == 32 || D == 64, "head size 32 or 64");
  constexpr int BKV = 64, NT = WAVES * 64;
  constexpr int ROWB = D * 2;           // bytes of one key / value row of a head
  constexpr int CH = D / 8;             // 16-byte chunks per row
  constexpr int DS = D / 32;            // 32-wide slices of d (score MFMA steps)
  constexpr int DT = D / 16;            // 16-wide output tiles
  constexpr int TILE = BKV * ROWB;      // bytes of one K or V tile
  constexpr int NLD = TILE / 16 / NT;   // 16-byte DMA loads per thread per tensor
  static_assert(TILE % (16 * NT) == 0, "tile/thread mismatch");
  // Rescale the running output only when a row max grows by more than
  // 2^8 in the exp2 domain; until then probabilities stay below 256.
  constexpr float kRescale = 8.0f;
  using V4 = T __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(1024))) char lds[2][2][TILE];  // [buffer][K, V]

  // The query blocks of one (sequence, head) run on one XCD and share its L2.
  const AttnWork w = p.work[xcd_group((int)blockIdx.x, (int)gridDim.x, p.group)];
  const int s0 = w.s0;
  const int L = w.len;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, g = lane >> 4;
  const int hoff = w.head * D;
  const T* Q = (const T*)p.q;
  const T* K = (const T*)p.k;
  const T* V = (const T*)p.v;

  // Q fragments: [q-tile][d-slice]; lane holds 8 consecutive d of one query.
  const int qbase = w.q0 + wave * 32;
  u32x4_t qf[2][DS];
  if constexpr (D != 64) {
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int qr = qbase + qt * 16 + lr;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        if (qr < L)
          qf[qt][ds] = *(const u32x4_t*)(Q + (size_t)(s0 + qr) * p.ld + hoff + ds * 32 + g * 8);
        else
          qf[qt][ds] = u32x4_t{0, 0, 0, 0};
      }
    }
  }

  // DMA: load j of this thread fills LDS chunk j*NT + tid, i.e. row
  // (j*NT + tid) / CH, holding global chunk (tid % CH) ^ (row % CH).  In the
  // last tile, rows past the sequence re-read its last key (their scores are
  // masked to -inf, so their probabilities are exactly 0).
  // Lane byte offsets from the sequence's first row (rows < 64 of a head, so
  // 32 bits suffice); the tile's row offset rides in the 64-bit scalar base
  // (global_load_lds with an SGPR base), so a tile's loads need no 64-bit
  // lane arithmetic.
  const size_t ldk = (size_t)p.ld;
  uint32_t voff[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int row = (j * NT + tid) / CH;
    voff[j] = (uint32_t)(((size_t)row * ldk + hoff + (((tid & (CH - 1)) ^ (row & (CH - 1))) << 3)) *
                         sizeof(T));
  }
  const char* kseq = (const char*)(K + (size_t)s0 * ldk);
  const char* vseq = (const char*)(V + (size_t)s0 * ldk);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_char*)&lds[0][0][0];
  auto issue = [&](int kv0, int buf) __attribute__((always_inline)) {
    const bool tail = kv0 + BKV > L;
    const size_t tb = (size_t)kv0 * ldk * sizeof(T);
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      uint32_t o = voff[j];
      if (tail) {
        const int row = (j * NT + tid) / CH;
        o -= (uint32_t)((size_t)max(kv0 + row - (L - 1), 0) * ldk * sizeof(T));
      }
      const uint32_t kd = lds_base + (uint32_t)((buf * 2) * TILE + (j * NT + wave * 64) * 16);
      attn_dma(kd, o, kseq + tb);
      attn_dma(kd + TILE, o, vseq + tb);
    }
  };

  // K fragment (S^T A operand): row kt*16 + lr, chunk ds*4 + g.
  int koff[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) koff[ds] = lr * ROWB + (((ds * 4 + g) ^ (lr & (CH - 1))) << 4);
  // V^T fragment (O^T A operand), transposing read: lane (g, s = lr) names
  // row 4g + s/4 (+16 for keys 16..31 of a 32-key step), bytes
  // [dt*32 + 8*(s%4), +8) of that row.
  const int vrow = 4 * g + (lr >> 2);
  const int vx = ((lr & 3) >> 1) ^ (vrow & (CH - 1));
  const int vbase = vrow * ROWB + (lr & 1) * 8;

  float4_t o[DT][2], lacc[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    lacc[qt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt][qt] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
  // Running row max m (exp2 domain); 0 until the first tile sets it.
  float ms[2] = {0.f, 0.f};
  float4_t cinit[2] = {float4_t{0.f, 0.f, 0.f, 0.f}, float4_t{0.f, 0.f, 0.f, 0.f}};
  const float c = p.scale * 1.4426950408889634f;
  const u32x4_t ones = {AttnMfma<T>::kOnes, AttnMfma<T>::kOnes, AttnMfma<T>::kOnes,
                        AttnMfma<T>::kOnes};

  // V^T fragment addresses in buffer 0, per 16-wide output tile dt; the
  // buffer and the key-row step ride in the reads' immediate offsets.
  uint32_t vaddr[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    vaddr[dt] = (uint32_t)(uintptr_t)(const lds_char*)lds[0][1] + vbase + (((dt * 2) ^ vx) << 4);

  const int ntiles = (L + BKV - 1) / BKV;
  // One key tile; CUR (the LDS buffer holding it) is a compile-time
  // constant, so every LDS address of the tile is a register plus an
  // immediate.
  auto tile = [&](int it, auto cur_c) __attribute__((always_inline)) {
    constexpr int CUR = decltype(cur_c)::value;
    const int kv0 = it * BKV;
    // The other buffer was last read in the previous iteration, which
    // ended with a barrier.
    if (it + 1 < ntiles) issue(kv0 + BKV, CUR ^ 1);
    const char* kt_lds = lds[CUR][0];

    // Relative scores x, transposed: [key-tile][q-tile]
    float4_t s[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      s[kt][0] = PRE ? cinit[0] : float4_t{0.f, 0.f, 0.f, 0.f};
      s[kt][1] = PRE ? cinit[1] : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const u32x4_t kf = *(const u32x4_t*)(kt_lds + kt * 16 * ROWB + koff[ds]);
        AttnMfma<T>::mma(s[kt][0], kf, qf[0][ds]);
        AttnMfma<T>::mma(s[kt][1], kf, qf[1][ds]);
      }
    }
    if constexpr (!PRE) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
          for (int i = 0; i < 4; ++i) s[kt][qt][i] = fmaf(s[kt][qt][i], c, -ms[qt]);
    }
    if (kv0 + BKV > L) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kv0 + kt * 16 + g * 4 + i >= L) {
            s[kt][0][i] = -INFINITY;
            s[kt][1][i] = -INFINITY;
          }
    }

    // Lazy rescale of the running output.  The first tile always sets m;
    // later tiles move it only when a row max grows past 2^8.  A row's
    // scores sit in the four lanes {l, l^16, l^32, l^48}; one of them holds a
    // score above the threshold iff the row max is above it, so the test
    // takes this lane's max alone and the cross-lane reduction runs only
    // when the wave rescales.
    float lm = fmaxf(s[0][0][0], s[0][0][1]);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kt | qt | (i >> 1)) lm = fmaxf(lm, s[kt][qt][i]);
    if (__any(it == 0 || lm > kRescale)) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        float m = fmaxf(s[0][qt][0], s[0][qt][1]);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = (kt == 0 ? 2 : 0); i < 4; ++i) m = fmaxf(m, s[kt][qt][i]);
        const float mx = quad_max(m);
        const float shift = it == 0 ? mx : fmaxf(mx, 0.f);
        ms[qt] += shift;
        cinit[qt] = float4_t{-ms[qt], -ms[qt], -ms[qt], -ms[qt]};
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) s[kt][qt] -= shift;
        if (it > 0) {
          const float alpha = __builtin_amdgcn_exp2f(-shift);
          lacc[qt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[dt][qt] *= alpha;
        }
      }
    }

    // P^T operand [key-step][q-tile]: key k of step ks is ks*32 + 4g + k
    // for k < 4 and ks*32 + 16 + 4g + k - 4 for k >= 4.
    u32x4_t pf[2][2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          s[kt][qt][i] = __builtin_amdgcn_exp2f(s[kt][qt][i]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        pf[ks][qt][0] = AttnMfma<T>::pack2(s[2 * ks][qt][0], s[2 * ks][qt][1]);
        pf[ks][qt][1] = AttnMfma<T>::pack2(s[2 * ks][qt][2], s[2 * ks][qt][3]);
        pf[ks][qt][2] = AttnMfma<T>::pack2(s[2 * ks + 1][qt][0], s[2 * ks + 1][qt][1]);
        pf[ks][qt][3] = AttnMfma<T>::pack2(s[2 * ks + 1][qt][2], s[2 * ks + 1][qt][3]);
      }
    }

    // O^T += V^T P^T; the row sums ride along as ones * P^T.  V^T
    // fragments come from the transposing LDS load ds_read_b64_tr_b16
    // (within each 16-lane block, lane i receives element i%4 of the 8-byte
    // rows addressed by lanes i/4 + 4j, j = 0..3), one 32-key step at a
    // time after the softmax: read earlier, they would be live beside the
    // scores and take the kernel past 128 VGPRs, from four waves per SIMD
    // to three.  Written as asm because the compiler cannot tell these
    // reads from the DMA into the other buffer and would wait for it.
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x2_t vr[DT][2];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        asm volatile(
            "ds_read_b64_tr_b16 %0, %2 offset:%3\n"
            "ds_read_b64_tr_b16 %1, %2 offset:%4\n"
            : "=&v"(vr[dt][0]), "=&v"(vr[dt][1])
            : "v"(vaddr[dt]), "n"(CUR * 2 * TILE + ks * 32 * ROWB),
              "n"(CUR * 2 * TILE + (ks * 32 + 16) * ROWB));
      }
      AttnMfma<T>::mma(lacc[0], ones, pf[ks][0]);
      AttnMfma<T>::mma(lacc[1], ones, pf[ks][1]);
      if constexpr (DT == 4) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(vr[0][0]), "+v"(vr[0][1]), "+v"(vr[1][0]), "+v"(vr[1][1]),
                       "+v"(vr[2][0]), "+v"(vr[2][1]), "+v"(vr[3][0]), "+v"(vr[3][1]));
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(vr[0][0]), "+v"(vr[0][1]), "+v"(vr[1][0]), "+v"(vr[1][1]));
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const u32x2_t lo = vr[dt][0], hi = vr[dt][1];
        const u32x4_t vf = {lo[0], lo[1], hi[0], hi[1]};
        AttnMfma<T>::mma(o[dt][0], vf, pf[ks][0]);
        AttnMfma<T>::mma(o[dt][1], vf, pf[ks][1]);
      }
    }

    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };

  // Head size 64: the wave's 32 Q rows come by DMA as whole 128-byte rows
  // into the four 1 KB blocks of buffer 1 that its own loads of tile 1 fill
  // later (K and V blocks wave and 4 + wave), chunk c of row r at slot
  // c ^ (r % 8); rows past the sequence re-read its last row.
  const lds_char* qlds[4] = {(const lds_char*)lds[1][0] + wave * 1024,
                             (const lds_char*)lds[1][0] + (4 + wave) * 1024,
                             (const lds_char*)lds[1][1] + wave * 1024,
                             (const lds_char*)lds[1][1] + (4 + wave) * 1024};
  if constexpr (D == 64) {
    const char* qseq = (const char*)(Q + (size_t)s0 * ldk);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = i * 8 + (lane >> 3);
      const int qr = min(qbase + row, L - 1);
      const uint32_t qo =
          (uint32_t)(((size_t)qr * ldk + hoff + (((lane & 7) ^ (row & 7)) << 3)) * sizeof(T));
      attn_dma((uint32_t)(uintptr_t)qlds[i], qo, qseq);
    }
  }
  issue(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (D == 64) {
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int row = qt * 16 + lr;
      const lds_char* rb = qlds[2 * qt + (lr >> 3)] + (row & 7) * 128;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        qf[qt][ds] = *(const __attribute__((address_space(3))) u32x4_t*)(
            rb + ((((ds * 4 + g) ^ (row & 7))) << 4));
    }
  }
  __syncthreads();
  for (int it = 0; it < ntiles; it += 2) {
    tile(it, std::integral_constant<int, 0>{});
    if (it + 1 < ntiles) tile(it + 1, std::integral_constant<int, 1>{});
  }

  // The output goes through LDS, each wave's 32 rows in an area of its own
  // (every wave has passed the last tile's barrier, so the K/V buffers are
  // free), to leave as 16-byte stores of whole rows instead of 8-byte pieces
  // of 16 rows.  Chunk c of row r sits at chunk c ^ (r % CH).
  T* out = (T*)p.out;
  char* ost = &lds[0][0][0] + wave * 32 * ROWB;
  // An opaque copy of the lane id keeps the stores' address arithmetic from
  // being hoisted into the key loop, where it would hold registers.
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int olr = ln & 15, og = ln >> 4;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float inv = 1.0f / lacc[qt][0];
    const int row = qt * 16 + olr;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      V4 h;
#pragma unroll
      for (int i = 0; i < 4; ++i) h[i] = (T)(o[dt][qt][i] * inv);
      const int c = dt * 2 + (og >> 1);
      *(V4*)(ost + row * ROWB + ((c ^ (row & (CH - 1))) << 4) + (og & 1) * 8) = h;
    }
  }
  if (p.out_tiled_cols > 0) {
    // Tiled output: the 16-row halves of each 32-column slice of the head
    // are contiguous 1 KB blocks (rows of one 256-row tile); lane l writes
    // 16-byte chunk l % 4 of row l / 4.
#pragma unroll
    for (int sl = 0; sl < D / 32; ++sl)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int row = j * 16 + (ln >> 2), c = sl * 4 + (ln & 3);
        const u32x4_t val =
            *(const u32x4_t*)(ost + row * ROWB + ((c ^ (row & (CH - 1))) << 4));
        const int qr = qbase + row;
        if (qr < L)
          *(u32x4_t*)(out + tiled_act_offset(s0 + qr, hoff + c * 8, p.out_tiled_cols)) = val;
      }
    return;
  }
  constexpr int RPR = 64 / CH;  // rows per 64 lanes x 16 bytes
#pragma unroll
  for (int k = 0; k < 32 / RPR; ++k) {
    const int row = k * RPR + ln / CH, c = ln % CH;
    const u32x4_t val = *(const u32x4_t*)(ost + row * ROWB + ((c ^ (row & (CH - 1))) << 4));
    const int qr = qbase + row;
    if (qr < L) *(u32x4_t*)(out + (size_t)(s0 + qr) * p.ldo + hoff + c * 8) = val;
  }
}

template <typename T>
static void launch_flash_typed(const AttnParams& p, int n_work, int head_dim, int waves,
                               bool prescaled, hipStream_t stream) {
  const dim3 grid(n_work);
  if (head_dim == 32) {
    // Only the unscaled form: the encoder pre-scales Q for head size 64 only.
    if (waves == 2) hipLaunchKernelGGL((attn_flash_kernel<T, 32, 2, false>), grid, dim3(128), 0, stream, p);
    else hipLaunchKernelGGL((attn_flash_kernel<T, 32, 4, false>), grid, dim3(256), 0, stream, p);
  } else if (waves == 2) {
    if (prescaled) hipLaunchKernelGGL((attn_flash_kernel<T, 64, 2, true>), grid, dim3(128), 0, stream, p);
    else hipLaunchKernelGGL((attn_flash_kernel<T, 64, 2, false>), grid, dim3(128), 0, stream, p);
  } else {
    if (prescaled) hipLaunchKernelGGL((attn_flash_kernel<T, 64, 4, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((attn_flash_kernel<T, 64, 4, false>), grid, dim3(256), 0, stream, p);
  }
}

hipError_t launch_attention_flash(int dtype, const void* q, const void* k, const void* v,
                                  int ldqkv, void* out, int ldo, const int* cu_seqlens,
                                  const AttnWork* work, int n_work, int head_dim, float scale,
                                  int waves, bool q_prescaled, int xcd_group_size,
                                  hipStream_t stream, int out_tiled_cols) {
  if (n_work <= 0) return hipSuccess;
  if (out_tiled_cols && (out_tiled_cols % 32 || head_dim != 64)) return hipErrorInvalidValue;
  if ((head_dim != 32 && head_dim != 64) || (head_dim == 32 && q_prescaled))
    return hipErrorInvalidValue;
  const AttnParams p{q, k, v, out, ldqkv, ldo, cu_seqlens, work, scale,
                     std::max(1, std::min(xcd_group_size, 32)), out_tiled_cols};
  if (dtype == F16) launch_flash_typed<_Float16>(p, n_work, head_dim, waves, q_prescaled, stream);
  else if (dtype == BF16) launch_flash_typed<__bf16>(p, n_work, head_dim, waves, q_prescaled, stream);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fp32 two-pass attention (head_dim 64).  Pass 1 finds the exact row max of
// scale*QK^T; pass 2 evaluates ExpFast(score - max) (MATH_REFERENCE, the
// reference's SoftmaxFast, simd.go:78-100) or exp, accumulates P V with fp32
// MFMA and divides by the sum.  An online rescale cannot reproduce ExpFast,
// whose products are not exponentials of sums, hence the second pass.
// Workgroup = 4 waves x 16 queries; key tiles of 32 rows.
// ---------------------------------------------------------------------------
template <int MATH>
__global__ void __launch_bounds__(256) attn_f32_kernel(AttnParams p) {
  constexpr int D = 64, BKV = 32, S = D + 4;
  __shared__ __attribute__((aligned(16))) float Ks[BKV * S];
  __shared__ __attribute__((aligned(16))) float Vs[BKV * S];

  const AttnWork w = p.work[blockIdx.x];
  const int s0 = w.s0;
  const int L = w.len;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int hoff = w.head * D;
  const float* Q = (const float*)p.q;
  const float* K = (const float*)p.k;
  const float* V = (const float*)p.v;
  const float scale = p.scale;

  const int qr = w.q0 + wave * 16 + lrow;
  // Chunk dc covers d in [16*dc, 16*dc+16); lane group g holds d = 16*dc + 4g + j.
  float4_t qf[4];
#pragma unroll
  for (int dc = 0; dc < 4; ++dc) {
    if (qr < L)
      qf[dc] = *(const float4_t*)(Q + (size_t)(s0 + qr) * p.ld + hoff + dc * 16 + lgrp * 4);
    else
      qf[dc] = float4_t{0.f, 0.f, 0.f, 0.f};
  }

  auto load_tile = [&](int kv0, bool with_v) {
    for (int c = tid; c < BKV * D / 4; c += 256) {
      const int row = c >> 4, col = (c & 15) * 4;
      const int key = kv0 + row;
      u32x4_t kk = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
      if (key < L) {
        const size_t off = (size_t)(s0 + key) * p.ld + hoff + col;
        kk = *(const u32x4_t*)(K + off);
        if (with_v) vv = *(const u32x4_t*)(V + off);
      }
      *(u32x4_t*)(&Ks[row * S + col]) = kk;
      if (with_v) *(u32x4_t*)(&Vs[row * S + col]) = vv;
    }
  };
  auto scores = [&](float4_t (&s)[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dc = 0; dc < 4; ++dc) {
        const float4_t kf = *(const float4_t*)(&Ks[(kt * 16 + lrow) * S + dc * 16 + lgrp * 4]);
        s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[0], qf[dc][0], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[1], qf[dc][1], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[2], qf[dc][2], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[3], qf[dc][3], s[kt], 0, 0, 0);
      }
    }
  };

  const int ntiles = (L + BKV - 1) / BKV;
  // Pass 1: exact row max of the scaled scores.
  float mx = -INFINITY;
  for (int it = 0; it < ntiles; ++it) {
    const int kv0 = it * BKV;
    load_tile(kv0, false);
    __syncthreads();
    float4_t s[2];
    scores(s);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (kv0 + kt * 16 + lgrp * 4 + i < L) mx = fmaxf(mx, mul_rn(s[kt][i], scale));
    __syncthreads();
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));

  // Pass 2: probabilities and P V.
  float4_t o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
  for (int it = 0; it < ntiles; ++it) {
    const int kv0 = it * BKV;
    load_tile(kv0, true);
    __syncthreads();
    float4_t s[2];
    scores(s);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float e = 0.f;
        if (kv0 + kt * 16 + lgrp * 4 + i < L) {
          const float sc = mul_rn(s[kt][i], scale);
          if constexpr (MATH == MATH_REFERENCE) e = exp_fast_ref(sc - mx);
          else e = expf(sc - mx);
        }
        s[kt][i] = e;
        lsum += e;
      }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float vv = Vs[(kt * 16 + lgrp * 4 + j) * S + dt * 16 + lrow];
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv, s[kt][j], o[dt], 0, 0, 0);
        }
    __syncthreads();
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  const float inv = 1.0f / lsum;
  if (qr < L) {
    float* orow = (float*)p.out + (size_t)(s0 + qr) * p.ldo + hoff + lgrp * 4;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      float4_t r = o[dt] * inv;
      *(float4_t*)(orow + dt * 16) = r;
    }
  }
}

hipError_t launch_attention_f32(const float* q, const float* k, const float* v, int ldqkv,
                                float* out, int ldo, const int* cu_seqlens,
                                const AttnWork* work, int n_work, float scale, int math,
                                hipStream_t stream) {
  if (n_work <= 0) return hipSuccess;
  AttnParams p{q, k, v, out, ldqkv, ldo, cu_seqlens, work, scale, 1};
  if (math == MATH_REFERENCE)
    hipLaunchKernelGGL(attn_f32_kernel<MATH_REFERENCE>, dim3(n_work), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(attn_f32_kernel<MATH_EXACT>, dim3(n_work), dim3(256), 0, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Generic attention: one thread per (sequence, head, query row), any
// head_dim <= 256; three sweeps over the keys (max, sum, weighted V).
// ---------------------------------------------------------------------------
template <typename T, int MATH>
__global__ void __launch_bounds__(128)
attn_generic_kernel(const T* q, const T* k, const T* v, int ld, T* out, int ldo, const int* cu,
                    int max_len, int heads, int hd, float scale) {
  const int seq = blockIdx.y, h = blockIdx.z;
  const int qi = blockIdx.x * blockDim.x + threadIdx.x;
  const int s0 = cu[seq], L = cu[seq + 1] - s0;
  if (qi >= L) return;
  (void)max_len;
  (void)heads;
  const T* qrow = q + (size_t)(s0 + qi) * ld + h * hd;
  float mx = -INFINITY;
  for (int j = 0; j < L; ++j) {
    const T* krow = k + (size_t)(s0 + j) * ld + h * hd;
    float acc = 0.f;
    for (int d = 0; d < hd; ++d) acc += to_f(qrow[d]) * to_f(krow[d]);
    mx = fmaxf(mx, mul_rn(acc, scale));
  }
  float sum = 0.f;
  for (int j = 0; j < L; ++j) {
    const T* krow = k + (size_t)(s0 + j) * ld + h * hd;
    float acc = 0.f;
    for (int d = 0; d < hd; ++d) acc += to_f(qrow[d]) * to_f(krow[d]);
    const float sc = mul_rn(acc, scale);
    sum += MATH == MATH_REFERENCE ? exp_fast_ref(sc - mx) : expf(sc - mx);
  }
  const float inv = 1.0f / sum;
  T* orow = out + (size_t)(s0 + qi) * ldo + h * hd;
  for (int d0 = 0; d0 < hd; d0 += 32) {
    float o[32];
    const int dn = min(32, hd - d0);
    for (int d = 0; d < 32; ++d) o[d] = 0.f;
    for (int j = 0; j < L; ++j) {
      const T* krow = k + (size_t)(s0 + j) * ld + h * hd;
      const T* vrow = v + (size_t)(s0 + j) * ld + h * hd;
      float acc = 0.f;
      for (int d = 0; d < hd; ++d) acc += to_f(qrow[d]) * to_f(krow[d]);
      const float sc = mul_rn(acc, scale);
      const float pr = (MATH == MATH_REFERENCE ? exp_fast_ref(sc - mx) : expf(sc - mx)) * inv;
      for (int d = 0; d < dn; ++d) o[d] += pr * to_f(vrow[d0 + d]);
    }
    for (int d = 0; d < dn; ++d) orow[d0 + d] = from_f<T>(o[d]);
  }
}

template <typename T>
static hipError_t gen_typed(const void* q, const void* k, const void* v, int ld, void* out,
                            int ldo, const int* cu, int nseq, int max_len, int heads, int hd,
                            float scale, int math, hipStream_t s) {
  dim3 grid((max_len + 127) / 128, nseq, heads), block(128);
  if (math == MATH_REFERENCE)
    hipLaunchKernelGGL((attn_generic_kernel<T, MATH_REFERENCE>), grid, block, 0, s, (const T*)q,
                       (const T*)k, (const T*)v, ld, (T*)out, ldo, cu, max_len, heads, hd,
                       scale);
  else
    hipLaunchKernelGGL((attn_generic_kernel<T, MATH_EXACT>), grid, block, 0, s, (const T*)q,
                       (const T*)k, (const T*)v, ld, (T*)out, ldo, cu, max_len, heads, hd,
                       scale);
  return hipGetLastError();
}

hipError_t launch_attention_generic(int dtype, const void* q, const void* k, const void* v,
                                    int ldqkv, void* out, int ldo, const int* cu_seqlens,
                                    int nseq, int max_len, int heads, int head_dim, float scale,
                                    int math, hipStream_t stream) {
  if (nseq <= 0 || max_len <= 0) return hipSuccess;
  switch (dtype) {
    case F32:
      return gen_typed<float>(q, k, v, ldqkv, out, ldo, cu_seqlens, nseq, max_len, heads,
                              head_dim, scale, math, stream);
    case F16:
      return gen_typed<_Float16>(q, k, v, ldqkv, out, ldo, cu_seqlens, nseq, max_len, heads,
                                 head_dim, scale, math, stream);
    case BF16:
      return gen_typed<__bf16>(q, k, v, ldqkv, out, ldo, cu_seqlens, nseq, max_len, heads,
                               head_dim, scale, math, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace fl
