// model.cpp -- model-level encoder forward (BertModel.ForwardBatch,
// internal/embeddings/model/bert.go:149-169) on gfx950.
//
// Per layer (bert.go:364-384, 610-824):
//   QKV   = X Wqkv^T + b        one GEMM, N = 3H, RoPE fused in the epilogue
//   CTX   = attention(Q, K, V)  flash (16-bit) / two-pass (fp32), varlen
//   TMP   = CTX Wo^T + bo
//   X     = LN(X + TMP)         residual.AddLayerNorm (cpu_backend.go:603-610)
//   G     = act(X Wi^T + bi)    GELU or SwiGLU fused in the epilogue
//   TMP   = G Wd^T + bd
//   X     = LN(X + TMP)
// then masked mean-pool (+L2) or the CLS tanh pooler.
//
// Weights arrive in the reference layout ([in, out], Y = X W) and are packed
// once: transposed to [out, in] so both GEMM operands stream along K,
// Q|K|V concatenated, SwiGLU gate/up interleaved in 16-column blocks.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "context.hpp"
#include "kernels.hpp"


namespace fl {

struct LayerW {
  void* wqkv = nullptr;  // [Nqkv, H] (rows past 3H zero)
  float* bqkv = nullptr; // [Nqkv]
  void* wo = nullptr;    // [Nh, H]
  float* bo = nullptr;
  float* ln1_g = nullptr;
  float* ln1_b = nullptr;
  void* wi = nullptr;    // [Ni, H] (SwiGLU interleaved)
  float* bi = nullptr;   // [Ni] (same order)
  void* wd = nullptr;    // [Nh, I]
  float* bd = nullptr;
  float* ln2_g = nullptr;
  float* ln2_b = nullptr;
};

enum ProfClass { P_EMBED = 0, P_QKV, P_ATTN, P_O, P_LN, P_UP, P_DOWN, P_POOL };

// Pinned host staging of a batch's metadata (attention work list,
// cu_seqlens, positions), two slots per lane used in turn so a batch's upload
// never waits for the previous batch's kernels: a slot is refilled only after
// its copy (event) has completed.
struct Staging {
  void* host = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
};

// Everything one batch's forward reads and writes besides the weights: the
// activation buffers, the batch metadata and the stream the forward runs on.
// Lane 0 runs on the context stream and serves every entry point; the
// batching loop of fl_model_embed also uses lanes 1 .. kLanes-1, each on a
// stream of its own, so consecutive forwards run concurrently and one
// forward's kernels fill the CUs the others' leave idle.  Three lanes (three
// of the four hardware queues a process gets) measured best with
// 16384-token forwards: two left the device idle while the host prepared the
// next forward, four gained nothing.
// Lanes of fl_model_embed's batch pipeline (lane 0 is the context stream's).
constexpr int kLanes = 3;
// Synchronous forwards of up to this many tokens (fl_model_forward[_ex],
// fl_model_forward_padded) replay a HIP graph of their kernels, captured the
// first time a lengths vector is seen; at most kGraphCache graphs are kept
// (least recently used dropped).  A short forward is ~86 kernels of a few
// microseconds each, so launch overhead is a large share of it.
constexpr int64_t kGraphTokens = 4096;
constexpr size_t kGraphCache = 16;

// fl_model_embed computes consecutive batches of its plan together, in
// forwards of up to this many tokens (a batch larger than that alone).  A
// sequence's vector does not depend on the other sequences of its forward,
// so the grouping changes no output bit; it only gives the GEMMs more rows:
// 16384-token forwards leave the N = 768 GEMMs 192 tiles for 256 CUs.
// Measured end to end (the whole call, PCIe included) against one forward per
// batch of the reference's 16384-token plan: config 3 +8%, the ragged batch
// +9%, BERT-base +4%; one 131072-token forward is no faster than two of
// 65536 tokens on two lanes.
constexpr int64_t kGroupTokens = 65536;

struct Lane {
  hipStream_t stream = nullptr;
  // activations (capacity in tokens / sequences)
  int64_t cap_tokens = 0;
  int cap_seq = 0;
  size_t cap_work = 0;
  size_t cap_part = 0;
  void* X = nullptr;
  void* QKV = nullptr;  // also holds the FFN intermediate
  void* CTX = nullptr;
  void* TMP = nullptr;
  void* G2 = nullptr;   // [T, 2I] unfused SwiGLU product (only without the fused epilogue)
  int* ids32 = nullptr;
  int* pos32 = nullptr;
  int* cu = nullptr;
  AttnWork* work = nullptr;
  float* part = nullptr;
  float* cls = nullptr;
  float* out = nullptr;
  uint16_t* out16 = nullptr;  // fp16 copy of `out` (FL_F16 output)
  int* flags = nullptr;       // [0] NaN in pooled output, [1] id out of range
  Staging meta[2];
  int meta_slot = 0;
  std::vector<int64_t> last_lengths;
  int64_t T = 0;
  int n_work = 0, max_len = 0, waves = 4;
  int qblocks = 1;  // query blocks of the longest sequence (flash work items per head)
  const float2* rope_cs = nullptr;
  const float2* rope_cs_q = nullptr;  // rope_cs * scale * log2(e), for a pre-scaled Q
};

}  // namespace fl

using namespace fl;

struct fl_model {
  fl_context* ctx = nullptr;
  fl_model_config cfg{};
  int H = 0, I = 0, Ni = 0, heads = 0, hd = 0, dtype = 0;
  // Output widths of the QKV projection and of the two H-wide projections
  // (O, FFN-down): 3H and H, or padded to whole 256-column tiles for the
  // four-wave GEMM (gemm_padded_width); QKV and TMP have these row strides.
  int Nqkv = 0, Nh = 0;
  size_t esz = 2;
  bool swiglu = false, rope = false;
  bool mfma_qkv = false, mfma_o = false, mfma_up = false, mfma_down = false;
  bool rope_fused = false;
  // PackLayout of each projection's packed weights and bias.
  int lay_qkv = PACK_PLAIN, lay_o = PACK_PLAIN, lay_up = PACK_PLAIN, lay_down = PACK_PLAIN;

  void* word = nullptr;
  void* pos = nullptr;
  void* type = nullptr;
  float* emb_g = nullptr;
  float* emb_b = nullptr;
  std::vector<LayerW> layers;
  float* pool_w = nullptr;  // fp32 [H, H] reference layout
  float* pool_b = nullptr;
  std::unordered_map<void*, size_t> owned;  // device buffers and their sizes

  // Lane 0: the context stream; lanes 1 .. kLanes-1: fl_model_embed's own.
  Lane lane[kLanes];

  // fl_model_embed's pipeline: one slot per lane; a lane's stream carries
  // its forward's id upload, the forward and the copies back.
  struct Pipe {
    int32_t* ids_pin[kLanes] = {};
    float* out_pin[kLanes] = {};
    int* flags_pin[kLanes] = {};
    int* rows_pin[kLanes] = {};   // per-sequence NaN/Inf flags of the forward's output
    int* ids_dev[kLanes] = {};
    float* out_dev[kLanes] = {};
    uint16_t* out16_dev[kLanes] = {};  // fp16 output of the forward (FL_F16)
    int* flags_dev[kLanes] = {};
    int* rows_dev[kLanes] = {};
    hipEvent_t d2h[kLanes] = {};
    bool ready = false;  // streams and events created
    int64_t cap_tok = 0;
    int cap_seq = 0;
  } pipe;

  bool q_prescaled = false;   // QKV epilogue multiplies Q by scale * log2(e) for the flash kernel
  // The SwiGLU output (FFN-down's activations) is kept in the tiled layout
  // (tiled_act_offset), so FFN-down streams it in contiguous 16 KB blocks.
  bool ffn_tiled = false;
  // The residual stream X (LayerNorm outputs, the QKV and FFN-up
  // activations) is kept tiled too; activation buffers then have rows up to
  // a multiple of 256 and the GEMMs reading X write their padding rows.
  bool x_tiled = false;
  // The attention output CTX (the O projection's activations) is kept tiled
  // as well, so the O projection streams it in contiguous 16 KB blocks.
  bool ctx_tiled = false;

  // The lane whose activations hold the most recent forward (fl_model_last_hidden).
  int last_lane = 0;

  // Captured forwards of lane 0 (kGraphTokens): the launches bake in the
  // lane's buffer and table addresses, so an entry is used only while they
  // are unchanged.
  struct FwdGraph {
    std::vector<int64_t> lengths;
    std::vector<const void*> addrs;
    hipGraphExec_t exec = nullptr;
    uint64_t used = 0;
  };
  std::vector<FwdGraph> graphs;
  uint64_t graph_clock = 0;
  bool graphs_on = true;

  bool prof = false;
  std::vector<hipEvent_t> ev_pool;
  size_t ev_next = 0;
  std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending;
  double prof_ms[FL_PROF_CLASSES] = {0};
  int64_t prof_cnt[FL_PROF_CLASSES] = {0};
};

namespace {

constexpr float kLog2e = 1.4426950408889634f;
// Attention scale 1/float32(sqrt(d)) (bert.go:643).
float attn_scale(int hd) { return 1.0f / (float)std::sqrt((double)hd); }

// A model-owned device buffer: counted in the context's allocated bytes and
// freed with the model.
template <typename P>
int track_alloc(fl_model* m, size_t bytes, P*& out) {
  void* p = nullptr;
  out = nullptr;
  int st = device_alloc(m->ctx, bytes, &p);
  if (st) return st;
  m->owned[p] = bytes;
  out = (P*)p;
  return FL_OK;
}

// Frees a buffer from track_alloc and clears the pointer, so that a failed
// reallocation never leaves a freed buffer in use.
template <typename P>
void untrack_free(fl_model* m, P*& p) {
  if (!p) return;
  auto it = m->owned.find((void*)p);
  size_t bytes = 0;
  if (it != m->owned.end()) {
    bytes = it->second;
    m->owned.erase(it);
  }
  device_free(m->ctx, (void*)p, bytes);
  p = nullptr;
}

void free_owned(fl_model* m) {
  for (auto& kv : m->owned) device_free(m->ctx, kv.first, kv.second);
  m->owned.clear();
}

#define M_CHECK(expr)                                  \
  do {                                                 \
    hipError_t _e = (expr);                            \
    if (_e != hipSuccess) return hip_fail(_e, #expr);  \
  } while (0)

#define M_ST(expr)        \
  do {                    \
    int _s = (expr);      \
    if (_s) return _s;    \
  } while (0)

hipEvent_t next_event(fl_model* m) {
  if (m->ev_next == m->ev_pool.size()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    m->ev_pool.push_back(e);
  }
  return m->ev_pool[m->ev_next++];
}

// Kernel timing of lane 0's forwards (the context stream).
struct ProfScope {
  fl_model* m;
  int cls;
  hipEvent_t a = nullptr;
  ProfScope(fl_model* mm, const Lane& L, int c) : m(mm), cls(c) {
    if (m->prof && L.stream == m->ctx->stream) {
      a = next_event(m);
      if (a) (void)hipEventRecord(a, m->ctx->stream);
    }
  }
  ~ProfScope() {
    if (a) {
      hipEvent_t b = next_event(m);
      if (b) {
        (void)hipEventRecord(b, m->ctx->stream);
        m->pending.push_back({cls, {a, b}});
      }
    }
  }
};

int collect_profile(fl_model* m) {
  if (m->pending.empty()) return FL_OK;
  M_CHECK(hipStreamSynchronize(m->ctx->stream));
  for (auto& p : m->pending) {
    float ms = 0.f;
    M_CHECK(hipEventElapsedTime(&ms, p.second.first, p.second.second));
    m->prof_ms[p.first] += ms;
    m->prof_cnt[p.first] += 1;
  }
  m->pending.clear();
  m->ev_next = 0;
  return FL_OK;
}

bool mfma_shape_ok(int dtype, int N, int K) {
  GemmEpilogue e;
  // Alignment of model-owned buffers is guaranteed; check the shape only.
  static const char dummy[64] __attribute__((aligned(256))) = {0};
  return gemm_nt_supported(dtype, 1, N, K, dummy, K, dummy, K, dummy, N, e);
}

// Grows the activation buffers.  Capacities drop to 0 and old buffers are
// freed (pointers cleared) before anything is allocated, so an allocation
// that fails leaves a model whose next call reallocates from scratch.
int ensure_capacity(fl_model* m, Lane& L, int64_t T, int nseq, size_t nwork, size_t part_elems) {
  if (T > L.cap_tokens) {
    M_CHECK(hipStreamSynchronize(L.stream));
    L.cap_tokens = 0;
    L.last_lengths.clear();
    untrack_free(m, L.X);
    untrack_free(m, L.QKV);
    untrack_free(m, L.CTX);
    untrack_free(m, L.TMP);
    untrack_free(m, L.G2);
    untrack_free(m, L.ids32);
    untrack_free(m, L.pos32);
    // Rows rounded up to whole 256-row tiles (tiled activations, padded GEMM outputs).
    int64_t cap = (std::max<int64_t>(T, 256) + 255) / 256 * 256;
    const int64_t wide = std::max<int64_t>(m->Nqkv, m->Ni);
    M_ST(track_alloc(m, (size_t)cap * m->H * m->esz, L.X));
    M_ST(track_alloc(m, (size_t)cap * wide * m->esz, L.QKV));
    M_ST(track_alloc(m, (size_t)cap * m->H * m->esz, L.CTX));
    M_ST(track_alloc(m, (size_t)cap * m->Nh * m->esz, L.TMP));
    if (m->swiglu && !m->mfma_up) M_ST(track_alloc(m, (size_t)cap * m->Ni * m->esz, L.G2));
    M_ST(track_alloc(m, (size_t)cap * 4, L.ids32));
    M_ST(track_alloc(m, (size_t)cap * 4, L.pos32));
    L.cap_tokens = cap;
  }
  if (nseq > L.cap_seq) {
    M_CHECK(hipStreamSynchronize(L.stream));
    L.cap_seq = 0;
    L.last_lengths.clear();
    untrack_free(m, L.cu);
    untrack_free(m, L.cls);
    untrack_free(m, L.out);
    untrack_free(m, L.out16);
    const int cap = std::max(nseq, 64);
    M_ST(track_alloc(m, (size_t)(cap + 1) * 4, L.cu));
    M_ST(track_alloc(m, (size_t)cap * m->H * 4, L.cls));
    M_ST(track_alloc(m, (size_t)cap * m->H * 4, L.out));
    M_ST(track_alloc(m, (size_t)cap * m->H * 2, L.out16));
    L.cap_seq = cap;
  }
  if (nwork > L.cap_work) {
    M_CHECK(hipStreamSynchronize(L.stream));
    L.cap_work = 0;
    L.last_lengths.clear();
    untrack_free(m, L.work);
    M_ST(track_alloc(m, nwork * sizeof(AttnWork), L.work));
    L.cap_work = nwork;
  }
  if (part_elems > L.cap_part) {
    M_CHECK(hipStreamSynchronize(L.stream));
    L.cap_part = 0;
    untrack_free(m, L.part);
    M_ST(track_alloc(m, part_elems * 4, L.part));
    L.cap_part = part_elems;
  }
  return FL_OK;
}

// Frees a lane's activation buffers (the lane reallocates them on its next use).
void release_activations(fl_model* m, Lane& L) {
  if (L.stream) (void)hipStreamSynchronize(L.stream);
  L.cap_tokens = 0;
  L.last_lengths.clear();
  untrack_free(m, L.X);
  untrack_free(m, L.QKV);
  untrack_free(m, L.CTX);
  untrack_free(m, L.TMP);
  untrack_free(m, L.G2);
  untrack_free(m, L.ids32);
  untrack_free(m, L.pos32);
}

constexpr int kPoolRows = 64;

// Uploads cu_seqlens, per-token positions and the attention work list when
// the batch's lengths differ from the previous call.
int prepare(fl_model* m, Lane& L, const int64_t* lengths, int nseq) {
  int64_t T = 0;
  int max_len = 0;
  for (int b = 0; b < nseq; ++b) {
    if (lengths[b] <= 0) return fail(FL_ERR_INVALID, "sequence lengths must be positive");
    T += lengths[b];
    max_len = std::max<int>(max_len, (int)lengths[b]);
  }
  if (T >= (int64_t)1 << 31) return fail(FL_ERR_INVALID, "too many tokens");
  // Flash kernels: 16-bit head sizes 32 and 64; fp32 head size 64.
  const bool fast_attn = m->hd == 64 || (m->hd == 32 && m->dtype != FL_F32);
  const int waves = max_len > 64 ? 4 : 2;
  const int bq = m->dtype == FL_F32 ? 64 : waves * 32;
  size_t nwork = 0;
  if (fast_attn)
    for (int b = 0; b < nseq; ++b) nwork += (size_t)m->heads * ((lengths[b] + bq - 1) / bq);
  const size_t part = (size_t)nseq * ((max_len + kPoolRows - 1) / kPoolRows) * m->H;
  M_ST(ensure_capacity(m, L, T, nseq, std::max<size_t>(nwork, 1), part));

  const bool same = (int)L.last_lengths.size() == nseq &&
                    std::equal(L.last_lengths.begin(), L.last_lengths.end(), lengths);
  if (!same) {
    // Layout of a staging slot: work list (16-byte entries) | cu | pos.
    const size_t need = nwork * sizeof(AttnWork) + (size_t)(nseq + 1) * 4 + (size_t)T * 4;
    Staging& sg = L.meta[L.meta_slot];
    L.meta_slot ^= 1;
    if (sg.pending) {
      M_CHECK(hipEventSynchronize(sg.done));
      sg.pending = false;
    }
    if (!sg.done) M_CHECK(hipEventCreateWithFlags(&sg.done, hipEventDisableTiming));
    if (sg.cap < need) {
      if (sg.host) M_CHECK(hipHostFree(sg.host));
      sg.host = nullptr;
      sg.cap = 0;
      const size_t cap = (need + (1 << 20) - 1) & ~(size_t)((1 << 20) - 1);
      if (hipHostMalloc(&sg.host, cap, hipHostMallocDefault) != hipSuccess || !sg.host)
        return fail(FL_ERR_OOM, "hipHostMalloc(batch metadata)");
      sg.cap = cap;
    }
    AttnWork* work = (AttnWork*)sg.host;
    int* cu = (int*)(work + nwork);
    int* pos = cu + nseq + 1;
    cu[0] = 0;
    for (int b = 0; b < nseq; ++b) {
      cu[b + 1] = cu[b] + (int)lengths[b];
      for (int i = 0; i < (int)lengths[b]; ++i) {
        // bert.go:223-234: absolute positions restart per sequence and clamp
        // at MaxPositionEmbeddings-1; RoPE uses the in-sequence index.
        pos[cu[b] + i] = m->rope ? i : std::min(i, m->cfg.max_pos - 1);
      }
    }
    size_t n_work = 0;
    if (fast_attn) {
      std::vector<int> order(nseq);
      for (int b = 0; b < nseq; ++b) order[b] = b;
      std::stable_sort(order.begin(), order.end(),
                       [&](int a, int b) { return lengths[a] > lengths[b]; });
      for (int b : order)
        for (int h = 0; h < m->heads; ++h)
          for (int q0 = 0; q0 < (int)lengths[b]; q0 += bq) work[n_work++] = AttnWork{cu[b], (int)lengths[b], h, q0};
    }
    if (m->rope) {
      int st;
      L.rope_cs = rope_table(m->ctx, m->cfg.rope_base, m->hd / 2, max_len, &st);
      if (st) return st;
      if (m->q_prescaled) {
        L.rope_cs_q = rope_table(m->ctx, m->cfg.rope_base, m->hd / 2, max_len, &st,
                                  attn_scale(m->hd) * kLog2e);
        if (st) return st;
      }
    }
    // Stream-ordered after the previous batch's kernels, which read the same
    // device buffers.
    hipStream_t s = L.stream;
    M_CHECK(hipMemcpyAsync(L.cu, cu, (nseq + 1) * 4, hipMemcpyHostToDevice, s));
    M_CHECK(hipMemcpyAsync(L.pos32, pos, (size_t)T * 4, hipMemcpyHostToDevice, s));
    if (n_work)
      M_CHECK(hipMemcpyAsync(L.work, work, n_work * sizeof(AttnWork), hipMemcpyHostToDevice, s));
    M_CHECK(hipEventRecord(sg.done, s));
    sg.pending = true;
    L.last_lengths.assign(lengths, lengths + nseq);
    L.n_work = (int)n_work;
    L.waves = waves;
    L.qblocks = (max_len + bq - 1) / bq;
  }
  L.T = T;
  L.max_len = max_len;
  return FL_OK;
}

int gemm(fl_model* m, const Lane& L, bool mfma, const void* A, const void* W, void* C, int M,
         int N, int K, const GemmEpilogue& epi) {
  hipStream_t s = L.stream;
  if (mfma) {
    M_CHECK(launch_gemm_nt(m->dtype, A, K, W, K, C, epi.kind == EPI_SWIGLU ? N / 2 : N, M, N, K,
                           epi, s));
    return FL_OK;
  }
  int act = epi.kind == EPI_GELU ? FL_ACT_GELU : (epi.kind == EPI_TANH ? FL_ACT_TANH : FL_ACT_IDENTITY);
  M_CHECK(launch_gemm_generic(m->dtype, 0, 1, M, N, K, 1.0f, A, K, W, K, C, N, epi.bias, act,
                              epi.math, s));
  return FL_OK;
}

// The forward on device-resident ids (L.ids32 or caller memory) into d_out, on L's stream.
int run(fl_model* m, Lane& L, const int* d_ids, int nseq, float* d_out, int* flags) {
  hipStream_t s = L.stream;
  m->last_lane = (int)(&L - m->lane);
  const int64_t T = L.T;
  const int H = m->H, dt = m->dtype;
  const int Ti = (int)T;
  M_CHECK(launch_fill_i32(flags, 2, 0, s));
  {
    ProfScope ps(m, L, P_EMBED);
    M_CHECK(launch_embed_ln(dt, d_ids, m->rope ? nullptr : L.pos32, m->word,
                            m->rope ? nullptr : m->pos, m->type, Ti, H, m->emb_g, m->emb_b,
                            m->cfg.ln_eps, m->cfg.vocab_size, flags + 1, L.X, s,
                            m->x_tiled));
  }
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const LayerW& w = m->layers[l];
    {
      ProfScope ps(m, L, P_QKV);
      GemmEpilogue e;
      e.bias = m->cfg.has_bias ? w.bqkv : nullptr;
      e.layout = m->lay_qkv;
      if (m->rope && m->rope_fused) {
        e.kind = EPI_ROPE;
        e.rope_cs = L.rope_cs;
        e.pos = L.pos32;
        e.rope_cols = 2 * H;
      }
      if (m->q_prescaled) {
        e.q_cols = H;
        e.q_scale = attn_scale(m->hd) * kLog2e;
        e.rope_cs_q = L.rope_cs_q;
      }
      e.a_tiled = e.c_padded = m->x_tiled;
      M_ST(gemm(m, L, m->mfma_qkv, L.X, w.wqkv, L.QKV, Ti, m->Nqkv, H, e));
      if (m->rope && !m->rope_fused)
        M_CHECK(launch_rope(dt, L.QKV, Ti, 2 * m->heads, m->hd, m->Nqkv, L.pos32, L.rope_cs, s));
    }
    {
      ProfScope ps(m, L, P_ATTN);
      const float scale = attn_scale(m->hd);
      const char* q = (const char*)L.QKV;
      const void* k = q + (size_t)H * m->esz;
      const void* v = q + (size_t)2 * H * m->esz;
      // XCD groups of two (sequence, head) pairs' query blocks: measured 2%
      // faster than one pair at 512 tokens (the kernel clamps groups at 32).
      if ((m->hd == 64 || m->hd == 32) && dt != FL_F32)
        M_CHECK(launch_attention_flash(dt, q, k, v, m->Nqkv, L.CTX, H, L.cu, L.work, L.n_work,
                                       m->hd, scale, L.waves, m->q_prescaled, 2 * L.qblocks, s,
                                       m->ctx_tiled ? H : 0));
      else if (m->hd == 64)
        M_CHECK(launch_attention_f32((const float*)q, (const float*)k, (const float*)v, m->Nqkv,
                                     (float*)L.CTX, H, L.cu, L.work, L.n_work, scale,
                                     m->cfg.math, s));
      else
        M_CHECK(launch_attention_generic(dt, q, k, v, m->Nqkv, L.CTX, H, L.cu, nseq, L.max_len,
                                         m->heads, m->hd, scale, m->cfg.math, s));
    }
    {
      ProfScope ps(m, L, P_O);
      GemmEpilogue e;
      e.bias = m->cfg.has_bias ? w.bo : nullptr;
      e.layout = m->lay_o;
      // A tiled CTX has rows up to the next 256 that the attention never
      // writes: O writes their (meaningless) outputs to TMP's own padding rows.
      e.a_tiled = e.c_padded = m->ctx_tiled;
      M_ST(gemm(m, L, m->mfma_o, L.CTX, w.wo, L.TMP, Ti, m->Nh, H, e));
    }
    {
      ProfScope ps(m, L, P_LN);
      M_CHECK(launch_layernorm(dt, L.X, L.TMP, Ti, H, w.ln1_g, w.ln1_b, m->cfg.ln_eps, s,
                               m->x_tiled, m->Nh));
    }
    {
      ProfScope ps(m, L, P_UP);
      GemmEpilogue e;
      e.bias = m->cfg.has_bias ? w.bi : nullptr;
      e.math = m->cfg.math;
      e.layout = m->lay_up;
      if (m->swiglu) {
        if (m->mfma_up) {
          e.kind = EPI_SWIGLU;
          e.out_tiled = m->ffn_tiled;
          e.a_tiled = m->x_tiled;
          // FFN-down reads this output tiled; without x_tiled it does not
          // write its own padding rows (c_padded), so those rows of the
          // output must be copies of row T-1, which only the four-wave
          // kernel writes.
          e.allow_small = !(m->ffn_tiled && !m->x_tiled);
          M_ST(gemm(m, L, true, L.X, w.wi, L.QKV, Ti, m->Ni, H, e));
        } else {
          // Unfused: [T, 2I] product, then silu(gate) * up into QKV.
          M_ST(gemm(m, L, false, L.X, w.wi, L.G2, Ti, m->Ni, H, e));
          M_CHECK(launch_swiglu(dt, L.G2, Ti, m->I, L.QKV, m->cfg.math, s));
        }
      } else {
        e.kind = EPI_GELU;
        M_ST(gemm(m, L, m->mfma_up, L.X, w.wi, L.QKV, Ti, m->Ni, H, e));
      }
    }
    {
      ProfScope ps(m, L, P_DOWN);
      GemmEpilogue e;
      e.bias = m->cfg.has_bias ? w.bd : nullptr;
      e.layout = m->lay_down;
      e.a_tiled = m->ffn_tiled;
      // With X tiled, the SwiGLU output's padding rows come from X's padding
      // rows (no copies of row T-1): FFN-down writes its own padding rows.
      e.c_padded = m->x_tiled;
      M_ST(gemm(m, L, m->mfma_down, L.QKV, w.wd, L.TMP, Ti, m->Nh, m->I, e));
    }
    {
      ProfScope ps(m, L, P_LN);
      M_CHECK(launch_layernorm(dt, L.X, L.TMP, Ti, H, w.ln2_g, w.ln2_b, m->cfg.ln_eps, s,
                               m->x_tiled, m->Nh));
    }
  }
  {
    ProfScope ps(m, L, P_POOL);
    if (m->cfg.pool == FL_POOL_CLS_TANH) {
      // BertPooler (bert.go:441-488) in fp32 (bert.go:459-476 forces fp32 for fp16 weights).
      M_CHECK(launch_gather_cls(dt, L.X, H, L.cu, nseq, L.cls, s, m->x_tiled));
      M_CHECK(launch_gemm_generic(FL_F32, 0, 0, nseq, H, H, 1.0f, L.cls, H, m->pool_w, H, d_out,
                                  H, m->pool_b, FL_ACT_TANH, m->cfg.math, s));
      M_CHECK(launch_has_nan(d_out, FL_F32, (int64_t)nseq * H, flags, s));
    } else {
      M_CHECK(launch_mean_pool_staged(dt, L.X, H, L.cu, nseq, L.max_len,
                                      m->cfg.pool == FL_POOL_MEAN_L2, L.part, d_out, flags,
                                      kPoolRows, s, m->x_tiled));
    }
  }
  return FL_OK;
}

// Every device address run() bakes into lane L's launches.
std::vector<const void*> lane_addrs(const fl_model* m, const Lane& L) {
  return {L.X,     L.QKV,  L.CTX,  L.TMP,  L.G2,      L.ids32,     L.pos32, L.cu,
          L.work,  L.part, L.cls,  L.out,  L.flags,   L.rope_cs,   L.rope_cs_q,
          m->ctx->stream};
}

// Destroys every captured forward.
void drop_graphs(fl_model* m) {
  for (auto& g : m->graphs)
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
  m->graphs.clear();
}

// Lane 0 runs on the context stream (looked up at every entry: the context
// owns it).
Lane& lane0(fl_model* m) {
  m->lane[0].stream = m->ctx->stream;
  return m->lane[0];
}

void free_staging(Staging& sg) {
  if (sg.pending && sg.done) (void)hipEventSynchronize(sg.done);
  if (sg.host) (void)hipHostFree(sg.host);
  if (sg.done) (void)hipEventDestroy(sg.done);
  sg = Staging{};
}

}  // namespace

const fl_model_config* fl::model_config(const fl_model* m) { return &m->cfg; }

extern "C" {

int fl_model_create(fl_context* ctx, const fl_model_config* cfg, fl_model** out) {
  if (!ctx || !cfg || !out) return fail(FL_ERR_INVALID, "null argument");
  std::lock_guard<std::recursive_mutex> lk(ctx->mu);
  M_ST(activate(ctx));
  *out = nullptr;
  const fl_model_config& c = *cfg;
  if (c.hidden <= 0 || c.layers < 0 || c.heads <= 0 || c.hidden % c.heads || c.intermediate <= 0 ||
      c.vocab_size <= 0 || c.max_pos <= 0)
    return fail(FL_ERR_INVALID, "bad model shape");
  if (c.activation != FL_ACT_GELU && c.activation != FL_ACT_SWIGLU)
    return fail(FL_ERR_UNSUPPORTED, "intermediate activation must be GELU or SwiGLU");
  if (c.position != FL_POS_ABSOLUTE && c.position != FL_POS_ROPE)
    return fail(FL_ERR_INVALID, "bad position type");
  if (c.dtype != FL_F32 && c.dtype != FL_F16 && c.dtype != FL_BF16)
    return fail(FL_ERR_INVALID, "bad dtype");
  if (c.pool < FL_POOL_CLS_TANH || c.pool > FL_POOL_MEAN_L2) return fail(FL_ERR_INVALID, "bad pool");
  if ((c.hidden / c.heads) % 2 && c.position == FL_POS_ROPE)
    return fail(FL_ERR_INVALID, "RoPE needs an even head size");
  auto* m = new fl_model();
  m->ctx = ctx;
  m->cfg = c;
  m->H = c.hidden;
  m->I = c.intermediate;
  m->swiglu = c.activation == FL_ACT_SWIGLU;
  m->Ni = m->swiglu ? 2 * m->I : m->I;
  m->heads = c.heads;
  m->hd = c.hidden / c.heads;
  m->dtype = c.dtype;
  m->esz = dtype_size(c.dtype);
  m->rope = c.position == FL_POS_ROPE;
  {
    // Widths that are not whole 256-column tiles (MiniLM's 384 and 1152) run
    // padded: zero weight rows up to the next tile, outputs with that row
    // stride.  RoPE QKV projections stay unpadded (their epilogue rotates
    // fixed column ranges).
    const bool has_bias = c.has_bias != 0;
    m->Nqkv = m->rope ? 3 * m->H
                      : gemm_padded_width(m->dtype, 3 * m->H, m->H, EPI_STORE, c.math, has_bias);
    m->Nh = gemm_padded_width(m->dtype, m->H, m->H, EPI_STORE, c.math, has_bias);
    if (gemm_padded_width(m->dtype, m->H, m->I, EPI_STORE, c.math, has_bias) != m->Nh)
      m->Nh = m->H;
  }
  m->mfma_qkv = mfma_shape_ok(m->dtype, m->Nqkv, m->H);
  m->mfma_o = mfma_shape_ok(m->dtype, m->Nh, m->H);
  m->mfma_up = mfma_shape_ok(m->dtype, m->Ni, m->H) && (!m->swiglu || m->I % 16 == 0);
  m->mfma_down = mfma_shape_ok(m->dtype, m->Nh, m->I);
  m->rope_fused = m->mfma_qkv && m->hd == 64;
  {
    const bool has_bias = c.has_bias != 0;
    auto pick = [&](bool mfma, int N, int K, int kind, int fallback) {
      if (!mfma) return (int)PACK_PLAIN;
      const int l = gemm_w4_layout(m->dtype, N, K, kind, c.math, has_bias);
      return l >= 0 ? l : fallback;
    };
    m->lay_qkv = pick(m->mfma_qkv, m->Nqkv, m->H,
                      m->rope && m->rope_fused ? EPI_ROPE : EPI_STORE, PACK_PLAIN);
    m->lay_o = pick(m->mfma_o, m->Nh, m->H, EPI_STORE, PACK_PLAIN);
    m->lay_up = m->swiglu ? pick(m->mfma_up, m->Ni, m->H, EPI_SWIGLU, PACK_SWIGLU16)
                          : pick(m->mfma_up, m->Ni, m->H, EPI_GELU, PACK_PLAIN);
    if (m->swiglu && !m->mfma_up) m->lay_up = PACK_PLAIN;
    m->lay_down = pick(m->mfma_down, m->Nh, m->I, EPI_STORE, PACK_PLAIN);
    // The flash kernel takes Q pre-scaled when the QKV projection runs on the
    // four-wave kernel, whose epilogue applies the scale.
    m->q_prescaled = m->hd == 64 && m->dtype != FL_F32 && m->lay_qkv >= PACK_LANE16 &&
                     m->H % 64 == 0;
    m->ffn_tiled = m->swiglu && m->lay_up == PACK_SWIGLU_LANE && m->lay_down >= PACK_LANE16 &&
                   gemm_tiled_ok(m->dtype, m->Ni, m->H, EPI_SWIGLU, c.math, has_bias, true, false,
                                 false) &&
                   gemm_tiled_ok(m->dtype, m->H, m->I, EPI_STORE, c.math, has_bias, false, true,
                                 true);
    const int qkv_kind = m->rope && m->rope_fused ? EPI_ROPE : EPI_STORE;
    m->x_tiled = m->ffn_tiled && m->lay_qkv >= PACK_LANE16 && m->H % 256 == 0 && m->H <= 1024 &&
                 gemm_tiled_ok(m->dtype, m->Nqkv, m->H, qkv_kind, c.math, has_bias, false, true,
                               true) &&
                 gemm_tiled_ok(m->dtype, m->Ni, m->H, EPI_SWIGLU, c.math, has_bias, true, true,
                               false);
    // The flash kernel writes CTX tiled for head size 64 (the 16-bit path).
    m->ctx_tiled = m->x_tiled && m->hd == 64 && m->mfma_o && m->lay_o >= PACK_LANE16 &&
                   gemm_tiled_ok(m->dtype, m->Nh, m->H, EPI_STORE, c.math, has_bias, false, true,
                                 true);
  }

  auto fill_f32 = [&](float** dst, size_t n, float v) -> int {
    M_ST(track_alloc(m, n * 4, *dst));
    std::vector<float> h(n, v);
    M_CHECK(hipMemcpy(*dst, h.data(), n * 4, hipMemcpyHostToDevice));
    return FL_OK;
  };
  auto zeros = [&](void** dst, size_t bytes) -> int {
    M_ST(track_alloc(m, bytes, *dst));
    M_CHECK(hipMemset(*dst, 0, bytes));
    return FL_OK;
  };
  int st = FL_OK;
  const size_t H = m->H, I = m->I, Ni = m->Ni;
  do {
    if ((st = zeros(&m->word, (size_t)c.vocab_size * H * m->esz))) break;
    if (!m->rope && (st = zeros(&m->pos, (size_t)c.max_pos * H * m->esz))) break;
    if ((st = zeros(&m->type, 2 * H * m->esz))) break;
    // NewLayerNorm (bert.go:271-283): gamma = 1, beta = 0.
    if ((st = fill_f32(&m->emb_g, H, 1.f)) || (st = fill_f32(&m->emb_b, H, 0.f))) break;
    m->layers.resize(c.layers);
    for (auto& L : m->layers) {
      const size_t Nq = m->Nqkv, Nh = m->Nh;
      if ((st = zeros(&L.wqkv, Nq * H * m->esz)) || (st = fill_f32(&L.bqkv, Nq, 0.f)) ||
          (st = zeros(&L.wo, Nh * H * m->esz)) || (st = fill_f32(&L.bo, Nh, 0.f)) ||
          (st = fill_f32(&L.ln1_g, H, 1.f)) || (st = fill_f32(&L.ln1_b, H, 0.f)) ||
          (st = zeros(&L.wi, Ni * H * m->esz)) || (st = fill_f32(&L.bi, Ni, 0.f)) ||
          (st = zeros(&L.wd, Nh * I * m->esz)) || (st = fill_f32(&L.bd, Nh, 0.f)) ||
          (st = fill_f32(&L.ln2_g, H, 1.f)) || (st = fill_f32(&L.ln2_b, H, 0.f)))
        break;
    }
    if (st) break;
    if ((st = fill_f32(&m->pool_w, H * H, 0.f)) || (st = fill_f32(&m->pool_b, H, 0.f))) break;
    void* f;
    if ((st = zeros(&f, 256))) break;
    m->lane[0].flags = (int*)f;
  } while (0);
  if (st) {
    free_owned(m);
    delete m;
    return st;
  }
  *out = m;
  return FL_OK;
}

int fl_model_free(fl_model* m) {
  if (!m) return FL_OK;
  {
    std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
    (void)activate(m->ctx);
    (void)hipStreamSynchronize(m->ctx->stream);
    fl_model::Pipe& P = m->pipe;
    for (int k = 1; k < kLanes; ++k)
      if (m->lane[k].stream) (void)hipStreamSynchronize(m->lane[k].stream);
    for (int k = 0; k < kLanes; ++k) {
      for (void* h : {(void*)P.ids_pin[k], (void*)P.out_pin[k], (void*)P.flags_pin[k],
                      (void*)P.rows_pin[k]})
        if (h) (void)hipHostFree(h);
      if (P.d2h[k]) (void)hipEventDestroy(P.d2h[k]);
    }
    for (Lane& L : m->lane)
      for (Staging& sg : L.meta) free_staging(sg);
    for (int k = 1; k < kLanes; ++k)
      if (m->lane[k].stream) (void)hipStreamDestroy(m->lane[k].stream);
    drop_graphs(m);
    free_owned(m);
    for (hipEvent_t e : m->ev_pool) (void)hipEventDestroy(e);
  }
  delete m;
  return FL_OK;
}

int fl_model_set_weight(fl_model* m, const char* name, const float* data, int64_t n) {
  if (!m || !name || (!data && n)) return fail(FL_ERR_INVALID, "null argument");
  fl_context* ctx = m->ctx;
  std::lock_guard<std::recursive_mutex> lk(ctx->mu);
  M_ST(activate(ctx));
  std::string nm(name), field = nm;
  int layer = -1;
  const size_t dot = nm.find('.');
  if (dot != std::string::npos) {
    field = nm.substr(0, dot);
    char* end = nullptr;
    layer = (int)std::strtol(nm.c_str() + dot + 1, &end, 10);
    if (!end || *end || layer < 0 || layer >= (int)m->layers.size())
      return fail(FL_ERR_INVALID, "bad layer index in weight name: " + nm);
  }
  const int64_t H = m->H, I = m->I, Ni = m->Ni, V = m->cfg.vocab_size;
  hipStream_t s = ctx->stream;
  const int dt = m->dtype;
  const bool per_layer = layer >= 0;
  auto expect = [&](int64_t want) -> int {
    if (n != want)
      return fail(FL_ERR_INVALID, "weight " + nm + ": expected " + std::to_string(want) +
                                      " values, got " + std::to_string(n));
    return FL_OK;
  };
  // Host fp32 -> scratch: [fp32 copy][dtype copy]
  int st;
  char* ws = (char*)workspace(ctx, ((size_t)n * 4 + 255) / 256 * 256 + (size_t)n * 4, &st);
  if (st) return st;
  float* f32 = (float*)ws;
  void* cvt = ws + ((size_t)n * 4 + 255) / 256 * 256;
  M_CHECK(hipMemcpyAsync(f32, data, (size_t)n * 4, hipMemcpyHostToDevice, s));
  auto to_dtype = [&](void* dst) -> int {
    M_CHECK(launch_cast(f32, FL_F32, dst, dt, n, 0, s));
    return FL_OK;
  };
  auto copy_f32 = [&](float* dst) -> int {
    M_CHECK(hipMemcpyAsync(dst, f32, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
    return FL_OK;
  };
  // [in, out] reference matrix -> rows [row0, row0 + out) of a packed
  // [ntot, in] matrix (optionally SwiGLU interleaved).
  auto pack = [&](void* dst, int rows, int cols, int layout, int row0, int ntot) -> int {
    M_CHECK(launch_cast(f32, FL_F32, cvt, dt, n, 0, s));
    M_CHECK(launch_transpose(dt, cvt, rows, cols, dst, layout, s, row0, ntot));
    return FL_OK;
  };
  // fp32 bias vector in the packed row order of its weights.
  auto pack_bias = [&](float* dst, int N, int layout, int row0, int ntot) -> int {
    M_CHECK(launch_pack_vec_f32(f32, N, dst, layout, s, row0, ntot));
    return FL_OK;
  };
  if (!per_layer) {
    if (field == "word_emb") { M_ST(expect(V * H)); M_ST(to_dtype(m->word)); }
    else if (field == "pos_emb") {
      M_ST(expect((int64_t)m->cfg.max_pos * H));
      if (m->pos) M_ST(to_dtype(m->pos));  // unused by RoPE models (bert.go:222)
    }
    else if (field == "type_emb") { M_ST(expect(2 * H)); M_ST(to_dtype(m->type)); }
    else if (field == "emb_ln_g") { M_ST(expect(H)); M_ST(copy_f32(m->emb_g)); }
    else if (field == "emb_ln_b") { M_ST(expect(H)); M_ST(copy_f32(m->emb_b)); }
    else if (field == "pool_w") { M_ST(expect(H * H)); M_ST(copy_f32(m->pool_w)); }
    else if (field == "pool_b") { M_ST(expect(H)); M_ST(copy_f32(m->pool_b)); }
    else return fail(FL_ERR_INVALID, "unknown weight " + nm);
  } else {
    LayerW& L = m->layers[layer];
    // A model created without biases (Nomic) never reads them: a projection
    // bias that is not zero is refused, as the weight-file loaders do.
    const bool proj_bias = field == "q_b" || field == "k_b" || field == "v_b" ||
                           field == "o_b" || field == "inter_b" || field == "out_b";
    if (proj_bias && !m->cfg.has_bias)
      for (int64_t i = 0; i < n; ++i)
        if (data[i] != 0.0f)
          return fail(FL_ERR_INVALID, "weight " + nm + ": the model was created without biases");
    if (field == "q_w" || field == "k_w" || field == "v_w") {
      M_ST(expect(H * H));
      const int part = field[0] == 'q' ? 0 : (field[0] == 'k' ? 1 : 2);
      // Rows [part * H, part * H + H) of the packed [Nqkv, H] matrix.
      M_ST(pack(L.wqkv, (int)H, (int)H, m->lay_qkv, part * (int)H, m->Nqkv));
    } else if (field == "q_b" || field == "k_b" || field == "v_b") {
      M_ST(expect(H));
      const int part = field[0] == 'q' ? 0 : (field[0] == 'k' ? 1 : 2);
      M_ST(pack_bias(L.bqkv, (int)H, m->lay_qkv, part * (int)H, m->Nqkv));
    } else if (field == "o_w") {
      M_ST(expect(H * H));
      M_ST(pack(L.wo, (int)H, (int)H, m->lay_o, 0, m->Nh));
    } else if (field == "o_b") { M_ST(expect(H)); M_ST(pack_bias(L.bo, (int)H, m->lay_o, 0, m->Nh)); }
    else if (field == "attn_ln_g") { M_ST(expect(H)); M_ST(copy_f32(L.ln1_g)); }
    else if (field == "attn_ln_b") { M_ST(expect(H)); M_ST(copy_f32(L.ln1_b)); }
    else if (field == "inter_w") {
      M_ST(expect(H * Ni));
      M_ST(pack(L.wi, (int)H, (int)Ni, m->lay_up, 0, (int)Ni));
    } else if (field == "inter_b") {
      M_ST(expect(Ni));
      M_ST(pack_bias(L.bi, (int)Ni, m->lay_up, 0, (int)Ni));
    } else if (field == "out_w") {
      M_ST(expect(I * H));
      M_ST(pack(L.wd, (int)I, (int)H, m->lay_down, 0, m->Nh));
    } else if (field == "out_b") {
      M_ST(expect(H));
      M_ST(pack_bias(L.bd, (int)H, m->lay_down, 0, m->Nh));
    }
    else if (field == "out_ln_g") { M_ST(expect(H)); M_ST(copy_f32(L.ln2_g)); }
    else if (field == "out_ln_b") { M_ST(expect(H)); M_ST(copy_f32(L.ln2_b)); }
    else return fail(FL_ERR_INVALID, "unknown weight " + nm);
  }
  M_CHECK(hipStreamSynchronize(s));
  return FL_OK;
}

// The pooled output leaves the device as fp32 or, for FL_F16, converted on
// the device with round-to-nearest-even (processOutput's Cast(Float16) and
// ExtractBytes, embeddings.go:256-286), half the bytes over PCIe.
static bool valid_out_dtype(int dt) { return dt == FL_F32 || dt == FL_F16; }

// run() on lane 0 through the graph cache (kGraphTokens).
static int run_graphed(fl_model* m, Lane& L, const int64_t* lengths, int nseq) {
  hipStream_t s = L.stream;
  if (!m->graphs_on || m->prof || L.T > kGraphTokens) return run(m, L, L.ids32, nseq, L.out, L.flags);
  std::vector<const void*> addrs = lane_addrs(m, L);
  fl_model::FwdGraph* hit = nullptr;
  for (auto& g : m->graphs)
    if ((int)g.lengths.size() == nseq && std::equal(g.lengths.begin(), g.lengths.end(), lengths) &&
        g.addrs == addrs) {
      hit = &g;
      break;
    }
  if (!hit) {
    M_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const int st = run(m, L, L.ids32, nseq, L.out, L.flags);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &graph);
    if (st || e != hipSuccess) {
      if (graph) (void)hipGraphDestroy(graph);
      if (st) return st;
      return hip_fail(e, "hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ie != hipSuccess) return hip_fail(ie, "hipGraphInstantiate");
    if (m->graphs.size() >= kGraphCache) {
      auto lru = std::min_element(m->graphs.begin(), m->graphs.end(),
                                  [](const auto& a, const auto& b) { return a.used < b.used; });
      (void)hipGraphExecDestroy(lru->exec);
      m->graphs.erase(lru);
    }
    m->graphs.push_back({std::vector<int64_t>(lengths, lengths + nseq), std::move(addrs), exec, 0});
    hit = &m->graphs.back();
  }
  hit->used = ++m->graph_clock;
  m->last_lane = 0;
  M_CHECK(hipGraphLaunch(hit->exec, s));
  return FL_OK;
}

static int forward_common(fl_model* m, const int64_t* ids, const int64_t* lengths, int nseq,
                          int out_dtype, void* out) {
  if (nseq <= 0) return FL_OK;
  Lane& L = lane0(m);
  M_ST(prepare(m, L, lengths, nseq));
  const int64_t T = L.T;
  std::vector<int> i32((size_t)T);
  for (int64_t t = 0; t < T; ++t) {
    // cpu_backend.go:500-502: out-of-range ids are an error.
    if (ids[t] < 0 || ids[t] >= m->cfg.vocab_size)
      return fail(FL_ERR_INVALID, "Gather index out of bounds");
    i32[t] = (int)ids[t];
  }
  hipStream_t s = m->ctx->stream;
  M_CHECK(hipMemcpyAsync(L.ids32, i32.data(), (size_t)T * 4, hipMemcpyHostToDevice, s));
  M_ST(run_graphed(m, L, lengths, nseq));
  const size_t n = (size_t)nseq * m->H;
  if (out_dtype == FL_F16) {
    M_CHECK(launch_cast(L.out, FL_F32, L.out16, FL_F16, (int64_t)n, 0, s));
    M_CHECK(hipMemcpyAsync(out, L.out16, n * 2, hipMemcpyDeviceToHost, s));
  } else {
    M_CHECK(hipMemcpyAsync(out, L.out, n * 4, hipMemcpyDeviceToHost, s));
  }
  M_CHECK(hipStreamSynchronize(s));
  return FL_OK;
}

int fl_model_forward_ex(fl_model* m, const int64_t* ids, const int64_t* lengths, int nseq,
                        int out_dtype, void* out) {
  if (!m || (nseq > 0 && (!ids || !lengths || !out))) return fail(FL_ERR_INVALID, "null argument");
  if (nseq < 0) return fail(FL_ERR_INVALID, "negative batch");
  if (!valid_out_dtype(out_dtype)) return fail(FL_ERR_INVALID, "output dtype must be F32 or F16");
  std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
  M_ST(activate(m->ctx));
  return forward_common(m, ids, lengths, nseq, out_dtype, out);
}

int fl_model_forward(fl_model* m, const int64_t* ids, const int64_t* lengths, int nseq,
                     float* out) {
  return fl_model_forward_ex(m, ids, lengths, nseq, FL_F32, out);
}

int fl_model_forward_padded(fl_model* m, const int64_t* ids, const int64_t* mask, int nseq,
                            int max_len, float* out) {
  if (!m || (nseq > 0 && (!ids || !mask || !out))) return fail(FL_ERR_INVALID, "null argument");
  if (nseq < 0 || max_len <= 0) return fail(FL_ERR_INVALID, "bad padded shape");
  std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
  M_ST(activate(m->ctx));
  std::vector<int64_t> packed, lengths(nseq);
  packed.reserve((size_t)nseq * max_len);
  for (int b = 0; b < nseq; ++b) {
    int64_t L = 0;
    bool ended = false;
    for (int t = 0; t < max_len; ++t) {
      const int64_t mk = mask[(size_t)b * max_len + t];
      if (mk) {
        if (ended) return fail(FL_ERR_UNSUPPORTED, "mask must be right padding (1...1 0...0)");
        packed.push_back(ids[(size_t)b * max_len + t]);
        ++L;
      } else {
        ended = true;
      }
    }
    if (L == 0) return fail(FL_ERR_INVALID, "sequence with no tokens");
    lengths[b] = L;
  }
  return forward_common(m, packed.data(), lengths.data(), nseq, FL_F32, out);
}

int fl_model_forward_device(fl_model* m, const int32_t* d_ids, const int64_t* lengths, int nseq,
                            float* d_out) {
  if (!m || (nseq > 0 && (!d_ids || !lengths || !d_out)))
    return fail(FL_ERR_INVALID, "null argument");
  if (nseq < 0) return fail(FL_ERR_INVALID, "negative batch");
  std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
  M_ST(activate(m->ctx));
  if (nseq == 0) return FL_OK;
  Lane& L = lane0(m);
  M_ST(prepare(m, L, lengths, nseq));
  note_write(m->ctx, d_out);
  return run(m, L, d_ids, nseq, d_out, L.flags);
}

int fl_model_embed(fl_model* m, const int64_t* ids, const int64_t* lengths, int nseq, int max_seqs,
                   int64_t max_tokens, float* out, int32_t* batch_nan, int* nbatches) {
  return fl_model_embed_ex(m, ids, lengths, nseq, max_seqs, max_tokens, FL_F32, out, batch_nan,
                           nbatches);
}

int fl_model_embed_ex(fl_model* m, const int64_t* ids, const int64_t* lengths, int nseq,
                      int max_seqs, int64_t max_tokens, int out_dtype, void* out,
                      int32_t* batch_nan, int* nbatches) {
  if (!m || (nseq > 0 && (!ids || !lengths || !out))) return fail(FL_ERR_INVALID, "null argument");
  if (nseq < 0) return fail(FL_ERR_INVALID, "negative batch");
  if (!valid_out_dtype(out_dtype)) return fail(FL_ERR_INVALID, "output dtype must be F32 or F16");
  std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
  M_ST(activate(m->ctx));
  if (nbatches) *nbatches = 0;
  if (nseq == 0) return FL_OK;
  // embeddings.go:704-731: sequences in order; a batch ends before the
  // sequence that would pass max_seqs sequences or max_tokens tokens, but
  // always holds at least one sequence.
  struct Batch { int first, count; int64_t tok0, tokens; };
  std::vector<Batch> plan;
  int64_t tok = 0;
  for (int i = 0; i < nseq;) {
    int count = 0;
    int64_t tokens = 0;
    for (int j = i; j < nseq; ++j) {
      if (lengths[j] <= 0) return fail(FL_ERR_INVALID, "sequence lengths must be positive");
      if (count >= max_seqs) break;
      if (tokens + lengths[j] > max_tokens && count > 0) break;
      tokens += lengths[j];
      ++count;
    }
    if (count == 0) {
      count = 1;
      tokens = lengths[i];
    }
    plan.push_back({i, count, tok, tokens});
    tok += tokens;
    i += count;
  }
  for (int64_t t = 0; t < tok; ++t)
    if (ids[t] < 0 || ids[t] >= m->cfg.vocab_size)  // cpu_backend.go:500-502
      return fail(FL_ERR_INVALID, "Gather index out of bounds");
  // Forwards: runs of consecutive batches of at most `cap` tokens (at least
  // one batch each).
  struct Group { int b0, nb; };
  std::vector<Group> groups;
  int64_t max_gt = 0;
  int max_gs = 0;
  auto make_groups = [&](int64_t cap) {
    groups.clear();
    max_gt = 0;
    max_gs = 0;
    for (int b = 0; b < (int)plan.size();) {
      Group g{b, 0};
      int64_t gt = 0;
      int gs = 0;
      while (b < (int)plan.size() && (g.nb == 0 || gt + plan[(size_t)b].tokens <= cap)) {
        gt += plan[(size_t)b].tokens;
        gs += plan[(size_t)b].count;
        ++g.nb;
        ++b;
      }
      groups.push_back(g);
      max_gt = std::max(max_gt, gt);
      max_gs = std::max(max_gs, gs);
    }
  };
  make_groups(kGroupTokens);

  fl_model::Pipe& P = m->pipe;
  Lane& L0 = lane0(m);
  hipStream_t cs = m->ctx->stream;
  if (!P.ready) {
    for (int k = 1; k < kLanes; ++k)
      if (!m->lane[k].stream)
        M_CHECK(hipStreamCreateWithFlags(&m->lane[k].stream, hipStreamNonBlocking));
    for (int k = 0; k < kLanes; ++k)
      if (!P.d2h[k]) M_CHECK(hipEventCreateWithFlags(&P.d2h[k], hipEventDisableTiming));
    P.ready = true;
  }
  // Every lane's activation buffers, sized for the largest forward, before
  // anything is enqueued (Nomic fp16: ~1.1 GB per lane for 65536 tokens).
  // When the device cannot hold them: one forward per batch of the plan, all
  // on lane 0 (the context stream), as the reference computes them.
  int nl = std::min<int>(kLanes, (int)groups.size());
  {
    int st = FL_OK;
    for (int k = 0; k < nl && st == FL_OK; ++k)
      st = ensure_capacity(m, m->lane[k], max_gt, max_gs, 1, 0);
    if (st == FL_ERR_OOM && groups.size() < plan.size()) {
      for (int k = 1; k < kLanes; ++k) release_activations(m, m->lane[k]);
      make_groups(0);
      nl = 1;
      st = ensure_capacity(m, L0, max_gt, max_gs, 1, 0);
    }
    M_ST(st);
  }
  if (max_gt > P.cap_tok || max_gs > P.cap_seq) {
    for (int k = 0; k < kLanes; ++k) M_CHECK(hipStreamSynchronize(m->lane[k].stream));
    const int64_t ct = std::max(max_gt, P.cap_tok);
    const int cq = std::max(max_gs, P.cap_seq);
    for (int k = 0; k < kLanes; ++k) {
      for (void* h : {(void*)P.ids_pin[k], (void*)P.out_pin[k], (void*)P.flags_pin[k],
                      (void*)P.rows_pin[k]})
        if (h) M_CHECK(hipHostFree(h));
      P.ids_pin[k] = nullptr;
      P.out_pin[k] = nullptr;
      P.flags_pin[k] = nullptr;
      P.rows_pin[k] = nullptr;
      untrack_free(m, P.ids_dev[k]);
      untrack_free(m, P.out_dev[k]);
      untrack_free(m, P.out16_dev[k]);
      untrack_free(m, P.flags_dev[k]);
      untrack_free(m, P.rows_dev[k]);
    }
    // Capacities stay 0 until every buffer of every slot exists: a failure
    // here leaves null pointers and the next call reallocates.
    P.cap_tok = P.cap_seq = 0;
    for (int k = 0; k < kLanes; ++k) {
      if (hipHostMalloc((void**)&P.ids_pin[k], (size_t)ct * 4, hipHostMallocDefault) != hipSuccess ||
          hipHostMalloc((void**)&P.out_pin[k], (size_t)cq * m->H * 4, hipHostMallocDefault) != hipSuccess ||
          hipHostMalloc((void**)&P.flags_pin[k], 8, hipHostMallocDefault) != hipSuccess ||
          hipHostMalloc((void**)&P.rows_pin[k], (size_t)cq * 4, hipHostMallocDefault) != hipSuccess)
        return fail(FL_ERR_OOM, "hipHostMalloc(embed pipeline)");
      M_ST(track_alloc(m, (size_t)ct * 4, P.ids_dev[k]));
      M_ST(track_alloc(m, (size_t)cq * m->H * 4, P.out_dev[k]));
      M_ST(track_alloc(m, (size_t)cq * m->H * 2, P.out16_dev[k]));
      M_ST(track_alloc(m, 8, P.flags_dev[k]));
      M_ST(track_alloc(m, (size_t)cq * 4, P.rows_dev[k]));
    }
    P.cap_tok = ct;
    P.cap_seq = cq;
  }

  // Forward f uses slot and lane f % nl: consecutive forwards compute on
  // the lanes' streams at the same time, each filling the CUs the others'
  // kernels leave idle.  A lane's stream carries its forward's upload,
  // kernels and download in order.  The host fills a slot's pinned ids only
  // after that slot's previous forward has been copied back, and copies
  // results out of it at the same point: the host runs up to kLanes forwards
  // ahead of the device, like the reference's double buffering of outputs
  // (embeddings.go:766-775) with one more buffer.
  const int64_t H = m->H;
  const size_t osz = out_dtype == FL_F16 ? 2 : 4;
  // A batch's NaN flag (embeddings.go:757-764: HasNaN on the batch's pooled
  // output): the forward's own flag when it is one batch, else the OR of
  // its sequences' row flags.
  auto batch_flag = [&](const Group& g, int b, int k) -> int {
    if (g.nb == 1) return P.flags_pin[k][0] != 0;
    const int r0 = plan[(size_t)b].first - plan[(size_t)g.b0].first;
    int any = 0;
    for (int i = 0; i < plan[(size_t)b].count; ++i) any |= P.rows_pin[k][r0 + i];
    return any != 0;
  };
  auto drain = [&](int f) -> int {
    const Group& g = groups[(size_t)f];
    const Batch& p0 = plan[(size_t)g.b0];
    const Batch& pl = plan[(size_t)(g.b0 + g.nb - 1)];
    const int k = f % nl;
    M_CHECK(hipEventSynchronize(P.d2h[k]));
    std::memcpy((char*)out + (size_t)p0.first * H * osz, P.out_pin[k],
                (size_t)(pl.first + pl.count - p0.first) * H * osz);
    if (batch_nan)
      for (int b = g.b0; b < g.b0 + g.nb; ++b) {
        const int flag = batch_flag(g, b, k);
        for (int i = 0; i < plan[(size_t)b].count; ++i) batch_nan[plan[(size_t)b].first + i] = flag;
      }
    return FL_OK;
  };
  const int nf = (int)groups.size();
  for (int f = 0; f < nf; ++f) {
    const Group& g = groups[(size_t)f];
    const Batch& p0 = plan[(size_t)g.b0];
    const Batch& pl = plan[(size_t)(g.b0 + g.nb - 1)];
    const int count = pl.first + pl.count - p0.first;
    const int64_t tokens = pl.tok0 + pl.tokens - p0.tok0;
    const int k = f % nl;
    if (f >= nl) M_ST(drain(f - nl));
    for (int64_t t = 0; t < tokens; ++t) P.ids_pin[k][t] = (int32_t)ids[p0.tok0 + t];
    Lane& L = m->lane[k];
    M_CHECK(hipMemcpyAsync(P.ids_dev[k], P.ids_pin[k], (size_t)tokens * 4, hipMemcpyHostToDevice,
                           L.stream));
    M_ST(prepare(m, L, lengths + p0.first, count));
    M_ST(run(m, L, P.ids_dev[k], count, P.out_dev[k], P.flags_dev[k]));
    if (g.nb > 1) {
      M_CHECK(launch_row_nonfinite(P.out_dev[k], count, (int)H, P.rows_dev[k], L.stream));
      M_CHECK(hipMemcpyAsync(P.rows_pin[k], P.rows_dev[k], (size_t)count * 4,
                             hipMemcpyDeviceToHost, L.stream));
    }
    const void* dev_out = P.out_dev[k];
    if (out_dtype == FL_F16) {
      M_CHECK(launch_cast(P.out_dev[k], FL_F32, P.out16_dev[k], FL_F16, (int64_t)count * H, 0,
                          L.stream));
      dev_out = P.out16_dev[k];
    }
    M_CHECK(hipMemcpyAsync(P.out_pin[k], dev_out, (size_t)count * H * osz, hipMemcpyDeviceToHost,
                           L.stream));
    M_CHECK(hipMemcpyAsync(P.flags_pin[k], P.flags_dev[k], 8, hipMemcpyDeviceToHost, L.stream));
    M_CHECK(hipEventRecord(P.d2h[k], L.stream));
  }
  for (int f = std::max(0, nf - nl); f < nf; ++f) M_ST(drain(f));
  // fl_model_status then reports the last batch (drained, so its forward is done).
  const Group& gl = groups.back();
  const int kl = (nf - 1) % nl;
  if (gl.nb == 1) {
    M_CHECK(hipMemcpyAsync(L0.flags, P.flags_dev[kl], 8, hipMemcpyDeviceToDevice, cs));
  } else {
    const int st[2] = {batch_flag(gl, gl.b0 + gl.nb - 1, kl), P.flags_pin[kl][1]};
    M_CHECK(hipMemcpyAsync(L0.flags, st, 8, hipMemcpyHostToDevice, cs));
    M_CHECK(hipStreamSynchronize(cs));
  }
  if (nbatches) *nbatches = (int)plan.size();
  return FL_OK;
}

int fl_model_status(fl_model* m, int* nan_in_output, int* bad_ids) {
  if (!m) return fail(FL_ERR_INVALID, "null model");
  std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
  M_ST(activate(m->ctx));
  int h[2] = {0, 0};
  M_CHECK(hipMemcpyAsync(h, lane0(m).flags, 8, hipMemcpyDeviceToHost, m->ctx->stream));
  M_CHECK(hipStreamSynchronize(m->ctx->stream));
  if (nan_in_output) *nan_in_output = h[0] != 0;
  if (bad_ids) *bad_ids = h[1] != 0;
  return FL_OK;
}

int fl_model_last_hidden(fl_model* m, float* out, int64_t n) {
  if (!m || !out) return fail(FL_ERR_INVALID, "null argument");
  std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
  M_ST(activate(m->ctx));
  lane0(m);
  // The lane of the most recent forward (fl_model_embed runs forward f on
  // lane f % kLanes); its stream has finished before the copies below read it.
  const Lane& L = m->lane[m->last_lane];
  if (n != L.T * m->H) return fail(FL_ERR_INVALID, "size mismatch");
  M_CHECK(hipStreamSynchronize(L.stream));
  int st;
  // fp32 copy, then (X tiled) the row-major fp16 rows just past it.
  void* tmp = workspace(m->ctx, (size_t)n * 4 + (m->x_tiled ? (size_t)n * m->esz : 0), &st);
  if (st) return st;
  const void* x = L.X;
  if (m->x_tiled) {
    void* rm = (char*)tmp + (size_t)n * 4;
    M_CHECK(launch_untile(m->dtype, L.X, L.T, m->H, rm, m->ctx->stream));
    x = rm;
  }
  M_CHECK(launch_cast(x, m->dtype, tmp, FL_F32, n, 0, m->ctx->stream));
  M_CHECK(hipMemcpyAsync(out, tmp, (size_t)n * 4, hipMemcpyDeviceToHost, m->ctx->stream));
  M_CHECK(hipStreamSynchronize(m->ctx->stream));
  return FL_OK;
}

int fl_model_set_profiling(fl_model* m, int enabled) {
  if (!m) return fail(FL_ERR_INVALID, "null model");
  std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
  M_ST(activate(m->ctx));
  M_ST(collect_profile(m));
  m->prof = enabled != 0;
  for (int i = 0; i < FL_PROF_CLASSES; ++i) {
    m->prof_ms[i] = 0;
    m->prof_cnt[i] = 0;
  }
  return FL_OK;
}

int fl_model_profile_read(fl_model* m, double* ms, int64_t* count) {
  if (!m || !ms || !count) return fail(FL_ERR_INVALID, "null argument");
  std::lock_guard<std::recursive_mutex> lk(m->ctx->mu);
  M_ST(activate(m->ctx));
  M_ST(collect_profile(m));
  for (int i = 0; i < FL_PROF_CLASSES; ++i) {
    ms[i] = m->prof_ms[i];
    count[i] = m->prof_cnt[i];
  }
  return FL_OK;
}

}  // extern "C"
