// api.cpp -- C ABI: context, buffers and per-op entry points
// (the Tensor methods of internal/device/device.go:5-116 on HIP).
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "context.hpp"
#include "kernels.hpp"

namespace fl {

static thread_local std::string g_err;

void set_error(const std::string& msg) { g_err = msg; }

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_err = std::string(what) + ": " + hipGetErrorString(e);
  // A failed call also sets the runtime's last error, which the next launch
  // check (hipGetLastError) would report.  Out-of-memory is recoverable:
  // clear it so the context keeps working.
  if (e == hipErrorOutOfMemory) (void)hipGetLastError();
  return e == hipErrorOutOfMemory ? FL_ERR_OOM : FL_ERR_HIP;
}

int activate(fl_context* ctx) {
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  return FL_OK;
}

int device_alloc(fl_context* ctx, size_t bytes, void** out) {
  void* p = nullptr;
  hipError_t e = malloc_retry(ctx, &p, bytes ? bytes : 16);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  ctx->allocated += (int64_t)bytes;
  *out = p;
  return FL_OK;
}

void device_free(fl_context* ctx, void* p, size_t bytes) {
  if (!p) return;
  (void)hipFree(p);
  ctx->allocated -= (int64_t)bytes;
}

void* workspace(fl_context* ctx, size_t bytes, int* status) {
  *status = FL_OK;
  if (bytes <= ctx->ws_size) return ctx->ws;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    *status = hip_fail(e, "hipStreamSynchronize");
    return nullptr;
  }
  if (ctx->ws) {
    (void)hipFree(ctx->ws);
    ctx->allocated -= (int64_t)ctx->ws_size;
    ctx->ws = nullptr;
    ctx->ws_size = 0;
  }
  size_t sz = 1 << 20;
  while (sz < bytes) sz <<= 1;
  void* p = nullptr;
  e = malloc_retry(ctx, &p, sz);
  if (e != hipSuccess) {
    *status = hip_fail(e, "hipMalloc(workspace)");
    return nullptr;
  }
  ctx->ws = p;
  ctx->ws_size = sz;
  ctx->allocated += (int64_t)sz;
  return p;
}

const float2* rope_table(fl_context* ctx, float base, int half, int max_pos, int* status,
                         float scale) {
  *status = FL_OK;
  uint32_t bits, sbits;
  std::memcpy(&bits, &base, 4);
  std::memcpy(&sbits, &scale, 4);
  auto& t = ctx->rope[{bits, sbits, half}];
  if (t.cap >= max_pos && t.cs) return t.cs;
  int cap = 64;
  while (cap < max_pos) cap <<= 1;
  std::vector<float2> host((size_t)cap * half);
  const int d = 2 * half;
  for (int p = 0; p < cap; ++p)
    for (int i = 0; i < half; ++i) {
      // cpu_backend.go:790-792 (base parameterised).
      const double theta = (double)p * std::pow((double)base, -2.0 * (double)i / (double)d);
      host[(size_t)p * half + i] = make_float2((float)(std::cos(theta) * (double)scale),
                                               (float)(std::sin(theta) * (double)scale));
    }
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    *status = hip_fail(e, "hipStreamSynchronize");
    return nullptr;
  }
  // A replaced table stays allocated (and counted) until teardown: a model
  // keeps the pointer it was handed for its own lengths.
  if (t.cs) ctx->rope_retired.push_back(t.cs);
  t.cs = nullptr;
  t.cap = 0;
  void* p = nullptr;
  e = malloc_retry(ctx, &p, host.size() * sizeof(float2));
  if (e != hipSuccess) {
    *status = hip_fail(e, "hipMalloc(rope)");
    return nullptr;
  }
  ctx->allocated += (int64_t)(host.size() * sizeof(float2));
  ctx->rope_bytes += (int64_t)(host.size() * sizeof(float2));
  e = hipMemcpy(p, host.data(), host.size() * sizeof(float2), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    *status = hip_fail(e, "hipMemcpy(rope)");
    return nullptr;
  }
  t.cs = (float2*)p;
  t.cap = cap;
  return t.cs;
}

}  // namespace fl

using namespace fl;

#define FL_ENTER(ctx)                                                  \
  if (!(ctx)) return fail(FL_ERR_INVALID, "null context");             \
  std::lock_guard<std::recursive_mutex> _fl_lock((ctx)->mu);           \
  do {                                                                 \
    int _fl_a = activate(ctx);                                         \
    if (_fl_a) return _fl_a;                                           \
  } while (0)

#define FL_CHECK_LAUNCH(expr)                                          \
  do {                                                                 \
    hipError_t _e = (expr);                                            \
    if (_e != hipSuccess) return hip_fail(_e, #expr);                  \
  } while (0)

static bool valid_dtype(int dt) { return dt == FL_F32 || dt == FL_F16 || dt == FL_BF16; }

// Bytes spanned by a [rows x cols] operand with row stride ld.
static int64_t span(int64_t rows, int64_t cols, int64_t ld, int dtype) {
  if (rows <= 0 || cols <= 0) return 0;
  return ((rows - 1) * ld + cols) * (int64_t)dtype_size(dtype);
}

// Rejects an operand that runs past the end of its fl_alloc buffer before
// anything is enqueued.
#define FL_EXTENT(ptr, bytes, what)                                         \
  do {                                                                      \
    int _fl_x = check_extent(ctx, (ptr), (int64_t)(bytes), (what));        \
    if (_fl_x) return _fl_x;                                                \
  } while (0)

// What a PackKey's `kind` packs.  PK_CONVERTED: a copy of an activation in
// another storage type (key.dtype), for a Linear whose weight has that type.
enum PackKind { PK_GEMM_B = 1, PK_LINEAR_W = 2, PK_LINEAR_BIAS = 3, PK_CONVERTED = 4 };

// The packed form of a weight: kept between calls when the source is an
// fl_alloc buffer (repacked after it is written), else packed into `fallback`
// (per-call scratch).
static const void* packed(fl_context* ctx, const fl_context::PackKey& key, size_t bytes,
                          const std::function<hipError_t(void*)>& pack, void* fallback,
                          int* st) {
  const void* p = cached_pack(ctx, key, bytes, pack, st);
  if (p || *st) return p;
  hipError_t e = pack(fallback);
  if (e != hipSuccess) {
    *st = hip_fail(e, "pack");
    return nullptr;
  }
  return fallback;
}

extern "C" {

const char* fl_last_error(void) { return g_err.c_str(); }

const char* fl_version(void) { return "fletcher-hip 0.1 (gfx950)"; }

int fl_device_count(int* count) {
  if (!count) return fail(FL_ERR_INVALID, "null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  *count = n;
  return FL_OK;
}

int fl_init(int device, fl_context** out) {
  if (!out) return fail(FL_ERR_INVALID, "null out");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (device < 0 || device >= n) return fail(FL_ERR_INVALID, "device index out of range");
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  auto* ctx = new fl_context();
  ctx->device = device;
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return hip_fail(e, "hipStreamCreate");
  }
  void* f = nullptr;
  e = hipMalloc(&f, 256);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return hip_fail(e, "hipMalloc(flag)");
  }
  ctx->flag = (int*)f;
  e = noalloc_scratch(device, &ctx->noalloc);
  if (e != hipSuccess) {
    (void)hipFree(f);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return hip_fail(e, "hipGetSymbolAddress(scratch)");
  }
  *out = ctx;
  return FL_OK;
}

int fl_free_context(fl_context* ctx) {
  if (!ctx) return FL_OK;
  {
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    release_memory_layer(ctx);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->flag) (void)hipFree(ctx->flag);
    for (auto& kv : ctx->rope)
      if (kv.second.cs) (void)hipFree(kv.second.cs);
    for (float2* p : ctx->rope_retired) (void)hipFree(p);
    (void)hipStreamDestroy(ctx->stream);
  }
  delete ctx;
  return FL_OK;
}

int fl_set_device(fl_context* ctx, int device) {
  if (!ctx) return fail(FL_ERR_INVALID, "null context");
  std::lock_guard<std::recursive_mutex> lk(ctx->mu);
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (device < 0 || device >= n) return fail(FL_ERR_INVALID, "device index out of range");
  if (device == ctx->device) return FL_OK;
  // Scratch, flag and tables live on the old device: release them there
  // (buffers from fl_alloc stay where they are).
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->ws) {
    (void)hipFree(ctx->ws);
    ctx->allocated -= (int64_t)ctx->ws_size;
  }
  if (ctx->flag) (void)hipFree(ctx->flag);
  for (auto& kv : ctx->rope)
    if (kv.second.cs) (void)hipFree(kv.second.cs);
  for (float2* p : ctx->rope_retired) (void)hipFree(p);
  ctx->rope_retired.clear();
  ctx->allocated -= ctx->rope_bytes;
  ctx->rope_bytes = 0;
  ctx->ws = nullptr;
  ctx->ws_size = 0;
  ctx->flag = nullptr;
  ctx->rope.clear();
  (void)hipStreamDestroy(ctx->stream);
  ctx->stream = nullptr;
  ctx->device = device;
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");
  void* f = nullptr;
  e = hipMalloc(&f, 256);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc(flag)");
  ctx->flag = (int*)f;
  ctx->noalloc = nullptr;
  e = noalloc_scratch(device, &ctx->noalloc);
  if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
  return FL_OK;
}

int fl_synchronize(fl_context* ctx) {
  FL_ENTER(ctx);
  FL_CHECK_LAUNCH(hipStreamSynchronize(ctx->stream));
  return FL_OK;
}

int fl_vram_usage(fl_context* ctx, int64_t* allocated, int64_t* total) {
  FL_ENTER(ctx);
  size_t free_b = 0, total_b = 0;
  FL_CHECK_LAUNCH(hipMemGetInfo(&free_b, &total_b));
  if (allocated) *allocated = ctx->allocated;
  if (total) *total = (int64_t)total_b;
  return FL_OK;
}

int fl_get_stream(fl_context* ctx, void** stream) {
  if (!ctx || !stream) return fail(FL_ERR_INVALID, "null argument");
  *stream = (void*)ctx->stream;
  return FL_OK;
}

static int alloc_block(fl_context* ctx, int64_t bytes, bool zero, void** out) {
  if (!out || bytes < 0) return fail(FL_ERR_INVALID, "bad allocation request");
  *out = nullptr;
  void* p = nullptr;
  size_t cls = 0;
  if (int st = pool_get(ctx, bytes > 0 ? (size_t)bytes : 16, &p, &cls)) return st;
  if (zero) {
    // Backend.GetTensor hands out zeroed memory (cpu_backend.go:147-156); the
    // fill is ordered on the stream after any earlier use of a reused block.
    hipError_t e = hipMemsetAsync(p, 0, bytes > 0 ? (size_t)bytes : 16, ctx->stream);
    if (e != hipSuccess) {
      pool_put(ctx, p, cls, ctx->device);
      return hip_fail(e, "hipMemsetAsync");
    }
  }
  ctx->live[(uintptr_t)p] =
      fl_context::Live{cls, bytes > 0 ? (size_t)bytes : 0, ctx->device, ++ctx->gen_counter};
  *out = p;
  return FL_OK;
}

int fl_alloc(fl_context* ctx, int64_t bytes, void** out) {
  FL_ENTER(ctx);
  return alloc_block(ctx, bytes, true, out);
}

int fl_alloc_uninit(fl_context* ctx, int64_t bytes, void** out) {
  FL_ENTER(ctx);
  return alloc_block(ctx, bytes, false, out);
}

int fl_free(fl_context* ctx, void* ptr) {
  FL_ENTER(ctx);
  if (!ptr) return FL_OK;
  auto it = ctx->live.find((uintptr_t)ptr);
  if (it == ctx->live.end()) return fail(FL_ERR_INVALID, "pointer not allocated by fl_alloc");
  // No wait: the block goes back to the cache, and whatever reuses it is
  // enqueued on the same stream behind the work already using it.
  drop_packs(ctx, it->first, it->second.cls);
  pool_put(ctx, ptr, it->second.cls, it->second.device);
  ctx->live.erase(it);
  return FL_OK;
}

int fl_pool_stats(fl_context* ctx, int64_t* stats) {
  FL_ENTER(ctx);
  if (!stats) return fail(FL_ERR_INVALID, "null stats");
  int64_t nbuf = 0;
  for (auto& kv : ctx->cached) nbuf += (int64_t)kv.second.size();
  stats[0] = ctx->pool_hits;
  stats[1] = ctx->pool_misses;
  stats[2] = ctx->cached_bytes;
  stats[3] = nbuf;
  stats[4] = ctx->pack_bytes;
  stats[5] = (int64_t)ctx->live.size();
  return FL_OK;
}

int fl_buffer_written(fl_context* ctx, const void* ptr) {
  FL_ENTER(ctx);
  if (!ptr) return fail(FL_ERR_INVALID, "null pointer");
  note_write(ctx, ptr);
  return FL_OK;
}

int fl_pool_trim(fl_context* ctx) {
  FL_ENTER(ctx);
  FL_CHECK_LAUNCH(hipStreamSynchronize(ctx->stream));
  pool_trim(ctx);
  return FL_OK;
}

int fl_copy_to_device(fl_context* ctx, void* dst, const void* src, int64_t bytes) {
  FL_ENTER(ctx);
  if (bytes < 0 || (bytes > 0 && (!dst || !src))) return fail(FL_ERR_INVALID, "bad copy");
  if (bytes == 0) return FL_OK;
  FL_EXTENT(dst, bytes, "fl_copy_to_device dst");
  note_write(ctx, dst);
  // The host buffer may be reused on return: small copies go through a
  // pinned slot without waiting, large ones wait.
  return stage_upload(ctx, dst, src, (size_t)bytes);
}

int fl_copy_to_host(fl_context* ctx, void* dst, const void* src, int64_t bytes) {
  FL_ENTER(ctx);
  if (bytes < 0 || (bytes > 0 && (!dst || !src))) return fail(FL_ERR_INVALID, "bad copy");
  if (bytes == 0) return FL_OK;
  FL_EXTENT(src, bytes, "fl_copy_to_host src");
  FL_CHECK_LAUNCH(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToHost, ctx->stream));
  FL_CHECK_LAUNCH(hipStreamSynchronize(ctx->stream));
  return FL_OK;
}

int fl_copy_device(fl_context* ctx, void* dst, const void* src, int64_t bytes) {
  FL_ENTER(ctx);
  if (bytes < 0 || (bytes > 0 && (!dst || !src))) return fail(FL_ERR_INVALID, "bad copy");
  if (bytes == 0) return FL_OK;
  FL_EXTENT(dst, bytes, "fl_copy_device dst");
  FL_EXTENT(src, bytes, "fl_copy_device src");
  note_write(ctx, dst);
  FL_CHECK_LAUNCH(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return FL_OK;
}

int fl_memset(fl_context* ctx, void* ptr, int value, int64_t bytes) {
  FL_ENTER(ctx);
  if (bytes < 0 || (bytes > 0 && !ptr)) return fail(FL_ERR_INVALID, "bad memset");
  if (bytes == 0) return FL_OK;
  FL_EXTENT(ptr, bytes, "fl_memset");
  note_write(ctx, ptr);
  FL_CHECK_LAUNCH(hipMemsetAsync(ptr, value, (size_t)bytes, ctx->stream));
  return FL_OK;
}

int fl_upload_f32(fl_context* ctx, void* dst, int dtype, const float* src, int64_t n,
                  int rounding) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || n < 0 || (n > 0 && (!dst || !src)))
    return fail(FL_ERR_INVALID, "bad upload");
  if (n == 0) return FL_OK;
  FL_EXTENT(dst, n * (int64_t)dtype_size(dtype), "fl_upload_f32 dst");
  note_write(ctx, dst);
  if (dtype == FL_F32) return stage_upload(ctx, dst, src, (size_t)n * 4);
  if (rounding == FL_ROUND_TRUNCATE && dtype != FL_F16)
    return fail(FL_ERR_UNSUPPORTED, "truncating upload is defined for fp16 only");
  int st;
  float* tmp = (float*)workspace(ctx, (size_t)n * 4, &st);
  if (st) return st;
  if (int s2 = stage_upload(ctx, tmp, src, (size_t)n * 4)) return s2;
  FL_CHECK_LAUNCH(launch_cast(tmp, FL_F32, dst, dtype, n, rounding == FL_ROUND_TRUNCATE,
                              ctx->stream));
  return FL_OK;
}

int fl_download_f32(fl_context* ctx, float* dst, const void* src, int dtype, int64_t n) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || n < 0 || (n > 0 && (!dst || !src)))
    return fail(FL_ERR_INVALID, "bad download");
  if (n == 0) return FL_OK;
  FL_EXTENT(src, n * (int64_t)dtype_size(dtype), "fl_download_f32 src");
  const void* from = src;
  if (dtype != FL_F32) {
    int st;
    float* tmp = (float*)workspace(ctx, (size_t)n * 4, &st);
    if (st) return st;
    FL_CHECK_LAUNCH(launch_cast(src, dtype, tmp, FL_F32, n, 0, ctx->stream));
    from = tmp;
  }
  FL_CHECK_LAUNCH(hipMemcpyAsync(dst, from, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
  FL_CHECK_LAUNCH(hipStreamSynchronize(ctx->stream));
  return FL_OK;
}

// ---------------------------------------------------------------------------
// Tensor ops
// ---------------------------------------------------------------------------

int fl_gemm(fl_context* ctx, int dtype, int trans_a, int trans_b, int m, int n, int k,
            float alpha, const void* a, int lda, const void* b, int ldb, void* c, int ldc) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || m < 0 || n < 0 || k < 0 || !a || !b || !c)
    return fail(FL_ERR_INVALID, "fl_gemm: bad arguments");
  if (m == 0 || n == 0) return FL_OK;
  // A is [m x k] ([k x m] when trans_a), B [k x n] ([n x k] when trans_b).
  const int ar = trans_a ? k : m, ac = trans_a ? m : k;
  const int br = trans_b ? n : k, bc = trans_b ? k : n;
  if (lda < std::max(ac, 1) || ldb < std::max(bc, 1) || ldc < n)
    return fail(FL_ERR_INVALID, "fl_gemm: leading dimension smaller than the row");
  FL_EXTENT(a, span(ar, ac, lda, dtype), "fl_gemm A");
  FL_EXTENT(b, span(br, bc, ldb, dtype), "fl_gemm B");
  FL_EXTENT(c, span(m, n, ldc, dtype), "fl_gemm C");
  note_write(ctx, c);
  GemmEpilogue epi;
  if (!trans_a && alpha == 1.0f) {
    // The four-wave kernel takes B packed [n x k] in its own row order.
    const int lay = gemm_w4_layout(dtype, n, k, EPI_STORE, FL_MATH_EXACT, false);
    const size_t esz = dtype_size(dtype);
    const bool rows_ok = trans_b && !(((uintptr_t)b | ((size_t)ldb * esz)) & 15);
    if (lay >= 0 && ((!trans_b && ldb == n) || rows_ok)) {
      int st;
      void* scratch = workspace(ctx, (size_t)n * k * esz, &st);
      if (st) return st;
      auto pack = [&](void* dst) {
        return trans_b ? launch_pack_rows(dtype, b, ldb, n, k, dst, lay, ctx->stream)
                       : launch_transpose(dtype, b, k, n, dst, lay, ctx->stream);
      };
      const void* w = packed(ctx, {(uintptr_t)b, PK_GEMM_B, dtype, n, k, lay, trans_b ? ldb : -1},
                             (size_t)n * k * esz, pack, scratch, &st);
      if (st) return st;
      GemmEpilogue pe;
      pe.layout = lay;
      if (gemm_nt_supported(dtype, m, n, k, a, lda, w, k, c, ldc, pe)) {
        FL_CHECK_LAUNCH(launch_gemm_nt(dtype, a, lda, w, k, c, ldc, m, n, k, pe, ctx->stream));
        return FL_OK;
      }
    }
    const void* bnk = b;
    int ldbn = ldb;
    if (!trans_b) {
      // B is [k x n]: pack to [n x k] for the MFMA kernel when the shape allows.
      if (gemm_nt_supported(dtype, m, n, k, a, lda, a, k, c, ldc, epi) && ldb == n) {
        int st;
        void* scratch = workspace(ctx, (size_t)n * k * dtype_size(dtype), &st);
        if (st) return st;
        auto pack = [&](void* dst) { return launch_transpose(dtype, b, k, n, dst, 0, ctx->stream); };
        bnk = packed(ctx, {(uintptr_t)b, PK_GEMM_B, dtype, n, k, PACK_PLAIN, -1},
                     (size_t)n * k * dtype_size(dtype), pack, scratch, &st);
        if (st) return st;
        ldbn = k;
      } else {
        bnk = nullptr;
      }
    }
    if (bnk && gemm_nt_supported(dtype, m, n, k, a, lda, bnk, ldbn, c, ldc, epi)) {
      FL_CHECK_LAUNCH(launch_gemm_nt(dtype, a, lda, bnk, ldbn, c, ldc, m, n, k, epi, ctx->stream));
      return FL_OK;
    }
  }
  FL_CHECK_LAUNCH(launch_gemm_generic(dtype, trans_a, trans_b, m, n, k, alpha, a, lda, b, ldb, c,
                                      ldc, nullptr, FL_ACT_IDENTITY, FL_MATH_EXACT, ctx->stream));
  return FL_OK;
}

int fl_linear(fl_context* ctx, int x_dtype, const void* x, int rows, int in_cols, int w_dtype,
              const void* w, int w_layout, int out_cols, const void* bias, int act, int math,
              void* out) {
  FL_ENTER(ctx);
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype) || rows < 0 || in_cols <= 0 ||
      out_cols <= 0 || !x || !w || !out)
    return fail(FL_ERR_INVALID, "fl_linear: bad arguments");
  if (w_layout != FL_W_IN_OUT && w_layout != FL_W_OUT_IN)
    return fail(FL_ERR_INVALID, "fl_linear: bad weight layout");
  if (act < FL_ACT_IDENTITY || act > FL_ACT_SWIGLU) return fail(FL_ERR_INVALID, "bad activation");
  if (act == FL_ACT_SWIGLU && out_cols % 2) return fail(FL_ERR_INVALID, "SwiGLU needs even width");
  // The result, the bias and the arithmetic follow the weight's type; x is
  // converted to it (metal_darwin.go:806-829, 887-903).
  const int dtype = w_dtype;
  const size_t esz = dtype_size(dtype);
  const int res_cols = act == FL_ACT_SWIGLU ? out_cols / 2 : out_cols;
  FL_EXTENT(x, span(rows, in_cols, in_cols, x_dtype), "fl_linear x");
  FL_EXTENT(w, span(in_cols, out_cols, out_cols, dtype), "fl_linear W");
  if (bias) FL_EXTENT(bias, span(1, out_cols, out_cols, dtype), "fl_linear bias");
  FL_EXTENT(out, span(rows, res_cols, res_cols, dtype), "fl_linear out");
  if (rows == 0) return FL_OK;
  note_write(ctx, out);
  const size_t bias_bytes = bias ? ((size_t)out_cols * 4 + 255) / 256 * 256 : 0;
  const size_t w_bytes = ((size_t)out_cols * in_cols * esz + 255) / 256 * 256;
  // SwiGLU runs in the four-wave kernel's epilogue when that kernel takes the
  // shape (16-bit, exact math); otherwise the full product is written first.
  // (A converted x lies in a 256-byte aligned block.)
  const uintptr_t x_addr = x_dtype != dtype ? 0 : (uintptr_t)x;
  const bool w_rows_ok =
      w_layout == FL_W_IN_OUT || !(((uintptr_t)w | ((size_t)in_cols * esz)) & 15);
  const bool fused_swiglu =
      act == FL_ACT_SWIGLU && w_rows_ok && !((x_addr | (uintptr_t)out) & 15) &&
      gemm_w4_layout(dtype, out_cols, in_cols, EPI_SWIGLU, math, bias != nullptr) >= 0;
  const bool unfused = (act == FL_ACT_SWIGLU && !fused_swiglu) || act == FL_ACT_SOFTMAX;
  const size_t y_bytes = unfused ? ((size_t)rows * out_cols * esz + 255) / 256 * 256 : 0;
  const size_t xc_bytes = x_dtype != dtype ? (size_t)rows * in_cols * esz : 0;
  int st;
  // [packed fp32 bias][fp32 bias staging][packed W][unfused product][x converted]
  char* ws = (char*)workspace(ctx, 2 * bias_bytes + w_bytes + y_bytes + xc_bytes, &st);
  if (st) return st;
  if (x_dtype != dtype) {
    // x in the weight's type: a copy kept with the buffer like a packed
    // weight, so the Q, K and V projections of one hidden state convert it
    // once (and a LayerNorm that rewrites the buffer refreshes the copy in
    // its own pass).
    auto conv = [&](void* dst) {
      return launch_cast(x, x_dtype, dst, dtype, (int64_t)rows * in_cols, 0, ctx->stream);
    };
    x = packed(ctx, {(uintptr_t)x, PK_CONVERTED, dtype, rows, in_cols, 0, x_dtype},
               (size_t)rows * in_cols * esz, conv, ws + 2 * bias_bytes + w_bytes + y_bytes, &st);
    if (st) return st;
  }
  void* y = unfused ? (void*)(ws + 2 * bias_bytes + w_bytes) : out;
  const int epi_act = (act == FL_ACT_GELU || act == FL_ACT_TANH) ? act : FL_ACT_IDENTITY;

  GemmEpilogue epi;
  epi.kind = fused_swiglu ? EPI_SWIGLU
                          : (epi_act == FL_ACT_GELU ? EPI_GELU
                                                    : (epi_act == FL_ACT_TANH ? EPI_TANH : EPI_STORE));
  epi.math = math;
  // The four-wave kernel takes W and the bias in its own row order.
  const int lay = gemm_w4_layout(dtype, out_cols, in_cols, epi.kind, math, bias != nullptr);
  epi.layout = lay >= 0 && w_rows_ok ? lay : PACK_PLAIN;
  const int ldy = fused_swiglu ? out_cols / 2 : out_cols;
  const void* wnk = w;
  void* pk = ws + 2 * bias_bytes;
  bool mfma = gemm_nt_supported(dtype, rows, out_cols, in_cols, x, in_cols, pk, in_cols, y,
                                ldy, epi);
  if (mfma && (w_layout == FL_W_IN_OUT || epi.layout != PACK_PLAIN)) {
    auto pack_w = [&](void* dst) -> hipError_t {
      if (w_layout == FL_W_IN_OUT)
        return launch_transpose(dtype, w, in_cols, out_cols, dst, epi.layout, ctx->stream);
      return launch_pack_rows(dtype, w, in_cols, out_cols, in_cols, dst, epi.layout, ctx->stream);
    };
    wnk = packed(ctx, {(uintptr_t)w, PK_LINEAR_W, dtype, in_cols, out_cols, epi.layout, w_layout},
                 (size_t)out_cols * in_cols * esz, pack_w, pk, &st);
    if (st) return st;
  }
  if (mfma) mfma = gemm_nt_supported(dtype, rows, out_cols, in_cols, x, in_cols, wnk, in_cols, y,
                                     ldy, epi);
  // fp32 bias: in the packed row order for the MFMA kernels, in column order
  // for the generic kernel.  Both the bias and the packed weight are kept
  // between calls when they are fl_alloc buffers.
  const int bias_layout = mfma ? epi.layout : -1;
  const float* bias32 = nullptr;
  if (bias) {
    float* stage = (float*)(ws + bias_bytes);
    auto pack_bias = [&](void* dst) -> hipError_t {
      if (bias_layout < 0) return launch_cast(bias, dtype, dst, FL_F32, out_cols, 0, ctx->stream);
      hipError_t e = launch_cast(bias, dtype, stage, FL_F32, out_cols, 0, ctx->stream);
      if (e != hipSuccess) return e;
      return launch_pack_vec_f32(stage, out_cols, (float*)dst, bias_layout, ctx->stream);
    };
    bias32 = (const float*)packed(
        ctx, {(uintptr_t)bias, PK_LINEAR_BIAS, dtype, 1, out_cols, bias_layout, 0},
        (size_t)out_cols * 4, pack_bias, ws, &st);
    if (st) return st;
  }
  epi.bias = mfma ? bias32 : nullptr;
  const float* bias_plain = mfma ? nullptr : bias32;
  if (mfma) {
    FL_CHECK_LAUNCH(launch_gemm_nt(dtype, x, in_cols, wnk, in_cols, y, ldy, rows, out_cols,
                                   in_cols, epi, ctx->stream));
  } else if (fused_swiglu) {
    return fail(FL_ERR_UNSUPPORTED, "fl_linear: SwiGLU operands not 16-byte aligned");
  } else {
    const int tb = w_layout == FL_W_OUT_IN;
    FL_CHECK_LAUNCH(launch_gemm_generic(dtype, 0, tb, rows, out_cols, in_cols, 1.0f, x, in_cols,
                                        w, tb ? in_cols : out_cols, y, out_cols, bias_plain, epi_act,
                                        math, ctx->stream));
  }
  if (act == FL_ACT_SWIGLU && !fused_swiglu) {
    FL_CHECK_LAUNCH(launch_swiglu(dtype, y, rows, out_cols / 2, out, math, ctx->stream));
  } else if (act == FL_ACT_SOFTMAX) {
    FL_CHECK_LAUNCH(hipMemcpyAsync(out, y, (size_t)rows * out_cols * esz, hipMemcpyDeviceToDevice,
                                   ctx->stream));
    FL_CHECK_LAUNCH(launch_activation(dtype, out, rows, out_cols, FL_ACT_SOFTMAX, math, ctx->stream));
  }
  return FL_OK;
}

int fl_add(fl_context* ctx, int dtype, void* t, int other_dtype, const void* other, int64_t n) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || !valid_dtype(other_dtype) || n < 0 || (n > 0 && (!t || !other)))
    return fail(FL_ERR_INVALID, "fl_add");
  FL_EXTENT(t, n * (int64_t)dtype_size(dtype), "fl_add t");
  FL_EXTENT(other, n * (int64_t)dtype_size(other_dtype), "fl_add other");
  note_write(ctx, t);
  FL_CHECK_LAUNCH(launch_add(dtype, t, other_dtype, other, n, ctx->stream));
  return FL_OK;
}

int fl_add_scalar(fl_context* ctx, int dtype, void* t, int64_t n, float v) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || n < 0 || (n > 0 && !t)) return fail(FL_ERR_INVALID, "fl_add_scalar");
  FL_EXTENT(t, n * (int64_t)dtype_size(dtype), "fl_add_scalar t");
  note_write(ctx, t);
  FL_CHECK_LAUNCH(launch_affine(dtype, t, n, 1.0f, v, ctx->stream));
  return FL_OK;
}

int fl_scale(fl_context* ctx, int dtype, void* t, int64_t n, float v) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || n < 0 || (n > 0 && !t)) return fail(FL_ERR_INVALID, "fl_scale");
  FL_EXTENT(t, n * (int64_t)dtype_size(dtype), "fl_scale t");
  if (v == 1.0f) return FL_OK;
  note_write(ctx, t);
  FL_CHECK_LAUNCH(launch_affine(dtype, t, n, v, 0.0f, ctx->stream));
  return FL_OK;
}

int fl_add_bias(fl_context* ctx, int dtype, void* t, int rows, int cols, const void* bias) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || rows < 0 || cols <= 0 || !t || !bias)
    return fail(FL_ERR_INVALID, "fl_add_bias");
  FL_EXTENT(t, span(rows, cols, cols, dtype), "fl_add_bias t");
  FL_EXTENT(bias, span(1, cols, cols, dtype), "fl_add_bias bias");
  note_write(ctx, t);
  FL_CHECK_LAUNCH(launch_add_bias(dtype, t, rows, cols, bias, ctx->stream));
  return FL_OK;
}

int fl_activation(fl_context* ctx, int dtype, void* t, int rows, int cols, int act, int math) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || rows < 0 || cols <= 0 || !t) return fail(FL_ERR_INVALID, "fl_activation");
  if (act != FL_ACT_GELU && act != FL_ACT_TANH && act != FL_ACT_SOFTMAX && act != FL_ACT_IDENTITY)
    return fail(FL_ERR_INVALID, "fl_activation: unsupported activation");
  FL_EXTENT(t, span(rows, cols, cols, dtype), "fl_activation t");
  note_write(ctx, t);
  FL_CHECK_LAUNCH(launch_activation(dtype, t, rows, cols, act, math, ctx->stream));
  return FL_OK;
}

// LayerNorm / AddLayerNorm over an fp32 receiver that a 16-bit Linear has
// read (so a converted copy is kept): the kernel rewrites that copy in the
// same pass, and it stays valid for the next Linear.
static int layernorm_common(fl_context* ctx, int dtype, void* t, int res_dtype, const void* residual,
                            int rows, int cols, const float* gamma, const float* beta, float eps) {
  FL_EXTENT(t, span(rows, cols, cols, dtype), "LayerNorm t");
  if (residual) FL_EXTENT(residual, span(rows, cols, cols, res_dtype), "AddLayerNorm residual");
  FL_EXTENT(gamma, (int64_t)cols * 4, "LayerNorm gamma");
  FL_EXTENT(beta, (int64_t)cols * 4, "LayerNorm beta");
  fl_context::PackEntry* copy = nullptr;
  int copy_dtype = FL_F16;
  if (dtype == FL_F32) {
    for (int cd : {FL_F16, FL_BF16}) {
      copy = find_pack(ctx, {(uintptr_t)t, PK_CONVERTED, cd, rows, cols, 0, FL_F32});
      if (copy) {
        copy_dtype = cd;
        break;
      }
    }
  }
  note_write(ctx, t);
  FL_CHECK_LAUNCH(launch_layernorm_mixed(dtype, t, res_dtype, residual, rows, cols, gamma, beta,
                                         eps, copy_dtype, copy ? copy->buf : nullptr,
                                         ctx->stream));
  if (copy)
    if (const fl_context::Live* l = find_live(ctx, t)) copy->gen = l->gen;
  return FL_OK;
}

int fl_layernorm(fl_context* ctx, int dtype, void* t, int rows, int cols, const float* gamma,
                 const float* beta, float eps) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || rows < 0 || cols <= 0 || !t || !gamma || !beta)
    return fail(FL_ERR_INVALID, "fl_layernorm");
  if (cols > 4096) return fail(FL_ERR_UNSUPPORTED, "fl_layernorm: cols > 4096");
  return layernorm_common(ctx, dtype, t, dtype, nullptr, rows, cols, gamma, beta, eps);
}

int fl_add_layernorm(fl_context* ctx, int dtype, void* t, int res_dtype, const void* residual,
                     int rows, int cols, const float* gamma, const float* beta, float eps) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || !valid_dtype(res_dtype) || rows < 0 || cols <= 0 || !t ||
      !residual || !gamma || !beta)
    return fail(FL_ERR_INVALID, "fl_add_layernorm");
  if (cols > 4096) return fail(FL_ERR_UNSUPPORTED, "fl_add_layernorm: cols > 4096");
  return layernorm_common(ctx, dtype, t, res_dtype, residual, rows, cols, gamma, beta, eps);
}

int fl_gather_rows(fl_context* ctx, int dtype, const void* table, int rows, int cols,
                   const int64_t* idx, int n, void* out) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || rows <= 0 || cols <= 0 || n < 0 || !table || (n > 0 && (!idx || !out)))
    return fail(FL_ERR_INVALID, "fl_gather_rows");
  if (n == 0) return FL_OK;
  FL_EXTENT(table, span(rows, cols, cols, dtype), "Gather table");
  FL_EXTENT(out, span(n, cols, cols, dtype), "Gather out");
  std::vector<int> i32(n);
  for (int i = 0; i < n; ++i) {
    // cpu_backend.go:500-502 panics on out-of-range indices.
    if (idx[i] < 0 || idx[i] >= rows) return fail(FL_ERR_INVALID, "Gather index out of bounds");
    i32[i] = (int)idx[i];
  }
  int st;
  int* d = (int*)workspace(ctx, (size_t)n * 4, &st);
  if (st) return st;
  note_write(ctx, out);
  if ((st = stage_upload(ctx, d, i32.data(), (size_t)n * 4))) return st;
  FL_CHECK_LAUNCH(launch_gather(dtype, table, cols, d, n, out, ctx->stream));
  return FL_OK;
}

static int rope_common(fl_context* ctx, int dtype, void* t, const std::vector<int>& pos, int heads,
                       int head_dim, float base) {
  if (head_dim % 2) return fail(FL_ERR_INVALID, "RoPE needs an even head_dim");
  const int rows = (int)pos.size();
  if (rows == 0) return FL_OK;
  // cpu_backend.go:760-805 rotates batch * seq rows of the tensor (an index
  // panic in Go when the tensor is shorter).
  FL_EXTENT(t, span(rows, (int64_t)heads * head_dim, (int64_t)heads * head_dim, dtype), "ApplyRoPE t");
  int maxp = 0;
  for (int p : pos) maxp = p > maxp ? p : maxp;
  int st;
  const float2* cs = rope_table(ctx, base, head_dim / 2, maxp + 1, &st);
  if (st) return st;
  int* d = (int*)workspace(ctx, (size_t)rows * 4, &st);
  if (st) return st;
  note_write(ctx, t);
  if ((st = stage_upload(ctx, d, pos.data(), (size_t)rows * 4))) return st;
  FL_CHECK_LAUNCH(launch_rope(dtype, t, rows, heads, head_dim, heads * head_dim, d, cs, ctx->stream));
  return FL_OK;
}

int fl_rope(fl_context* ctx, int dtype, void* t, int batch, int seq, int heads, int head_dim,
            float base) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || batch < 0 || seq <= 0 || heads <= 0 || head_dim <= 0 || !t)
    return fail(FL_ERR_INVALID, "fl_rope");
  std::vector<int> pos((size_t)batch * seq);
  for (size_t r = 0; r < pos.size(); ++r) pos[r] = (int)(r % seq);  // cpu_backend.go:783
  return rope_common(ctx, dtype, t, pos, heads, head_dim, base);
}

int fl_rope_varlen(fl_context* ctx, int dtype, void* t, const int64_t* lengths, int nseq, int heads,
                   int head_dim, float base) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || nseq < 0 || heads <= 0 || head_dim <= 0 || !t || (nseq && !lengths))
    return fail(FL_ERR_INVALID, "fl_rope_varlen");
  std::vector<int> pos;
  for (int b = 0; b < nseq; ++b) {
    if (lengths[b] < 0) return fail(FL_ERR_INVALID, "negative length");
    for (int64_t i = 0; i < lengths[b]; ++i) pos.push_back((int)i);
  }
  return rope_common(ctx, dtype, t, pos, heads, head_dim, base);
}

// Builds cu_seqlens and the attention work list on the host and runs the
// kernel that fits the dtype / head size / math mode.
static int attention_common(fl_context* ctx, int dtype, const void* q, const void* k,
                            const void* v, void* out, const std::vector<int64_t>& lengths,
                            int heads, int hidden, float scale, int math) {
  if (heads <= 0 || hidden <= 0 || hidden % heads) return fail(FL_ERR_INVALID, "bad head split");
  const int nseq = (int)lengths.size();
  if (nseq == 0) return FL_OK;
  const int hd = hidden / heads;
  std::vector<int> cu(nseq + 1, 0);
  int max_len = 0;
  int64_t total = 0;
  for (int b = 0; b < nseq; ++b) {
    if (lengths[b] < 0) return fail(FL_ERR_INVALID, "negative length");
    total += lengths[b];
    if (total > INT32_MAX) return fail(FL_ERR_INVALID, "attention: too many rows");
    cu[b + 1] = cu[b] + (int)lengths[b];
    max_len = (int)lengths[b] > max_len ? (int)lengths[b] : max_len;
  }
  const int64_t ext = span(total, hidden, hidden, dtype);
  FL_EXTENT(q, ext, "Attention q");
  FL_EXTENT(k, ext, "Attention k");
  FL_EXTENT(v, ext, "Attention v");
  FL_EXTENT(out, ext, "Attention out");
  const bool fast16 = (dtype == FL_F16 || dtype == FL_BF16) && (hd == 64 || hd == 32) &&
                      math == FL_MATH_EXACT &&
                      hidden % 8 == 0 && (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15) == 0 &&
                      ((uintptr_t)out & 7) == 0;
  const bool fast32 = dtype == FL_F32 && hd == 64 && hidden % 4 == 0 &&
                      (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15) == 0;
  std::vector<AttnWork> work;
  const int waves = max_len > 64 ? 4 : 2;
  const int bq = fast16 ? waves * 32 : 64;
  if (fast16 || fast32) {
    std::vector<int> order(nseq);
    for (int b = 0; b < nseq; ++b) order[b] = b;
    std::stable_sort(order.begin(), order.end(),
                     [&](int a, int b) { return lengths[a] > lengths[b]; });
    for (int b : order)
      for (int h = 0; h < heads; ++h)
        for (int q0 = 0; q0 < (int)lengths[b]; q0 += bq) work.push_back(AttnWork{cu[b], (int)lengths[b], h, q0});
  }
  const size_t cu_bytes = ((size_t)(nseq + 1) * 4 + 255) / 256 * 256;
  int st;
  char* ws = (char*)workspace(ctx, cu_bytes + work.size() * sizeof(AttnWork), &st);
  if (st) return st;
  note_write(ctx, out);
  // cu_seqlens then the work list, one staged copy.
  std::vector<char> meta(cu_bytes + work.size() * sizeof(AttnWork));
  std::memcpy(meta.data(), cu.data(), (size_t)(nseq + 1) * 4);
  if (!work.empty()) std::memcpy(meta.data() + cu_bytes, work.data(), work.size() * sizeof(AttnWork));
  if ((st = stage_upload(ctx, ws, meta.data(), meta.size()))) return st;
  const int* dcu = (const int*)ws;
  const AttnWork* dwork = (const AttnWork*)(ws + cu_bytes);
  if (fast16) {
    FL_CHECK_LAUNCH(launch_attention_flash(dtype, q, k, v, hidden, out, hidden, dcu, dwork,
                                           (int)work.size(), hd, scale, waves, false,
                                           (max_len + bq - 1) / bq, ctx->stream));
  } else if (fast32) {
    FL_CHECK_LAUNCH(launch_attention_f32((const float*)q, (const float*)k, (const float*)v, hidden,
                                         (float*)out, hidden, dcu, dwork, (int)work.size(), scale,
                                         math, ctx->stream));
  } else {
    FL_CHECK_LAUNCH(launch_attention_generic(dtype, q, k, v, hidden, out, hidden, dcu, nseq,
                                             max_len, heads, hd, scale, math, ctx->stream));
  }
  return FL_OK;
}

int fl_attention(fl_context* ctx, int dtype, const void* q, const void* k, const void* v, void* out,
                 int batch, int seq, int heads, int hidden, float scale, int math) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || batch < 0 || seq < 0 || !q || !k || !v || !out)
    return fail(FL_ERR_INVALID, "fl_attention");
  std::vector<int64_t> lengths(batch, seq);
  return attention_common(ctx, dtype, q, k, v, out, lengths, heads, hidden, scale, math);
}

int fl_attention_varlen(fl_context* ctx, int dtype, const void* q, const void* k, const void* v,
                        void* out, const int64_t* lengths, int nseq, int heads, int hidden,
                        float scale, int math) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || nseq < 0 || !q || !k || !v || !out || (nseq && !lengths))
    return fail(FL_ERR_INVALID, "fl_attention_varlen");
  std::vector<int64_t> l(lengths, lengths + nseq);
  return attention_common(ctx, dtype, q, k, v, out, l, heads, hidden, scale, math);
}

int fl_cast(fl_context* ctx, const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n) {
  FL_ENTER(ctx);
  if (!valid_dtype(src_dtype) || !valid_dtype(dst_dtype) || n < 0 || (n > 0 && (!src || !dst)))
    return fail(FL_ERR_INVALID, "fl_cast");
  FL_EXTENT(src, n * (int64_t)dtype_size(src_dtype), "Cast src");
  FL_EXTENT(dst, n * (int64_t)dtype_size(dst_dtype), "Cast dst");
  note_write(ctx, dst);
  FL_CHECK_LAUNCH(launch_cast(src, src_dtype, dst, dst_dtype, n, 0, ctx->stream));
  return FL_OK;
}

int fl_has_nan(fl_context* ctx, const void* t, int dtype, int64_t n, int* out) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || n < 0 || !out || (n > 0 && !t)) return fail(FL_ERR_INVALID, "fl_has_nan");
  FL_EXTENT(t, n * (int64_t)dtype_size(dtype), "HasNaN t");
  FL_CHECK_LAUNCH(hipMemsetAsync(ctx->flag, 0, 4, ctx->stream));
  FL_CHECK_LAUNCH(launch_has_nan(t, dtype, n, ctx->flag, ctx->stream));
  int h = 0;
  FL_CHECK_LAUNCH(hipMemcpyAsync(&h, ctx->flag, 4, hipMemcpyDeviceToHost, ctx->stream));
  FL_CHECK_LAUNCH(hipStreamSynchronize(ctx->stream));
  *out = h != 0;
  return FL_OK;
}

int fl_slice(fl_context* ctx, int dtype, const void* src, int rows, int cols, int r0, int r1, int c0,
             int c1, void* dst) {
  FL_ENTER(ctx);
  // cpu_backend.go:288-294 panics on empty slices.
  if (!valid_dtype(dtype) || !src || !dst || r0 < 0 || c0 < 0 || r1 > rows || c1 > cols ||
      r1 - r0 <= 0 || c1 - c0 <= 0)
    return fail(FL_ERR_INVALID, "Slice: invalid dimensions");
  FL_EXTENT(src, span(rows, cols, cols, dtype), "Slice src");
  FL_EXTENT(dst, span(r1 - r0, c1 - c0, c1 - c0, dtype), "Slice dst");
  note_write(ctx, dst);
  FL_CHECK_LAUNCH(launch_slice(dtype, src, cols, r0, r1, c0, c1, dst, ctx->stream));
  return FL_OK;
}

int fl_mean_pool(fl_context* ctx, int dtype, const void* hidden, int cols, const int64_t* lengths,
                 int nseq, int l2, float* out) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || cols <= 0 || nseq < 0 || (nseq && (!hidden || !lengths || !out)))
    return fail(FL_ERR_INVALID, "fl_mean_pool");
  if (nseq == 0) return FL_OK;
  std::vector<int> cu(nseq + 1, 0);
  int max_len = 0;
  int64_t total = 0;
  for (int b = 0; b < nseq; ++b) {
    if (lengths[b] <= 0) return fail(FL_ERR_INVALID, "mean pool needs non-empty sequences");
    total += lengths[b];
    if (total > INT32_MAX) return fail(FL_ERR_INVALID, "fl_mean_pool: too many rows");
    cu[b + 1] = cu[b] + (int)lengths[b];
    max_len = (int)lengths[b] > max_len ? (int)lengths[b] : max_len;
  }
  FL_EXTENT(hidden, span(cu[nseq], cols, cols, dtype), "mean pool hidden");
  FL_EXTENT(out, span(nseq, cols, cols, FL_F32), "mean pool out");
  const int rpc = 64;
  const size_t chunks = (size_t)(max_len + rpc - 1) / rpc;
  const size_t cu_bytes = ((size_t)(nseq + 1) * 4 + 255) / 256 * 256;
  int st;
  char* ws = (char*)workspace(ctx, cu_bytes + (size_t)nseq * chunks * cols * 4, &st);
  if (st) return st;
  note_write(ctx, out);
  if ((st = stage_upload(ctx, ws, cu.data(), (size_t)(nseq + 1) * 4))) return st;
  FL_CHECK_LAUNCH(launch_mean_pool_staged(dtype, hidden, cols, (const int*)ws, nseq, max_len, l2,
                                          (float*)(ws + cu_bytes), out, nullptr, rpc, ctx->stream));
  return FL_OK;
}

int fl_mean_pool_noalloc(fl_context* ctx, int dtype, const void* hidden, int cols,
                         const int64_t* lengths, int nseq, int l2, float* out) {
  FL_ENTER(ctx);
  if (!valid_dtype(dtype) || cols <= 0 || nseq < 0 || (nseq && (!hidden || !lengths || !out)))
    return fail(FL_ERR_INVALID, "fl_mean_pool_noalloc");
  if (nseq == 0) return FL_OK;
  if (nseq > FL_NOALLOC_MAX_SEQS)
    return fail(FL_ERR_INVALID, "fl_mean_pool_noalloc: more than " +
                                    std::to_string(FL_NOALLOC_MAX_SEQS) + " sequences");
  NoAllocLengths la;
  la.n = nseq;
  int64_t total = 0;
  int max_len = 0;
  for (int b = 0; b < nseq; ++b) {
    if (lengths[b] <= 0) return fail(FL_ERR_INVALID, "mean pool needs non-empty sequences");
    total += lengths[b];
    if (total > INT32_MAX) return fail(FL_ERR_INVALID, "fl_mean_pool_noalloc: too many rows");
    la.len[b] = (int)lengths[b];
    max_len = la.len[b] > max_len ? la.len[b] : max_len;
  }
  const int64_t chunks = (max_len + kNoAllocRowsPerChunk - 1) / kNoAllocRowsPerChunk;
  const int64_t need = (int64_t)nseq * chunks * cols * 4;
  if (need > (int64_t)FL_NOALLOC_PARTIAL_BYTES)
    return fail(FL_ERR_INVALID, "fl_mean_pool_noalloc: partial sums need " +
                                    std::to_string(need) + " bytes, the scratch array holds " +
                                    std::to_string((int64_t)FL_NOALLOC_PARTIAL_BYTES));
  if (!ctx->noalloc) return fail(FL_ERR_HIP, "fl_mean_pool_noalloc: no scratch address");
  FL_EXTENT(hidden, span(total, cols, cols, dtype), "mean pool hidden");
  FL_EXTENT(out, span(nseq, cols, cols, FL_F32), "mean pool out");
  note_write(ctx, out);
  FL_CHECK_LAUNCH(launch_mean_pool_noalloc(dtype, hidden, cols, la, max_len, l2, out,
                                           ctx->device, ctx->noalloc, ctx->stream));
  return FL_OK;
}

}  // extern "C"
