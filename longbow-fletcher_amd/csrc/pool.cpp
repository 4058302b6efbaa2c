// pool.cpp -- the per-op path's memory layer (internal, host only):
//
//  * a caching device allocator behind fl_alloc / fl_free, the counterpart of
//    the Metal backend's size-bucketed buffer pool
//    (internal/device/metal_darwin.go:151-274, GetTensor / PutTensor);
//  * write tracking of fl_alloc buffers, so that fl_linear / fl_gemm can keep
//    the packed form of a weight between calls and repack it only after the
//    weight was written;
//  * pinned staging of small host-to-device copies, so entry points that take
//    host arrays (indices, positions, lengths) return without waiting for the
//    device.
//
// Everything here is stream-ordered on the context stream: a block freed by
// fl_free goes back to the cache at once, because any later use of it is
// enqueued on the same stream behind the work that used it before.
#include <algorithm>
#include <cstring>
#include <string>

#include "context.hpp"

namespace fl {

// Size class of a request: multiples of 256 B up to 4 KiB, then eight classes
// per power of two (at most 12.5% over the request).
size_t pool_class(size_t bytes) {
  if (bytes <= 4096) return std::max<size_t>(256, (bytes + 255) & ~(size_t)255);
  size_t p = 1;
  while (p * 2 <= bytes) p *= 2;
  const size_t g = p / 8;
  return (bytes + g - 1) / g * g;
}

hipError_t malloc_retry(fl_context* ctx, void** out, size_t bytes, bool evict_packs) {
  *out = nullptr;
  hipError_t e = hipMalloc(out, bytes ? bytes : 16);
  if (e != hipErrorOutOfMemory) return e;
  // The device is full: clear the error, wait until the stream no longer
  // uses the cached blocks, give them back (and the packed copies when the
  // caller holds none) and try once more.
  (void)hipGetLastError();
  e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return e;
  pool_trim(ctx);
  if (evict_packs) drop_all_packs(ctx);
  e = hipMalloc(out, bytes ? bytes : 16);
  if (e == hipErrorOutOfMemory) (void)hipGetLastError();
  return e;
}

int pool_get(fl_context* ctx, size_t bytes, void** out, size_t* cls_out, bool evict_packs) {
  *out = nullptr;
  const size_t cls = pool_class(bytes);
  // A cached block of this class or up to two classes larger (like the
  // Metal pool's bucket + 2 search), smallest first.
  auto it = ctx->cached.lower_bound({ctx->device, cls});
  size_t limit = cls;
  for (int k = 0; k < 2; ++k) limit = pool_class(limit + 1);
  for (; it != ctx->cached.end() && it->first.first == ctx->device && it->first.second <= limit;
       ++it) {
    if (it->second.empty()) continue;
    *out = it->second.back();
    it->second.pop_back();
    ctx->cached_bytes -= (int64_t)it->first.second;
    *cls_out = it->first.second;
    ++ctx->pool_hits;
    return FL_OK;
  }
  ++ctx->pool_misses;
  void* p = nullptr;
  hipError_t e = malloc_retry(ctx, &p, cls, evict_packs);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc(pool)");
  ctx->allocated += (int64_t)cls;
  *out = p;
  *cls_out = cls;
  return FL_OK;
}

void pool_put(fl_context* ctx, void* p, size_t cls, int device) {
  if (!p) return;
  ctx->cached[{device, cls}].push_back(p);
  ctx->cached_bytes += (int64_t)cls;
}

void pool_trim(fl_context* ctx) {
  for (auto& kv : ctx->cached)
    for (void* p : kv.second) {
      (void)hipFree(p);
      ctx->allocated -= (int64_t)kv.first.second;
      ctx->cached_bytes -= (int64_t)kv.first.second;
    }
  ctx->cached.clear();
}

fl_context::Live* find_live(fl_context* ctx, const void* ptr, uintptr_t* base) {
  const uintptr_t a = (uintptr_t)ptr;
  auto it = ctx->live.upper_bound(a);
  if (it == ctx->live.begin()) return nullptr;
  --it;
  if (a >= it->first + it->second.cls) return nullptr;
  if (base) *base = it->first;
  return &it->second;
}

int check_extent(fl_context* ctx, const void* ptr, int64_t bytes, const char* what) {
  if (bytes <= 0 || !ptr) return FL_OK;
  uintptr_t base = 0;
  const fl_context::Live* l = find_live(ctx, ptr, &base);
  if (!l) return FL_OK;
  const uint64_t off = (uintptr_t)ptr - base;
  if (off + (uint64_t)bytes <= l->bytes) return FL_OK;
  return fail(FL_ERR_INVALID, std::string(what) + ": operand of " + std::to_string(bytes) +
                                  " bytes at offset " + std::to_string(off) +
                                  " runs past the end of its " + std::to_string(l->bytes) +
                                  "-byte buffer");
}

void note_write(fl_context* ctx, const void* ptr) {
  if (fl_context::Live* l = find_live(ctx, ptr)) l->gen = ++ctx->gen_counter;
}

void drop_packs(fl_context* ctx, uintptr_t base, size_t cls) {
  auto it = ctx->packs.lower_bound(fl_context::PackKey{base, 0, 0, 0, 0, 0, 0});
  while (it != ctx->packs.end() && it->first.src < base + cls) {
    pool_put(ctx, it->second.buf, it->second.cls, it->second.device);
    ctx->pack_bytes -= (int64_t)it->second.cls;
    it = ctx->packs.erase(it);
  }
}

void drop_all_packs(fl_context* ctx) {
  for (auto& kv : ctx->packs) {
    (void)hipSetDevice(kv.second.device);
    (void)hipFree(kv.second.buf);
    ctx->allocated -= (int64_t)kv.second.cls;
  }
  (void)hipSetDevice(ctx->device);
  ctx->packs.clear();
  ctx->pack_bytes = 0;
}

fl_context::PackEntry* find_pack(fl_context* ctx, const fl_context::PackKey& key) {
  auto it = ctx->packs.find(key);
  if (it == ctx->packs.end() || it->second.device != ctx->device) return nullptr;
  return &it->second;
}

const void* cached_pack(fl_context* ctx, const fl_context::PackKey& key, size_t bytes,
                        const std::function<hipError_t(void*)>& pack, int* status) {
  *status = FL_OK;
  fl_context::Live* src = find_live(ctx, (const void*)key.src);
  if (!src) return nullptr;
  auto it = ctx->packs.find(key);
  if (it != ctx->packs.end() && it->second.device != ctx->device) {
    // Packed on the context's previous device: drop it.
    pool_put(ctx, it->second.buf, it->second.cls, it->second.device);
    ctx->pack_bytes -= (int64_t)it->second.cls;
    ctx->packs.erase(it);
    it = ctx->packs.end();
  }
  if (it != ctx->packs.end()) {
    if (it->second.gen == src->gen) return it->second.buf;
    // The source was written since: pack again into the same block.
    hipError_t e = pack(it->second.buf);
    if (e != hipSuccess) {
      *status = hip_fail(e, "pack");
      return nullptr;
    }
    it->second.gen = src->gen;
    return it->second.buf;
  }
  if (ctx->pack_bytes + (int64_t)bytes > kPackCacheLimit) return nullptr;
  void* buf = nullptr;
  size_t cls = 0;
  // The caller may already hold another entry of this cache (a weight while
  // its bias is packed): no eviction of packs here, and a full device only
  // means this copy is not kept (the caller packs into its scratch).
  const int st = pool_get(ctx, bytes, &buf, &cls, false);
  if (st == FL_ERR_OOM) {
    set_error("");
    return nullptr;
  }
  if (st) {
    *status = st;
    return nullptr;
  }
  hipError_t e = pack(buf);
  if (e != hipSuccess) {
    pool_put(ctx, buf, cls, ctx->device);
    *status = hip_fail(e, "pack");
    return nullptr;
  }
  ctx->packs[key] = fl_context::PackEntry{buf, cls, src->gen, ctx->device};
  ctx->pack_bytes += (int64_t)cls;
  return buf;
}

int stage_upload(fl_context* ctx, void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return FL_OK;
  if (bytes > kStageMax) {
    // Large copies go straight from pageable memory and are waited for, so
    // the caller may reuse its buffer on return.
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync");
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    return FL_OK;
  }
  fl_context::Stage& sg = ctx->stage[ctx->stage_next];
  ctx->stage_next = (ctx->stage_next + 1) % fl_context::kStages;
  hipError_t e;
  if (sg.pending) {
    // The slot's previous copy (kStages uploads ago) has normally finished.
    e = hipEventSynchronize(sg.done);
    if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
    sg.pending = false;
  }
  if (!sg.done) {
    e = hipEventCreateWithFlags(&sg.done, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
  }
  if (sg.cap < bytes) {
    if (sg.host) (void)hipHostFree(sg.host);
    sg.host = nullptr;
    sg.cap = 0;
    size_t cap = 64 << 10;
    while (cap < bytes) cap *= 2;
    e = hipHostMalloc(&sg.host, cap, hipHostMallocDefault);
    if (e != hipSuccess) return hip_fail(e, "hipHostMalloc(staging)");
    sg.cap = cap;
  }
  std::memcpy(sg.host, src, bytes);
  e = hipMemcpyAsync(dst, sg.host, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync");
  e = hipEventRecord(sg.done, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
  sg.pending = true;
  return FL_OK;
}

void release_memory_layer(fl_context* ctx) {
  for (auto& kv : ctx->packs) (void)hipFree(kv.second.buf);
  ctx->packs.clear();
  ctx->pack_bytes = 0;
  for (auto& kv : ctx->live) (void)hipFree((void*)kv.first);
  ctx->live.clear();
  pool_trim(ctx);
  for (auto& sg : ctx->stage) {
    if (sg.pending) (void)hipEventSynchronize(sg.done);
    if (sg.host) (void)hipHostFree(sg.host);
    if (sg.done) (void)hipEventDestroy(sg.done);
    sg = fl_context::Stage{};
  }
}

}  // namespace fl
