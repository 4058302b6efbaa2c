// context.hpp -- the fl_context behind the C ABI (internal, host only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <map>
#include <tuple>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/fletcher_hip.h"

namespace fl {

// Thread-local message for fl_last_error().
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

}  // namespace fl

struct fl_context {
  int device = 0;
  hipStream_t stream = nullptr;
  std::recursive_mutex mu;
  // Device bytes this context holds (fl_vram_usage): pool blocks in use and
  // cached, workspace, tables, model buffers.
  int64_t allocated = 0;

  // fl_alloc buffers in use, by base address: size class, the bytes asked
  // for (the extent every per-op entry point checks its operands against),
  // device, and the write generation (bumped by every entry point that writes
  // into it).
  struct Live {
    size_t cls = 0;
    size_t bytes = 0;
    int device = 0;
    uint64_t gen = 0;
  };
  std::map<uintptr_t, Live> live;
  uint64_t gen_counter = 0;
  // Free blocks by (device, size class), reused in stream order.
  std::map<std::pair<int, size_t>, std::vector<void*>> cached;
  int64_t cached_bytes = 0;
  int64_t pool_hits = 0, pool_misses = 0;

  // Packed weights of fl_linear / fl_gemm, and converted copies of
  // activations (an fp32 tensor read by a 16-bit Linear), keyed by the source
  // pointer and how it was packed; valid while the source buffer's generation
  // matches.
  struct PackKey {
    uintptr_t src;
    int kind, dtype, rows, cols, layout, extra;
    bool operator<(const PackKey& o) const {
      return std::tie(src, kind, dtype, rows, cols, layout, extra) <
             std::tie(o.src, o.kind, o.dtype, o.rows, o.cols, o.layout, o.extra);
    }
  };
  struct PackEntry {
    void* buf = nullptr;
    size_t cls = 0;
    uint64_t gen = 0;
    int device = 0;
  };
  std::map<PackKey, PackEntry> packs;
  int64_t pack_bytes = 0;

  // Pinned host slots of stage_upload, used in turn.
  static constexpr int kStages = 4;
  struct Stage {
    void* host = nullptr;
    size_t cap = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
  } stage[kStages];
  int stage_next = 0;

  // Grow-only scratch for per-op temporaries (stream-ordered reuse).
  void* ws = nullptr;
  size_t ws_size = 0;
  int* flag = nullptr;  // 4-byte device flag (HasNaN)
  // The current device's static scratch array of fl_mean_pool_noalloc
  // (noalloc_scratch), looked up when the context is set to a device.
  void* noalloc = nullptr;

  // RoPE (cos, sin) tables keyed by (base bits, half dim); capacity in positions.
  struct RopeTable {
    float2* cs = nullptr;
    int cap = 0;
  };
  // keyed by (bits of base, bits of scale, half)
  std::map<std::tuple<uint32_t, uint32_t, int>, RopeTable> rope;
  // Tables replaced by larger ones stay allocated until teardown: a model
  // keeps the pointer it was handed for its own lengths.
  std::vector<float2*> rope_retired;
  int64_t rope_bytes = 0;  // all tables, current and retired (part of `allocated`)
};

namespace fl {

inline size_t dtype_size(int dt) { return dt == FL_F32 ? 4 : 2; }

// The configuration a model was created with.
const fl_model_config* model_config(const fl_model* m);

// Makes ctx current on the calling thread (cgo calls land on arbitrary OS threads).
int activate(fl_context* ctx);
// Returns scratch of at least `bytes` (synchronises the stream when it grows).
void* workspace(fl_context* ctx, size_t bytes, int* status);
// Device-side (cos, sin) table for positions [0, max_pos) (float64 angles,
// cpu_backend.go:790-792 with the base as a parameter).
// (cos, sin) of position p and pair i, times `scale`, at [p * half + i] for
// p < max_pos: angles and products in float64, cast to float32 once.
const float2* rope_table(fl_context* ctx, float base, int half, int max_pos, int* status,
                         float scale = 1.0f);
// hipMalloc that, when the device is full, waits for the context stream,
// gives the cached blocks back (and, with evict_packs, the packed weights and
// converted activations) and tries once more.  Every device allocation of the
// library goes through it.  evict_packs must be false while the caller holds
// a pointer from cached_pack.
hipError_t malloc_retry(fl_context* ctx, void** out, size_t bytes, bool evict_packs = true);
// hipMalloc / hipFree counted in ctx->allocated (fl_vram_usage).
int device_alloc(fl_context* ctx, size_t bytes, void** out);
void device_free(fl_context* ctx, void* p, size_t bytes);

// ---- pool.cpp: caching allocator, write tracking, packed weights, staging ----
constexpr int64_t kPackCacheLimit = (int64_t)8 << 30;  // packed weights kept at most
constexpr size_t kStageMax = (size_t)64 << 20;          // larger uploads are synchronous
size_t pool_class(size_t bytes);
// A block of at least `bytes` on the current device (not zeroed): a cached
// one when available, else malloc_retry.
int pool_get(fl_context* ctx, size_t bytes, void** out, size_t* cls, bool evict_packs = true);
void pool_put(fl_context* ctx, void* p, size_t cls, int device);
// hipFree of every cached block.
void pool_trim(fl_context* ctx);
// hipFree of every packed weight and converted activation (the stream must be idle).
void drop_all_packs(fl_context* ctx);
// The fl_alloc buffer containing ptr (base address in *base), or null.
fl_context::Live* find_live(fl_context* ctx, const void* ptr, uintptr_t* base = nullptr);
// FL_OK when [ptr, ptr + bytes) lies inside the fl_alloc buffer that holds
// ptr, or when ptr is not inside any fl_alloc buffer of the context (memory
// of another allocator, which the library cannot size); FL_ERR_INVALID
// naming `what` when the operand runs past the end of its buffer.
int check_extent(fl_context* ctx, const void* ptr, int64_t bytes, const char* what);
// The cache entry of key, or null (no packing, no generation check).
fl_context::PackEntry* find_pack(fl_context* ctx, const fl_context::PackKey& key);
// Marks the fl_alloc buffer containing ptr (if any) as written.
void note_write(fl_context* ctx, const void* ptr);
// Releases the packed copies of sources inside [base, base + cls).
void drop_packs(fl_context* ctx, uintptr_t base, size_t cls);
// The packed form of key.src (an fl_alloc buffer), made by pack(dst) when
// missing or when the source was written since; null when the source is not
// an fl_alloc buffer or the cache is full or the device has no room for it
// (the caller packs into scratch).
const void* cached_pack(fl_context* ctx, const fl_context::PackKey& key, size_t bytes,
                        const std::function<hipError_t(void*)>& pack, int* status);
// Host -> device copy on the context stream that returns without waiting:
// the bytes go through a pinned slot (copies over kStageMax are synchronous).
int stage_upload(fl_context* ctx, void* dst, const void* src, size_t bytes);
// Frees every pool block, packed weight and staging slot (teardown).
void release_memory_layer(fl_context* ctx);

}  // namespace fl
