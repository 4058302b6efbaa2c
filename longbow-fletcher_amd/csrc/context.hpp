// context.hpp -- the fl_context behind the C ABI (internal, host only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
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
  std::unordered_map<void*, int64_t> allocs;  // buffers handed out by fl_alloc
  int64_t allocated = 0;

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
int device_alloc(fl_context* ctx, size_t bytes, void** out);
void device_free(fl_context* ctx, void* p);

}  // namespace fl
