// Host-side context: device, stream, scratch workspace, allocation stats and per-kernel
// timestamps.  Internal to liblocalfold.so (the C ABI in include/localfold.h wraps it).
#pragma once
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "../../include/localfold.h"

struct lf_context {
  int device = 0;
  int num_cus = 256;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  // scratch workspace: one grow-only device buffer carved per call
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // caller allocations through lf_malloc
  size_t user_bytes = 0, peak_bytes = 0, alloc_count = 0;
  size_t mask_bytes = 0;   // mask tables below (kept for the context's lifetime)
  size_t resident() const { return user_bytes + ws_bytes + mask_bytes; }
  std::vector<std::pair<void*, size_t>> user_allocs;
  // Tables derived from a mask alone (attention key-bias rows, OPM pair normalisers), kept
  // while `mask_scope` > 0 -- a stack call, whose masks do not change -- so that the later
  // blocks reuse the first block's tables instead of recomputing them.  The buffers are kept
  // for the context's lifetime and refilled by the next scope.
  struct MaskTable {
    const void* mask;
    int kind;
    long long a, b;
    float f;
    bool valid;
    void* buf;
    size_t bytes;
  };
  int mask_scope = 0;
  std::vector<MaskTable> mask_tables;
  // profiling
  bool profile = false;
  const char* label_prefix = nullptr;   // block stage naming the launches (profiling only)
  struct Rec {
    std::string label;
    hipEvent_t start, stop;
  };
  std::vector<Rec> recs;
};

namespace lf {

int set_error(int code, const std::string& msg);
int check_hip(hipError_t e, const char* what);

// Carves `n` buffers from the context workspace (256-byte aligned), growing it if needed.
// Growing synchronises the stream first, so earlier kernels finish with the old buffer.
int workspace(lf_context* ctx, const size_t* sizes, void** out, int n);

// A table derived from `mask` (kind and shape a, b, f) for the current stack scope: returns
// its buffer in *out, and whether it is already filled (*filled; false: the caller computes it
// into *out now).  Outside a stack scope *out is null and the caller uses its workspace.
int mask_table(lf_context* ctx, const void* mask, int kind, long long a, long long b, float f, size_t bytes,
               void** out, bool* filled);

// Opens a stack scope for mask tables (nested scopes share the outer one).
struct MaskScope {
  lf_context* ctx;
  explicit MaskScope(lf_context* c) : ctx(c) { ++c->mask_scope; }
  ~MaskScope() {
    if (--ctx->mask_scope == 0)
      for (auto& t : ctx->mask_tables) t.valid = false;
  }
};

// Brackets a kernel launch with events when profiling is on.
struct LaunchScope {
  lf_context* ctx;
  int idx = -1;
  LaunchScope(lf_context* c, const char* label);
  ~LaunchScope();
};

// Names the block stage that the launches inside it belong to ("stage/kernel" labels).
struct StageScope {
  lf_context* ctx;
  const char* saved;
  StageScope(lf_context* c, const char* stage) : ctx(c), saved(c->label_prefix) { c->label_prefix = stage; }
  ~StageScope() { ctx->label_prefix = saved; }
};

}  // namespace lf

#define LF_TRY(expr)            \
  do {                          \
    int _rc = (expr);           \
    if (_rc != LF_OK) return _rc; \
  } while (0)

#define LF_REQUIRE(cond, msg)                                     \
  do {                                                            \
    if (!(cond)) return ::lf::set_error(LF_ERR_INVALID, (msg));   \
  } while (0)
