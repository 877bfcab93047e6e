// The C ABI of liblocalfold.so (include/localfold.h): context, memory, profiling, weight
// views, and the op entry points that validate and forward to the launchers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>

#include "lf_context.h"
#include "lf_ops.h"

namespace {
thread_local std::string g_error;
}

namespace lf {

int set_error(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return LF_OK;
  return set_error(e == hipErrorOutOfMemory ? LF_ERR_MEMORY : LF_ERR_DEVICE,
                   std::string(what) + ": " + hipGetErrorString(e));
}

int workspace(lf_context* ctx, const size_t* sizes, void** out, int n) {
  size_t total = 0;
  for (int i = 0; i < n; ++i) total += (sizes[i] + 255) & ~size_t(255);
  if (total > ctx->ws_bytes) {
    if (ctx->ws) {
      LF_TRY(check_hip(hipStreamSynchronize(ctx->stream), "workspace sync"));
      LF_TRY(check_hip(hipFree(ctx->ws), "workspace free"));
      ctx->ws = nullptr;
      ctx->ws_bytes = 0;
    }
    const size_t grow = std::max(total, size_t(1) << 20);
    LF_TRY(check_hip(hipMalloc(&ctx->ws, grow), "workspace allocation"));
    ctx->ws_bytes = grow;
    ctx->peak_bytes = std::max(ctx->peak_bytes, ctx->resident());
  }
  char* p = static_cast<char*>(ctx->ws);
  for (int i = 0; i < n; ++i) {
    out[i] = p;
    p += (sizes[i] + 255) & ~size_t(255);
  }
  return LF_OK;
}

int mask_table(lf_context* ctx, const void* mask, int kind, long long a, long long b, float f, size_t bytes,
               void** out, bool* filled) {
  *out = nullptr;
  *filled = false;
  if (ctx->mask_scope <= 0) return LF_OK;
  for (auto& t : ctx->mask_tables)
    if (t.valid && t.mask == mask && t.kind == kind && t.a == a && t.b == b && t.f == f && t.bytes >= bytes) {
      *out = t.buf;
      *filled = true;
      return LF_OK;
    }
  for (auto& t : ctx->mask_tables)   // a buffer of an earlier scope
    if (!t.valid && t.bytes >= bytes) {
      t = lf_context::MaskTable{mask, kind, a, b, f, true, t.buf, t.bytes};
      *out = t.buf;
      return LF_OK;
    }
  void* buf = nullptr;
  LF_TRY(check_hip(hipMalloc(&buf, bytes), "mask table allocation"));
  ctx->mask_tables.push_back(lf_context::MaskTable{mask, kind, a, b, f, true, buf, bytes});
  ctx->mask_bytes += bytes;
  ctx->peak_bytes = std::max(ctx->peak_bytes, ctx->resident());
  *out = buf;
  return LF_OK;
}

LaunchScope::LaunchScope(lf_context* c, const char* label) : ctx(c) {
  if (!ctx->profile) return;
  lf_context::Rec r;
  r.label = ctx->label_prefix ? std::string(ctx->label_prefix) + "/" + label : std::string(label);
  if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) return;
  hipEventRecord(r.start, ctx->stream);
  ctx->recs.push_back(r);
  idx = (int)ctx->recs.size() - 1;
}

LaunchScope::~LaunchScope() {
  if (idx >= 0) hipEventRecord(ctx->recs[idx].stop, ctx->stream);
}

// How the kernels fetch the view: in runs of 8 adjacent stored weights when the run's first
// flat index is a multiple of 8 (so an int5 run is 5 whole bytes and a flat group, a
// power-of-two multiple of 8, holds the whole run), the data pointer is aligned for the run's
// vector load and flat and int5 bit offsets fit 32 bits; per-column groups need the run along
// k (one column, one scale).  Otherwise weight by weight.
static int weight_run(WView& v, long long elements) {
  static const int align[] = {16, 16, 16, 8, 4};   // f32 (two 16-byte loads), f16, bf16, int8, int5
  if (elements >= (1LL << 28)) return WRUN_GATHER;
  if ((reinterpret_cast<uintptr_t>(v.data) & (uintptr_t)(align[v.dtype] - 1)) != 0) return WRUN_GATHER;
  const bool quant = v.dtype == LF_INT8 || v.dtype == LF_INT5;
  v.gshift = 0;
  if (quant && v.group > 0) {
    if (v.group % 8 != 0 || (v.group & (v.group - 1)) != 0) return WRUN_GATHER;
    while ((1 << v.gshift) < v.group) ++v.gshift;
  }
  if (v.ld_k == 1 && v.K % 8 == 0 && v.ld_n % 8 == 0) return WRUN_K;
  if (v.ld_n == 1 && v.col_stride == 1 && v.col_off % 8 == 0 && v.N % 8 == 0 && v.ld_k % 8 == 0 &&
      !(quant && v.group == 0))
    return WRUN_N;
  return WRUN_GATHER;
}

int make_view(const lf_weight& w, int K, int N, const char* name, WView* out, int col_off, int col_stride,
              bool subset) {
  const std::string nm(name);
  if (!w.data) return set_error(LF_ERR_INVALID, nm + ": weight data is NULL");
  if (w.layout != LF_IN_OUT && w.layout != LF_OUT_IN) return set_error(LF_ERR_INVALID, nm + ": bad layout");
  const int in = w.layout == LF_IN_OUT ? w.rows : w.cols;
  const int outc = w.layout == LF_IN_OUT ? w.cols : w.rows;
  if (in != K) return set_error(LF_ERR_INVALID, nm + " has " + std::to_string(in) + " inputs; expected " + std::to_string(K));
  if (col_off + (long long)(N - 1) * col_stride >= outc || (!subset && col_stride == 1 && col_off == 0 && outc != N))
    return set_error(LF_ERR_INVALID,
                     nm + " has " + std::to_string(outc) + " outputs; expected " + std::to_string((long long)N * col_stride));
  WView v{};
  v.data = w.data;
  v.scales = static_cast<const uint16_t*>(w.scales);
  v.zeros = static_cast<const uint16_t*>(w.zeros);
  v.dtype = w.dtype;
  v.group = w.group;
  v.K = K;
  v.N = N;
  v.col_off = col_off;
  v.col_stride = col_stride;
  if (w.layout == LF_IN_OUT) {
    v.ld_k = w.cols;
    v.ld_n = 1;
  } else {
    v.ld_k = 1;
    v.ld_n = w.cols;
  }
  switch (w.dtype) {
    case LF_F32:
    case LF_F16:
    case LF_BF16:
      break;
    case LF_INT8:
      if (!w.scales) return set_error(LF_ERR_INVALID, nm + ": int8 weight needs scales");
      if (w.group < 0) return set_error(LF_ERR_INVALID, nm + ": group must be >= 0");
      break;
    case LF_INT5:
      if (!w.scales || !w.zeros) return set_error(LF_ERR_INVALID, nm + ": int5 weight needs scales and zeros");
      if (w.group < 0 || (w.group > 0 && (w.group * 5) % 8 != 0))
        return set_error(LF_ERR_INVALID, nm + ": int5 group must pack into whole bytes");
      break;
    default:
      return set_error(LF_ERR_INVALID, nm + ": unknown dtype " + std::to_string(w.dtype));
  }
  v.run = weight_run(v, (long long)w.rows * w.cols);
  *out = v;
  return LF_OK;
}

}  // namespace lf

using lf::check_hip;
using lf::set_error;

extern "C" {

const char* lf_last_error(void) { return g_error.c_str(); }
const char* lf_version(void) { return "localfold-mi355x 0.1 (gfx950)"; }

lf_context* lf_context_create(int device_ordinal) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    set_error(LF_ERR_DEVICE, "no HIP device is available");
    return nullptr;
  }
  if (device_ordinal < 0 || device_ordinal >= count) {
    set_error(LF_ERR_INVALID, "device ordinal out of range");
    return nullptr;
  }
  if (check_hip(hipSetDevice(device_ordinal), "hipSetDevice") != LF_OK) return nullptr;
  lf_context* ctx = new lf_context();
  ctx->device = device_ordinal;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_ordinal) == hipSuccess && cus > 0)
    ctx->num_cus = cus;
  if (check_hip(hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking), "hipStreamCreate") != LF_OK) {
    delete ctx;
    return nullptr;
  }
  ctx->stream = ctx->own_stream;
  if (lf::tri_noalloc_init(device_ordinal) != LF_OK) {
    hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return nullptr;
  }
  return ctx;
}

void lf_context_destroy(lf_context* ctx) {
  if (!ctx) return;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  for (auto& r : ctx->recs) {
    hipEventDestroy(r.start);
    hipEventDestroy(r.stop);
  }
  for (auto& a : ctx->user_allocs) hipFree(a.first);
  for (auto& t : ctx->mask_tables) hipFree(t.buf);
  if (ctx->ws) hipFree(ctx->ws);
  if (ctx->own_stream) hipStreamDestroy(ctx->own_stream);
  delete ctx;
}

int lf_context_set_stream(lf_context* ctx, void* hip_stream) {
  if (!ctx) return set_error(LF_ERR_INVALID, "context is NULL");
  ctx->stream = static_cast<hipStream_t>(hip_stream);
  return LF_OK;
}

int lf_malloc(lf_context* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return set_error(LF_ERR_INVALID, "lf_malloc: NULL argument");
  hipSetDevice(ctx->device);
  void* p = nullptr;
  int rc = check_hip(hipMalloc(&p, std::max<size_t>(bytes, 1)), "lf_malloc");
  if (rc != LF_OK) return rc;
  ctx->user_allocs.emplace_back(p, bytes);
  ctx->user_bytes += bytes;
  ctx->alloc_count += 1;
  ctx->peak_bytes = std::max(ctx->peak_bytes, ctx->resident());
  *out = p;
  return LF_OK;
}

int lf_free(lf_context* ctx, void* ptr) {
  if (!ctx) return set_error(LF_ERR_INVALID, "lf_free: NULL context");
  if (!ptr) return LF_OK;
  auto it = std::find_if(ctx->user_allocs.begin(), ctx->user_allocs.end(),
                         [ptr](const std::pair<void*, size_t>& a) { return a.first == ptr; });
  if (it == ctx->user_allocs.end()) return set_error(LF_ERR_INVALID, "lf_free: pointer was not allocated by lf_malloc");
  int rc = check_hip(hipStreamSynchronize(ctx->stream), "lf_free sync");
  if (rc != LF_OK) return rc;
  ctx->user_bytes -= it->second;
  ctx->user_allocs.erase(it);
  return check_hip(hipFree(ptr), "lf_free");
}

int lf_memcpy_htod(lf_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return set_error(LF_ERR_INVALID, "NULL context");
  int rc = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "memcpy htod");
  if (rc != LF_OK) return rc;
  return check_hip(hipStreamSynchronize(ctx->stream), "memcpy htod sync");
}

int lf_memcpy_dtoh(lf_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return set_error(LF_ERR_INVALID, "NULL context");
  int rc = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "memcpy dtoh");
  if (rc != LF_OK) return rc;
  return check_hip(hipStreamSynchronize(ctx->stream), "memcpy dtoh sync");
}

int lf_memset(lf_context* ctx, void* dst, int value, size_t bytes) {
  if (!ctx) return set_error(LF_ERR_INVALID, "NULL context");
  return check_hip(hipMemsetAsync(dst, value, bytes, ctx->stream), "memset");
}

int lf_synchronize(lf_context* ctx) {
  if (!ctx) return set_error(LF_ERR_INVALID, "NULL context");
  return check_hip(hipStreamSynchronize(ctx->stream), "synchronize");
}

int lf_memory_stats(lf_context* ctx, size_t* current_bytes, size_t* peak_bytes, size_t* allocation_count) {
  if (!ctx) return set_error(LF_ERR_INVALID, "NULL context");
  if (current_bytes) *current_bytes = ctx->resident();
  if (peak_bytes) *peak_bytes = ctx->peak_bytes;
  if (allocation_count) *allocation_count = ctx->alloc_count + (ctx->ws ? 1 : 0) + ctx->mask_tables.size();
  return LF_OK;
}

int lf_profile_enable(lf_context* ctx, int enable) {
  if (!ctx) return set_error(LF_ERR_INVALID, "NULL context");
  ctx->profile = enable != 0;
  return LF_OK;
}

int lf_profile_read(lf_context* ctx, lf_kernel_timing* out, int max) {
  if (!ctx) return set_error(LF_ERR_INVALID, "NULL context");
  int rc = check_hip(hipStreamSynchronize(ctx->stream), "profile sync");
  if (rc != LF_OK) return -rc;
  int n = 0;
  for (auto& r : ctx->recs) {
    if (out && n < max) {
      float ms = 0.f;
      hipEventElapsedTime(&ms, r.start, r.stop);
      std::memset(out[n].label, 0, sizeof(out[n].label));
      std::strncpy(out[n].label, r.label.c_str(), sizeof(out[n].label) - 1);
      out[n].ms = ms;
      ++n;
    }
    hipEventDestroy(r.start);
    hipEventDestroy(r.stop);
  }
  ctx->recs.clear();
  return n;
}

#define LF_ENTRY(fn, argtype)                                                          \
  int fn(lf_context* ctx, const argtype* args) {                                       \
    if (!ctx || !args) return set_error(LF_ERR_INVALID, #fn ": NULL context or args"); \
    hipSetDevice(ctx->device);                                                         \
    return lf::impl_##fn(ctx, *args);                                                  \
  }

}  // extern "C"

namespace lf {
inline int impl_lf_tri_mult(lf_context* c, const lf_tri_mult_args& a) { return tri_mult(c, a); }
inline int impl_lf_tri_mult_noalloc(lf_context* c, const lf_tri_mult_args& a) { return tri_mult_noalloc(c, a); }
inline int impl_lf_attention(lf_context* c, const lf_attention_args& a) { return attention(c, a); }
inline int impl_lf_transition(lf_context* c, const lf_transition_args& a) { return transition(c, a); }
inline int impl_lf_outer_product_mean(lf_context* c, const lf_opm_args& a) { return outer_product_mean(c, a); }
inline int impl_lf_global_column_attention(lf_context* c, const lf_global_attention_args& a) {
  return global_attention(c, a);
}
inline int impl_lf_input_embedder(lf_context* c, const lf_input_embedder_args& a) { return input_embedder(c, a); }
}  // namespace lf

extern "C" {
LF_ENTRY(lf_tri_mult, lf_tri_mult_args)
LF_ENTRY(lf_tri_mult_noalloc, lf_tri_mult_args)
LF_ENTRY(lf_attention, lf_attention_args)
LF_ENTRY(lf_transition, lf_transition_args)
LF_ENTRY(lf_outer_product_mean, lf_opm_args)
LF_ENTRY(lf_global_column_attention, lf_global_attention_args)
LF_ENTRY(lf_input_embedder, lf_input_embedder_args)
}
