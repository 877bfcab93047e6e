// localfold_napi.node: a thin N-API binding of the C ABI in include/localfold.h for the Node
// host (localfold_amd/js/index.js).  It marshals plain JS objects into the C argument structs;
// device memory is handled as opaque buffer handles (napi externals) created by `upload` /
// `alloc` and released by `free` (or by the garbage collector as a last resort).
//
// Errors: every C call's status is checked; a failure throws a JS Error carrying
// lf_last_error().  Argument-shape validation happens in JS before crossing (the reference's
// RangeErrors, webgpu/kernels/triangle/types.js:13-48) and again in the library.
#include <node_api.h>

#include <dlfcn.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/localfold.h"

namespace {

// A context handle shared by the JS context object and every buffer made on it.  Buffers are
// freed by their finalizers, which N-API may run after contextDestroy (or at exit, in any
// order), so the holder outlives the context: once the context is gone a finalizer frees
// nothing (lf_context_destroy released every allocation), and the last reference deletes
// the holder.
//
// One lf_context is not safe for concurrent use (its workspace, mask tables, allocation list
// and profile records are unguarded), so every use of it from this addon holds `mu`: a run on
// a worker thread holds it for the whole run, and a call on the JS thread (an op, an upload,
// a free, a finalizer, contextDestroy) waits for a pending run to finish.  index.js also
// queues the runs of one device, so the JS thread does not normally wait here.
struct CtxHolder {
  lf_context* ctx;
  bool alive;
  long refs;
  std::mutex mu;
};

// Holds the context's lock for the scope of a JS-thread call.
struct CtxGuard {
  std::unique_lock<std::mutex> lock;
  explicit CtxGuard(CtxHolder* h) {
    if (h) lock = std::unique_lock<std::mutex>(h->mu);
  }
};

void holder_release(CtxHolder* h) {
  if (--h->refs == 0) delete h;
}

struct DevBuf {
  CtxHolder* h;
  void* ptr;
  size_t bytes;
};

#define NAPI_OK(call)                                                   \
  do {                                                                  \
    napi_status _s = (call);                                            \
    if (_s != napi_ok) {                                                \
      napi_throw_error(env, nullptr, "N-API call failed: " #call);      \
      return nullptr;                                                   \
    }                                                                   \
  } while (0)

napi_value throw_lf(napi_env env, int rc, const char* what) {
  std::string m = std::string(what) + " failed (" + std::to_string(rc) + "): " + lf_last_error();
  napi_throw_error(env, nullptr, m.c_str());
  return nullptr;
}

// Long runs (the stacks, a Pairformer block) execute on a libuv worker thread through
// napi_async_work: the JS thread gets a promise at once, the worker calls the C entry point
// and waits for the stream, and completion (back on the JS thread) resolves the promise or
// rejects it with the worker's lf_last_error().  The call owns copies of its argument
// structs (plain device pointers and sizes); the JS side keeps the device buffers alive until
// the promise settles.  The worker holds the context's lock for the whole run (CtxHolder).
struct AsyncRun {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  CtxHolder* h = nullptr;
  std::function<int(lf_context*)> fn;
  int rc = LF_OK;
  std::string err;
  const char* what = "";
};

void async_execute(napi_env, void* data) {
  AsyncRun* r = static_cast<AsyncRun*>(data);
  std::lock_guard<std::mutex> g(r->h->mu);
  if (!r->h->alive) {
    r->rc = LF_ERR_INVALID;
    r->err = "the context was destroyed";
    return;
  }
  r->rc = r->fn(r->h->ctx);
  if (r->rc == LF_OK) r->rc = lf_synchronize(r->h->ctx);
  if (r->rc != LF_OK) r->err = lf_last_error();
}

void async_complete(napi_env env, napi_status status, void* data) {
  AsyncRun* r = static_cast<AsyncRun*>(data);
  if (status == napi_ok && r->rc == LF_OK) {
    napi_value u;
    napi_get_undefined(env, &u);
    napi_resolve_deferred(env, r->deferred, u);
  } else {
    const std::string m = status != napi_ok ? std::string(r->what) + ": the async work was cancelled"
                                            : std::string(r->what) + " failed (" + std::to_string(r->rc) + "): " + r->err;
    napi_value msg, e;
    napi_create_string_utf8(env, m.c_str(), NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, nullptr, msg, &e);
    napi_reject_deferred(env, r->deferred, e);
  }
  napi_delete_async_work(env, r->work);
  holder_release(r->h);
  delete r;
}

napi_value start_async(napi_env env, CtxHolder* h, std::function<int(lf_context*)> fn, const char* what) {
  if (!h || !h->alive) {
    napi_throw_error(env, nullptr, "the context was destroyed");
    return nullptr;
  }
  AsyncRun* r = new AsyncRun();
  ++h->refs;   // released in async_complete
  r->h = h;
  r->fn = std::move(fn);
  r->what = what;
  napi_value promise, name;
  if (napi_create_promise(env, &r->deferred, &promise) != napi_ok ||
      napi_create_string_utf8(env, what, NAPI_AUTO_LENGTH, &name) != napi_ok ||
      napi_create_async_work(env, nullptr, name, async_execute, async_complete, r, &r->work) != napi_ok ||
      napi_queue_async_work(env, r->work) != napi_ok) {
    holder_release(h);
    delete r;
    napi_throw_error(env, nullptr, "could not queue the async work");
    return nullptr;
  }
  return promise;
}

void buf_finalize(napi_env, void* data, void*) {
  DevBuf* b = static_cast<DevBuf*>(data);
  {
    CtxGuard g(b->h);
    if (b->ptr && b->h->alive) lf_free(b->h->ctx, b->ptr);
  }
  holder_release(b->h);
  delete b;
}

// a context object collected without contextDestroy releases its device memory here
void ctx_finalize(napi_env, void* data, void*) {
  CtxHolder* h = static_cast<CtxHolder*>(data);
  {
    CtxGuard g(h);
    if (h->alive) {
      lf_context_destroy(h->ctx);
      h->alive = false;
    }
  }
  holder_release(h);
}

DevBuf* new_buf(CtxHolder* h, size_t bytes) {
  ++h->refs;
  return new DevBuf{h, nullptr, bytes};
}

void drop_buf(DevBuf* b) {
  holder_release(b->h);
  delete b;
}

bool get_args(napi_env env, napi_callback_info info, size_t n, napi_value* argv) {
  size_t argc = n;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok) return false;
  return argc >= n;
}

CtxHolder* as_holder(napi_env env, napi_value v) {
  void* p = nullptr;
  napi_get_value_external(env, v, &p);
  return static_cast<CtxHolder*>(p);
}

// NULL once destroyed: every lf_* entry point rejects a NULL context with an error
lf_context* as_ctx(napi_env env, napi_value v) {
  CtxHolder* h = as_holder(env, v);
  return h && h->alive ? h->ctx : nullptr;
}

bool has(napi_env env, napi_value obj, const char* name) {
  bool h = false;
  napi_has_named_property(env, obj, name, &h);
  if (!h) return false;
  napi_value v;
  napi_get_named_property(env, obj, name, &v);
  napi_valuetype t;
  napi_typeof(env, v, &t);
  return t != napi_undefined && t != napi_null;
}

napi_value prop(napi_env env, napi_value obj, const char* name) {
  napi_value v = nullptr;
  napi_get_named_property(env, obj, name, &v);
  return v;
}

int get_int(napi_env env, napi_value obj, const char* name, int dflt = 0) {
  if (!has(env, obj, name)) return dflt;
  int32_t v = dflt;
  napi_get_value_int32(env, prop(env, obj, name), &v);
  return v;
}

double get_num(napi_env env, napi_value obj, const char* name, double dflt) {
  if (!has(env, obj, name)) return dflt;
  double v = dflt;
  napi_get_value_double(env, prop(env, obj, name), &v);
  return v;
}

// a device buffer handle (external) or null
void* get_dev(napi_env env, napi_value obj, const char* name) {
  if (!has(env, obj, name)) return nullptr;
  void* p = nullptr;
  if (napi_get_value_external(env, prop(env, obj, name), &p) != napi_ok || !p) return nullptr;
  return static_cast<DevBuf*>(p)->ptr;
}

int dtype_code(const std::string& s) {
  if (s == "float32") return LF_F32;
  if (s == "float16") return LF_F16;
  if (s == "bfloat16") return LF_BF16;
  if (s == "int8") return LF_INT8;
  if (s == "int5") return LF_INT5;
  return -1;
}

std::string get_str(napi_env env, napi_value obj, const char* name) {
  if (!has(env, obj, name)) return "";
  char buf[64] = {0};
  size_t len = 0;
  napi_get_value_string_utf8(env, prop(env, obj, name), buf, sizeof(buf), &len);
  return std::string(buf, len);
}

// {dtype, layout: "in_out"|"out_in", rows, cols, group, data, scales?, zeros?}
lf_weight get_weight(napi_env env, napi_value obj, const char* name) {
  lf_weight w{};
  if (!has(env, obj, name)) return w;
  napi_value r = prop(env, obj, name);
  w.dtype = dtype_code(get_str(env, r, "dtype"));
  w.layout = get_str(env, r, "layout") == "out_in" ? LF_OUT_IN : LF_IN_OUT;
  w.rows = get_int(env, r, "rows");
  w.cols = get_int(env, r, "cols");
  w.group = get_int(env, r, "group");
  w.data = get_dev(env, r, "data");
  w.scales = get_dev(env, r, "scales");
  w.zeros = get_dev(env, r, "zeros");
  return w;
}

const float* get_vec(napi_env env, napi_value obj, const char* name) {
  return static_cast<const float*>(get_dev(env, obj, name));
}

lf_tri_mult_weights tri_weights(napi_env env, napi_value w) {
  lf_tri_mult_weights t{};
  t.ln_in_scale = get_vec(env, w, "lnInScale");
  t.ln_in_offset = get_vec(env, w, "lnInOffset");
  t.ap = get_weight(env, w, "ap");
  t.ag = get_weight(env, w, "ag");
  t.bp = get_weight(env, w, "bp");
  t.bg = get_weight(env, w, "bg");
  t.ap_bias = get_vec(env, w, "apBias");
  t.ag_bias = get_vec(env, w, "agBias");
  t.bp_bias = get_vec(env, w, "bpBias");
  t.bg_bias = get_vec(env, w, "bgBias");
  t.ln_out_scale = get_vec(env, w, "lnOutScale");
  t.ln_out_offset = get_vec(env, w, "lnOutOffset");
  t.wz = get_weight(env, w, "wz");
  t.wz_bias = get_vec(env, w, "wzBias");
  t.wg = get_weight(env, w, "wg");
  t.wg_bias = get_vec(env, w, "wgBias");
  return t;
}

lf_attention_weights att_weights(napi_env env, napi_value w) {
  lf_attention_weights t{};
  t.norm_scale = get_vec(env, w, "normScale");
  t.norm_offset = get_vec(env, w, "normOffset");
  t.wq = get_weight(env, w, "wq");
  t.wk = get_weight(env, w, "wk");
  t.wv = get_weight(env, w, "wv");
  t.wg = get_weight(env, w, "wg");
  t.wo = get_weight(env, w, "wo");
  t.q_bias = get_vec(env, w, "qBias");
  t.g_bias = get_vec(env, w, "gBias");
  t.o_bias = get_vec(env, w, "oBias");
  t.pair_norm_scale = get_vec(env, w, "pairNormScale");
  t.pair_norm_offset = get_vec(env, w, "pairNormOffset");
  t.wb = get_weight(env, w, "wb");
  return t;
}

lf_transition_weights tr_weights(napi_env env, napi_value w) {
  lf_transition_weights t{};
  t.norm_scale = get_vec(env, w, "normScale");
  t.norm_offset = get_vec(env, w, "normOffset");
  t.w1 = get_weight(env, w, "w1");
  t.b1 = get_vec(env, w, "b1");
  t.w2 = get_weight(env, w, "w2");
  t.b2 = get_vec(env, w, "b2");
  return t;
}

lf_opm_weights opm_w(napi_env env, napi_value w) {
  lf_opm_weights t{};
  t.norm_scale = get_vec(env, w, "normScale");
  t.norm_offset = get_vec(env, w, "normOffset");
  t.wl = get_weight(env, w, "wl");
  t.wr = get_weight(env, w, "wr");
  t.bl = get_vec(env, w, "bl");
  t.br = get_vec(env, w, "br");
  t.wo = get_weight(env, w, "wo");
  t.bo = get_vec(env, w, "bo");
  return t;
}

napi_value undefined_value(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

// ---- context and memory ----------------------------------------------------------------

napi_value ContextCreate(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  int dev = 0;
  if (get_args(env, info, 1, argv)) napi_get_value_int32(env, argv[0], &dev);
  lf_context* ctx = lf_context_create(dev);
  if (!ctx) return throw_lf(env, LF_ERR_DEVICE, "lf_context_create");
  CtxHolder* h = new CtxHolder{ctx, true, 1, {}};
  napi_value ext;
  NAPI_OK(napi_create_external(env, h, ctx_finalize, nullptr, &ext));
  return ext;
}

napi_value ContextDestroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  CtxHolder* h = as_holder(env, argv[0]);
  CtxGuard g(h);
  if (h && h->alive) {
    lf_context_destroy(h->ctx);
    h->alive = false;
  }
  return undefined_value(env);
}

// upload(ctx, typedArrayOrBuffer) -> device buffer handle
napi_value Upload(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) {
    napi_throw_type_error(env, nullptr, "upload(ctx, typedArray)");
    return nullptr;
  }
  CtxGuard guard(as_holder(env, argv[0]));
  lf_context* ctx = as_ctx(env, argv[0]);
  if (!ctx) return throw_lf(env, LF_ERR_INVALID, "upload: the context was destroyed");
  void* data = nullptr;
  size_t bytes = 0;
  bool is_ta = false;
  napi_is_typedarray(env, argv[1], &is_ta);
  if (is_ta) {
    napi_typedarray_type t;
    size_t len, off;
    napi_value ab;
    NAPI_OK(napi_get_typedarray_info(env, argv[1], &t, &len, &data, &ab, &off));
    size_t es = 1;
    switch (t) {
      case napi_int16_array: case napi_uint16_array: es = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
      case napi_float64_array: es = 8; break;
      default: es = 1;
    }
    bytes = len * es;
  } else {
    NAPI_OK(napi_get_buffer_info(env, argv[1], &data, &bytes));
  }
  DevBuf* b = new_buf(as_holder(env, argv[0]), bytes);
  int rc = lf_malloc(ctx, bytes, &b->ptr);
  if (rc != LF_OK) {
    drop_buf(b);
    return throw_lf(env, rc, "lf_malloc");
  }
  if (bytes) {
    rc = lf_memcpy_htod(ctx, b->ptr, data, bytes);
    if (rc != LF_OK) {
      lf_free(ctx, b->ptr);
      drop_buf(b);
      return throw_lf(env, rc, "lf_memcpy_htod");
    }
  }
  napi_value ext;
  NAPI_OK(napi_create_external(env, b, buf_finalize, nullptr, &ext));
  return ext;
}

// alloc(ctx, bytes) -> device buffer handle (uninitialised)
napi_value Alloc(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  CtxGuard guard(as_holder(env, argv[0]));
  lf_context* ctx = as_ctx(env, argv[0]);
  if (!ctx) return throw_lf(env, LF_ERR_INVALID, "alloc: the context was destroyed");
  double bytes = 0;
  napi_get_value_double(env, argv[1], &bytes);
  DevBuf* b = new_buf(as_holder(env, argv[0]), (size_t)bytes);
  int rc = lf_malloc(ctx, b->bytes, &b->ptr);
  if (rc != LF_OK) {
    drop_buf(b);
    return throw_lf(env, rc, "lf_malloc");
  }
  napi_value ext;
  NAPI_OK(napi_create_external(env, b, buf_finalize, nullptr, &ext));
  return ext;
}

// download(ctx, handle, typedArray) copies device -> host (synchronises)
napi_value Download(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return nullptr;
  CtxGuard guard(as_holder(env, argv[0]));
  lf_context* ctx = as_ctx(env, argv[0]);
  if (!ctx) {
    napi_throw_error(env, nullptr, "download: the context was destroyed");
    return nullptr;
  }
  void* p = nullptr;
  if (napi_get_value_external(env, argv[1], &p) != napi_ok || p == nullptr) {
    napi_throw_type_error(env, nullptr, "download: the second argument is not a device buffer handle");
    return nullptr;
  }
  DevBuf* b = static_cast<DevBuf*>(p);
  if (b->ptr == nullptr) {
    napi_throw_error(env, nullptr, "download: the device buffer was freed");
    return nullptr;
  }
  napi_typedarray_type t;
  size_t len, off;
  void* data;
  napi_value ab;
  NAPI_OK(napi_get_typedarray_info(env, argv[2], &t, &len, &data, &ab, &off));
  size_t es = (t == napi_float32_array || t == napi_int32_array || t == napi_uint32_array) ? 4
              : (t == napi_uint16_array || t == napi_int16_array) ? 2 : (t == napi_float64_array ? 8 : 1);
  size_t bytes = len * es;
  if (bytes > b->bytes) {
    napi_throw_range_error(env, nullptr, "download: destination larger than the device buffer");
    return nullptr;
  }
  int rc = lf_memcpy_dtoh(ctx, data, b->ptr, bytes);
  if (rc != LF_OK) return throw_lf(env, rc, "lf_memcpy_dtoh");
  return undefined_value(env);
}

napi_value Free(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  void* p = nullptr;
  napi_get_value_external(env, argv[0], &p);
  DevBuf* b = static_cast<DevBuf*>(p);
  CtxGuard g(b ? b->h : nullptr);
  if (b && b->ptr) {
    if (b->h->alive) lf_free(b->h->ctx, b->ptr);
    b->ptr = nullptr;
  }
  return undefined_value(env);
}

napi_value Synchronize(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  CtxGuard guard(as_holder(env, argv[0]));
  int rc = lf_synchronize(as_ctx(env, argv[0]));
  if (rc != LF_OK) return throw_lf(env, rc, "lf_synchronize");
  return undefined_value(env);
}

napi_value MemoryStats(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  size_t cur = 0, peak = 0, cnt = 0;
  CtxGuard guard(as_holder(env, argv[0]));
  int rc = lf_memory_stats(as_ctx(env, argv[0]), &cur, &peak, &cnt);
  if (rc != LF_OK) return throw_lf(env, rc, "lf_memory_stats");
  napi_value o, v;
  napi_create_object(env, &o);
  napi_create_double(env, (double)cur, &v);
  napi_set_named_property(env, o, "currentBytes", v);
  napi_create_double(env, (double)peak, &v);
  napi_set_named_property(env, o, "peakBytes", v);
  napi_create_double(env, (double)cnt, &v);
  napi_set_named_property(env, o, "allocationCount", v);
  return o;
}

napi_value ProfileEnable(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  bool on = false;
  napi_get_value_bool(env, argv[1], &on);
  CtxGuard guard(as_holder(env, argv[0]));
  lf_profile_enable(as_ctx(env, argv[0]), on ? 1 : 0);
  return undefined_value(env);
}

// profileRead(ctx) -> [{label, ms}]
napi_value ProfileRead(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  const int cap = 4096;
  lf_kernel_timing* recs = static_cast<lf_kernel_timing*>(calloc(cap, sizeof(lf_kernel_timing)));
  CtxGuard guard(as_holder(env, argv[0]));
  int n = lf_profile_read(as_ctx(env, argv[0]), recs, cap);
  napi_value arr;
  napi_create_array_with_length(env, n > 0 ? n : 0, &arr);
  for (int i = 0; i < n; ++i) {
    napi_value o, v;
    napi_create_object(env, &o);
    napi_create_string_utf8(env, recs[i].label, NAPI_AUTO_LENGTH, &v);
    napi_set_named_property(env, o, "label", v);
    napi_create_double(env, recs[i].ms, &v);
    napi_set_named_property(env, o, "ms", v);
    napi_set_element(env, arr, i, o);
  }
  free(recs);
  return arr;
}

napi_value Version(napi_env env, napi_callback_info) {
  napi_value v;
  napi_create_string_utf8(env, lf_version(), NAPI_AUTO_LENGTH, &v);
  return v;
}

// The file the dynamic loader resolved liblocalfold.so to for this process (the library whose
// lf_context_create this addon calls), so a test can check which build ran.
napi_value NativeLibraryPath(napi_env env, napi_callback_info) {
  Dl_info info{};
  napi_value v;
  if (!dladdr(reinterpret_cast<void*>(&lf_context_create), &info) || !info.dli_fname) {
    napi_throw_error(env, nullptr, "dladdr(lf_context_create) failed");
    return nullptr;
  }
  napi_create_string_utf8(env, info.dli_fname, NAPI_AUTO_LENGTH, &v);
  return v;
}

// ---- ops: op(ctx, args) with args mirroring the C structs (camelCase) -------------------

napi_value TriMult(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  napi_value o = argv[1];
  lf_tri_mult_weights w = tri_weights(env, prop(env, o, "weights"));
  lf_tri_mult_args a{};
  a.direction = get_int(env, o, "direction");
  a.dialect = get_int(env, o, "dialect");
  a.divide_by_length = get_int(env, o, "divideByLength");
  a.length = get_int(env, o, "length");
  a.c_z = get_int(env, o, "cZ");
  a.c_hidden = get_int(env, o, "cHidden");
  a.act_dtype = get_int(env, o, "actDtype");
  a.z = get_dev(env, o, "z");
  a.mask = static_cast<const float*>(get_dev(env, o, "mask"));
  a.out = get_dev(env, o, "out");
  a.accumulate = get_int(env, o, "accumulate");
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
  a.w = &w;
  CtxGuard guard(as_holder(env, argv[0]));
  int rc = lf_tri_mult(as_ctx(env, argv[0]), &a);
  if (rc != LF_OK) return throw_lf(env, rc, "lf_tri_mult");
  return undefined_value(env);
}

void fill_attention(napi_env env, napi_value o, lf_attention_args& a) {
  a.batch = get_int(env, o, "batch");
  a.queries = get_int(env, o, "queries");
  a.channels = get_int(env, o, "channels");
  a.heads = get_int(env, o, "heads");
  a.head_dim = get_int(env, o, "headDim");
  a.transpose = get_int(env, o, "transpose");
  a.act_dtype = get_int(env, o, "actDtype");
  a.act = get_dev(env, o, "act");
  a.mask = static_cast<const float*>(get_dev(env, o, "mask"));
  a.out = get_dev(env, o, "out");
  a.accumulate = get_int(env, o, "accumulate");
  a.fast_variance = get_int(env, o, "fastVariance");
  a.bias_mode = get_int(env, o, "biasMode");
  a.swap_bias = get_int(env, o, "swapBias");
  a.pair_dtype = get_int(env, o, "pairDtype");
  a.pair = get_dev(env, o, "pair");
  a.pair_channels = get_int(env, o, "pairChannels");
  a.bias_logits = static_cast<const float*>(get_dev(env, o, "biasLogits"));
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
}

napi_value Attention(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  lf_attention_weights w = att_weights(env, prop(env, argv[1], "weights"));
  lf_attention_args a{};
  fill_attention(env, argv[1], a);
  a.w = &w;
  CtxGuard guard(as_holder(env, argv[0]));
  int rc = lf_attention(as_ctx(env, argv[0]), &a);
  if (rc != LF_OK) return throw_lf(env, rc, "lf_attention");
  return undefined_value(env);
}

napi_value Transition(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  napi_value o = argv[1];
  lf_transition_weights w = tr_weights(env, prop(env, o, "weights"));
  lf_transition_args a{};
  a.kind = get_int(env, o, "kind");
  a.rows = get_int(env, o, "rows");
  a.channels = get_int(env, o, "channels");
  a.hidden = get_int(env, o, "hidden");
  a.act_dtype = get_int(env, o, "actDtype");
  a.act = get_dev(env, o, "act");
  a.out = get_dev(env, o, "out");
  a.accumulate = get_int(env, o, "accumulate");
  a.fast_variance = get_int(env, o, "fastVariance");
  a.chunk_bytes = (long long)get_num(env, o, "chunkBytes", 0);
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
  a.w = &w;
  CtxGuard guard(as_holder(env, argv[0]));
  int rc = lf_transition(as_ctx(env, argv[0]), &a);
  if (rc != LF_OK) return throw_lf(env, rc, "lf_transition");
  return undefined_value(env);
}

napi_value OuterProductMean(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  napi_value o = argv[1];
  lf_opm_weights w = opm_w(env, prop(env, o, "weights"));
  lf_opm_args a{};
  a.sequences = get_int(env, o, "sequences");
  a.length = get_int(env, o, "length");
  a.c_m = get_int(env, o, "cM");
  a.c_outer = get_int(env, o, "cOuter");
  a.c_z = get_int(env, o, "cZ");
  a.msa_dtype = get_int(env, o, "msaDtype");
  a.msa = get_dev(env, o, "msa");
  a.mask = static_cast<const float*>(get_dev(env, o, "mask"));
  a.pair_dtype = get_int(env, o, "pairDtype");
  a.pair_in = get_dev(env, o, "pairIn");
  a.out = get_dev(env, o, "out");
  a.accumulate = get_int(env, o, "accumulate");
  a.fast_variance = get_int(env, o, "fastVariance");
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
  a.norm_epsilon = (float)get_num(env, o, "normEpsilon", 1e-3);
  a.w = &w;
  CtxGuard guard(as_holder(env, argv[0]));
  int rc = lf_outer_product_mean(as_ctx(env, argv[0]), &a);
  if (rc != LF_OK) return throw_lf(env, rc, "lf_outer_product_mean");
  return undefined_value(env);
}

lf_evoformer_weights evo_weights(napi_env env, napi_value w) {
  lf_evoformer_weights e{};
  if (has(env, w, "rowAttention")) {   // absent for the pair halves only
    e.row_attention = att_weights(env, prop(env, w, "rowAttention"));
    e.row_heads = get_int(env, w, "rowHeads");
  }
  if (has(env, w, "columnAttention")) {   // absent in an extra-MSA block
    e.column_attention = att_weights(env, prop(env, w, "columnAttention"));
    e.column_heads = get_int(env, w, "columnHeads");
  }
  if (has(env, w, "msaTransition")) e.msa_transition = tr_weights(env, prop(env, w, "msaTransition"));
  e.outer_product_mean = opm_w(env, prop(env, w, "outerProductMean"));
  e.tri_out = tri_weights(env, prop(env, w, "triOut"));
  e.tri_in = tri_weights(env, prop(env, w, "triIn"));
  e.tri_att_start = att_weights(env, prop(env, w, "triAttStart"));
  e.tri_att_start_heads = get_int(env, w, "triAttStartHeads");
  e.tri_att_end = att_weights(env, prop(env, w, "triAttEnd"));
  e.tri_att_end_heads = get_int(env, w, "triAttEndHeads");
  e.pair_transition = tr_weights(env, prop(env, w, "pairTransition"));
  return e;
}

lf_global_attention_weights glob_weights(napi_env env, napi_value w) {
  lf_global_attention_weights t{};
  t.norm_scale = get_vec(env, w, "normScale");
  t.norm_offset = get_vec(env, w, "normOffset");
  t.wq = get_weight(env, w, "wq");
  t.wk = get_weight(env, w, "wk");
  t.wv = get_weight(env, w, "wv");
  t.wg = get_weight(env, w, "wg");
  t.g_bias = get_vec(env, w, "gBias");
  t.wo = get_weight(env, w, "wo");
  t.o_bias = get_vec(env, w, "oBias");
  return t;
}

napi_value GlobalColumnAttention(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  napi_value o = argv[1];
  lf_global_attention_weights w = glob_weights(env, prop(env, o, "weights"));
  lf_global_attention_args a{};
  a.sequences = get_int(env, o, "sequences");
  a.length = get_int(env, o, "length");
  a.channels = get_int(env, o, "channels");
  a.heads = get_int(env, o, "heads");
  a.head_dim = get_int(env, o, "headDim");
  a.act_dtype = get_int(env, o, "actDtype");
  a.act = get_dev(env, o, "act");
  a.mask = static_cast<const float*>(get_dev(env, o, "mask"));
  a.out = get_dev(env, o, "out");
  a.accumulate = get_int(env, o, "accumulate");
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
  a.w = &w;
  CtxGuard guard(as_holder(env, argv[0]));
  int rc = lf_global_column_attention(as_ctx(env, argv[0]), &a);
  if (rc != LF_OK) return throw_lf(env, rc, "lf_global_column_attention");
  return undefined_value(env);
}

lf_evoformer_block_args evo_args(napi_env env, napi_value o) {
  lf_evoformer_block_args a{};
  a.sequences = get_int(env, o, "sequences");
  a.length = get_int(env, o, "length");
  a.c_m = get_int(env, o, "cM");
  a.c_z = get_int(env, o, "cZ");
  a.c_outer = get_int(env, o, "cOuter");
  a.tri_hidden = get_int(env, o, "triangleHidden");
  a.msa_hidden = get_int(env, o, "msaHidden");
  a.pair_hidden = get_int(env, o, "pairHidden");
  a.msa_dtype = get_int(env, o, "msaDtype");
  a.msa = get_dev(env, o, "msa");
  a.pair_dtype = get_int(env, o, "pairDtype");
  a.pair = get_dev(env, o, "pair");
  a.msa_mask = static_cast<const float*>(get_dev(env, o, "msaMask"));
  a.pair_mask = static_cast<const float*>(get_dev(env, o, "pairMask"));
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
  return a;
}

// evoformerStack(ctx, args, [blockWeights...]) - one block when the array has length 1
napi_value EvoformerStack(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return nullptr;
  lf_evoformer_block_args a = evo_args(env, argv[1]);
  uint32_t n = 0;
  napi_get_array_length(env, argv[2], &n);
  std::vector<lf_evoformer_weights> ws(n > 0 ? n : 1);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, argv[2], i, &e);
    ws[i] = evo_weights(env, e);
  }
  // returns a promise: the stack runs on a worker thread (see start_async)
  return start_async(env, as_holder(env, argv[0]), [a, ws, n](lf_context* c) {
    return lf_evoformer_stack(c, &a, ws.data(), (int)n);
  }, "lf_evoformer_stack");
}

// evoformerPairStack(ctx, args, [blockWeights...]): the pair halves only (msa read, not written)
napi_value EvoformerPairStack(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return nullptr;
  lf_evoformer_block_args a = evo_args(env, argv[1]);
  uint32_t n = 0;
  napi_get_array_length(env, argv[2], &n);
  std::vector<lf_evoformer_weights> ws(n > 0 ? n : 1);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, argv[2], i, &e);
    ws[i] = evo_weights(env, e);
  }
  return start_async(env, as_holder(env, argv[0]), [a, ws, n](lf_context* c) {
    return lf_evoformer_pair_stack(c, &a, ws.data(), (int)n);
  }, "lf_evoformer_pair_stack");
}

// extraMsaStack(ctx, args, [blockWeights...]): Evoformer block weights with columnGlobal
napi_value ExtraMsaStack(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return nullptr;
  lf_evoformer_block_args a = evo_args(env, argv[1]);
  uint32_t n = 0;
  napi_get_array_length(env, argv[2], &n);
  std::vector<lf_extra_msa_weights> ws(n > 0 ? n : 1);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, argv[2], i, &e);
    ws[i].base = evo_weights(env, e);
    ws[i].column_global = glob_weights(env, prop(env, e, "columnGlobal"));
    ws[i].column_global_heads = get_int(env, e, "columnGlobalHeads");
  }
  // returns a promise: the stack runs on a worker thread (see start_async)
  return start_async(env, as_holder(env, argv[0]), [a, ws, n](lf_context* c) {
    return lf_extra_msa_stack(c, &a, ws.data(), (int)n);
  }, "lf_extra_msa_stack");
}

napi_value PairformerBlock(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  napi_value o = argv[1];
  napi_value wv = prop(env, o, "weights");
  lf_pairformer_weights w{};
  w.tri_out = tri_weights(env, prop(env, wv, "triOut"));
  w.tri_in = tri_weights(env, prop(env, wv, "triIn"));
  w.att_start = att_weights(env, prop(env, wv, "attStart"));
  w.att_end = att_weights(env, prop(env, wv, "attEnd"));
  w.pair_heads = get_int(env, wv, "pairHeads");
  w.pair_transition = tr_weights(env, prop(env, wv, "pairTransition"));
  w.single_logits_norm_scale = get_vec(env, wv, "singleLogitsNormScale");
  w.single_logits_norm_offset = get_vec(env, wv, "singleLogitsNormOffset");
  w.single_logits_projection = get_weight(env, wv, "singleLogitsProjection");
  if (has(env, wv, "singleAttention")) w.single_attention = att_weights(env, prop(env, wv, "singleAttention"));
  w.single_heads = get_int(env, wv, "singleHeads");
  w.single_head_dim = get_int(env, wv, "singleHeadDim");
  if (has(env, wv, "singleTransition")) w.single_transition = tr_weights(env, prop(env, wv, "singleTransition"));
  lf_pairformer_block_args a{};
  a.tokens = get_int(env, o, "tokens");
  a.c_z = get_int(env, o, "cZ");
  a.c_s = get_int(env, o, "cS");
  a.swap_transposed_bias = get_int(env, o, "swapTransposedBias");
  a.divide_by_length = get_int(env, o, "divideByLength");
  a.pair_dtype = get_int(env, o, "pairDtype");
  a.pair = get_dev(env, o, "pair");
  a.single_dtype = get_int(env, o, "singleDtype");
  a.single = get_dev(env, o, "single");
  a.pair_mask = static_cast<const float*>(get_dev(env, o, "pairMask"));
  a.seq_mask = static_cast<const float*>(get_dev(env, o, "seqMask"));
  a.transition_chunk_bytes = (long long)get_num(env, o, "transitionChunkBytes", 0);
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
  // returns a promise: the block runs on a worker thread (see start_async)
  return start_async(env, as_holder(env, argv[0]), [a, w](lf_context* c) {
    lf_pairformer_block_args args = a;
    args.w = &w;
    return lf_pairformer_block(c, &args);
  }, "lf_pairformer_block");
}

// msaModuleBlock(ctx, args): one AF3 MSA-module block, weights {opm, cOuter, pwa, msaHeads,
// msaHeadDim, msaTransition, pair: {triOut, triIn, attStart, attEnd, pairHeads, pairTransition}}
napi_value MsaModuleBlock(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  napi_value o = argv[1];
  napi_value wv = prop(env, o, "weights");
  lf_msa_module_weights w{};
  w.outer_product_mean = opm_w(env, prop(env, wv, "opm"));
  w.c_outer = get_int(env, wv, "cOuter");
  napi_value pv = prop(env, wv, "pwa");
  w.msa_attention.act_norm_scale = get_vec(env, pv, "actNormScale");
  w.msa_attention.act_norm_offset = get_vec(env, pv, "actNormOffset");
  w.msa_attention.pair_norm_scale = get_vec(env, pv, "pairNormScale");
  w.msa_attention.pair_norm_offset = get_vec(env, pv, "pairNormOffset");
  w.msa_attention.pair_logits = get_weight(env, pv, "pairLogits");
  w.msa_attention.wv = get_weight(env, pv, "wv");
  w.msa_attention.wg = get_weight(env, pv, "wg");
  w.msa_attention.wo = get_weight(env, pv, "wo");
  w.msa_heads = get_int(env, wv, "msaHeads");
  w.msa_head_dim = get_int(env, wv, "msaHeadDim");
  w.msa_transition = tr_weights(env, prop(env, wv, "msaTransition"));
  napi_value q = prop(env, wv, "pair");
  w.pair.tri_out = tri_weights(env, prop(env, q, "triOut"));
  w.pair.tri_in = tri_weights(env, prop(env, q, "triIn"));
  w.pair.att_start = att_weights(env, prop(env, q, "attStart"));
  w.pair.att_end = att_weights(env, prop(env, q, "attEnd"));
  w.pair.pair_heads = get_int(env, q, "pairHeads");
  w.pair.pair_transition = tr_weights(env, prop(env, q, "pairTransition"));
  lf_msa_block_args a{};
  a.sequences = get_int(env, o, "sequences");
  a.tokens = get_int(env, o, "tokens");
  a.c_m = get_int(env, o, "cM");
  a.c_z = get_int(env, o, "cZ");
  a.msa_update_before_opm = get_int(env, o, "msaUpdateBeforeOuterProduct");
  a.swap_transposed_bias = get_int(env, o, "swapTransposedBias");
  a.divide_by_length = get_int(env, o, "divideByLength");
  a.msa_dtype = get_int(env, o, "msaDtype");
  a.msa = get_dev(env, o, "msa");
  a.pair_dtype = get_int(env, o, "pairDtype");
  a.pair = get_dev(env, o, "pair");
  a.msa_mask = static_cast<const float*>(get_dev(env, o, "msaMask"));
  a.pair_mask = static_cast<const float*>(get_dev(env, o, "pairMask"));
  a.transition_chunk_bytes = (long long)get_num(env, o, "transitionChunkBytes", 0);
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
  // returns a promise: the block runs on a worker thread (see start_async)
  return start_async(env, as_holder(env, argv[0]), [a, w](lf_context* c) {
    lf_msa_block_args args = a;
    args.w = &w;
    return lf_msa_module_block(c, &args);
  }, "lf_msa_module_block");
}

// inputEmbedder(ctx, args): device pointers for every feature, weight and output
napi_value InputEmbedder(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  napi_value o = argv[1];
  napi_value wv = prop(env, o, "weights");
  lf_input_embedder_weights w{};
  const struct { const float** dst; const char* name; } ws[] = {
      {&w.preprocess_1d_w, "preprocess1dWeight"}, {&w.preprocess_1d_b, "preprocess1dBias"},
      {&w.preprocess_msa_w, "preprocessMsaWeight"}, {&w.preprocess_msa_b, "preprocessMsaBias"},
      {&w.left_w, "leftSingleWeight"}, {&w.left_b, "leftSingleBias"}, {&w.right_w, "rightSingleWeight"},
      {&w.right_b, "rightSingleBias"}, {&w.prev_pos_w, "previousPositionWeight"},
      {&w.prev_pos_b, "previousPositionBias"}, {&w.prev_msa_norm_scale, "previousMsaNormScale"},
      {&w.prev_msa_norm_offset, "previousMsaNormOffset"}, {&w.prev_pair_norm_scale, "previousPairNormScale"},
      {&w.prev_pair_norm_offset, "previousPairNormOffset"}, {&w.relpos_w, "relativePositionWeight"},
      {&w.relpos_b, "relativePositionBias"}, {&w.extra_w, "extraMsaWeight"}, {&w.extra_b, "extraMsaBias"},
  };
  for (const auto& e : ws) *e.dst = get_vec(env, wv, e.name);
  lf_input_embedder_args a{};
  a.length = get_int(env, o, "length");
  a.msa_sequences = get_int(env, o, "msaSequences");
  a.extra_sequences = get_int(env, o, "extraSequences");
  a.target_channels = get_int(env, o, "targetChannels");
  a.msa_feature_channels = get_int(env, o, "msaFeatureChannels");
  a.c_m = get_int(env, o, "msaChannels");
  a.c_z = get_int(env, o, "pairChannels");
  a.c_e = get_int(env, o, "extraMsaChannels");
  a.target_feat = static_cast<const float*>(get_dev(env, o, "targetFeatures"));
  a.msa_feat = static_cast<const float*>(get_dev(env, o, "msaFeatures"));
  a.extra_msa = static_cast<const float*>(get_dev(env, o, "extraMsa"));
  a.extra_has_deletion = static_cast<const float*>(get_dev(env, o, "extraHasDeletion"));
  a.extra_deletion_value = static_cast<const float*>(get_dev(env, o, "extraDeletionValue"));
  a.residue_index = static_cast<const float*>(get_dev(env, o, "residueIndex"));
  a.aatype = static_cast<const float*>(get_dev(env, o, "aatype"));
  a.prev_msa_first_row = get_dev(env, o, "previousMsaFirstRow");
  a.prev_pair = get_dev(env, o, "previousPair");
  a.prev_positions = static_cast<const float*>(get_dev(env, o, "previousPositions"));
  a.msa_dtype = a.pair_dtype = a.extra_dtype = LF_F32;
  a.msa = get_dev(env, o, "msa");
  a.pair = get_dev(env, o, "pair");
  a.extra = get_dev(env, o, "extra");
  a.epsilon = (float)get_num(env, o, "epsilon", 1e-5);
  a.w = &w;
  CtxGuard guard(as_holder(env, argv[0]));
  int rc = lf_input_embedder(as_ctx(env, argv[0]), &a);
  if (rc != LF_OK) return throw_lf(env, rc, "lf_input_embedder");
  return undefined_value(env);
}

napi_value Init(napi_env env, napi_value exports) {
  const struct {
    const char* name;
    napi_callback fn;
  } fns[] = {
      {"contextCreate", ContextCreate}, {"contextDestroy", ContextDestroy}, {"upload", Upload},
      {"alloc", Alloc}, {"download", Download}, {"free", Free}, {"synchronize", Synchronize},
      {"memoryStats", MemoryStats}, {"profileEnable", ProfileEnable}, {"profileRead", ProfileRead},
      {"version", Version}, {"nativeLibraryPath", NativeLibraryPath}, {"triMult", TriMult}, {"attention", Attention}, {"transition", Transition},
      {"outerProductMean", OuterProductMean}, {"evoformerStack", EvoformerStack}, {"evoformerPairStack", EvoformerPairStack},
      {"pairformerBlock", PairformerBlock}, {"globalColumnAttention", GlobalColumnAttention},
      {"extraMsaStack", ExtraMsaStack}, {"msaModuleBlock", MsaModuleBlock}, {"inputEmbedder", InputEmbedder},
  };
  for (const auto& f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
