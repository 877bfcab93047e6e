// Weight expansion: the codec records of an op (f32 / f16 / bf16 / int8 / int5, flat-group or
// per-output-channel tables) decoded on the device into f16 E[n][k] tiles in the workspace,
// once per op call.  The decode is the reference's readTensorRange arithmetic
// (shared/weights/dtype.js:212-406): code*scale for int8, fma(code, scale, zero) for int5,
// exact in float32 before the f16 rounding the MFMA operand needs.
#include "lf_gemm.h"
#include "lf_ops.h"

namespace lf {

// One thread per run of 8 stored weights (wrun_fetch / wrun_decode): along k, 8 values of one
// destination row in one 16-byte store; along n ((in,out) storage, consecutive threads on
// consecutive k, so each of the 8 row stores is coalesced), 8 rows of one column k.  Column n
// goes to row (n / W) * 64 + off + n % W; runs along n never straddle a W group (W is a
// multiple of 8 for such views).
__global__ __launch_bounds__(256) void expand_weights_kernel(ExpandBatch b) {
  const int m = blockIdx.y;
  if (m >= b.count) return;
  const WView& v = b.v[m];
  const int kp = b.kp[m], W = b.W[m], off = b.off[m];
  const float sc = b.scale[m];
  const bool krun = v.run != WRUN_N;
  const int per = krun ? kp >> 3 : kp;
  const long total = krun ? (long)b.ncols[m] * per : (long)((b.ncols[m] + 7) >> 3) * kp;
  _Float16* dst = b.dst[m];
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < total; e += (long)gridDim.x * 256) {
    const int q = (int)(e / per), r = (int)(e - (long)q * per);
    const int n = krun ? q : 8 * q, k = krun ? 8 * r : r;
    const h8 h = wrun_decode(v, wrun_fetch(v, k, n, sc), k, n, sc);
    const long row = (long)(n / W) * 64 + off + n % W;
    if (krun) {
      *reinterpret_cast<h8*>(dst + row * kp + k) = h;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (n + j < b.ncols[m]) dst[(row + j) * kp + k] = h[j];
    }
  }
}

int expand_flush(lf_context* ctx, ExpandList& l, const char* label) {
  if (l.b.count == 0) return LF_OK;
  {
    LaunchScope ls(ctx, label);
    dim3 grid((unsigned)std::min<long>(std::max<long>((l.most / 8 + 255) / 256, 1), 1024), l.b.count);
    hipLaunchKernelGGL(expand_weights_kernel, grid, dim3(256), 0, ctx->stream, l.b);
  }
  l = ExpandList{};
  return check_hip(hipGetLastError(), "expand launch");
}

static int expand_add(lf_context* ctx, ExpandList& l, const WView& v, _Float16* dst, int kp, int W, int off, int ncols,
                      float scale, const char* label) {
  if (l.b.count == 8) LF_TRY(expand_flush(ctx, l, label));
  const int i = l.b.count++;
  l.b.v[i] = v;
  l.b.dst[i] = dst;
  l.b.kp[i] = kp;
  l.b.W[i] = W;
  l.b.off[i] = off;
  l.b.ncols[i] = ncols;
  l.b.scale[i] = scale;
  l.most = std::max(l.most, (long)ncols * kp);
  return LF_OK;
}

int expand_add_plain(lf_context* ctx, ExpandList& l, const WView& v, void* dst, WExp* out, float scale,
                     const char* label) {
  const int kp = (v.K + 31) & ~31;
  *out = WExp{static_cast<_Float16*>(dst), kp, v.N};
  return expand_add(ctx, l, v, static_cast<_Float16*>(dst), kp, std::max(v.N, 1), 0, v.N, scale, label);
}

int expand_add_packed(lf_context* ctx, ExpandList& l, const WView* views, const int* W, const int* off,
                      const long long* row0, int count, _Float16* dst, int kp, const char* label) {
  for (int m = 0; m < count; ++m)
    LF_TRY(expand_add(ctx, l, views[m], dst + row0[m] * kp, kp, W[m], off[m], (views[m].N + W[m] - 1) / W[m] * W[m],
                      1.f, label));
  return LF_OK;
}

int expand_weights(lf_context* ctx, const WView* views, int count, void* const* dst, WExp* out, const char* label,
                   const float* scales) {
  ExpandList l;
  for (int i = 0; i < count; ++i)
    LF_TRY(expand_add_plain(ctx, l, views[i], dst[i], &out[i], scales ? scales[i] : 1.f, label));
  return expand_flush(ctx, l, label);
}

int expand_packed(lf_context* ctx, const WView* views, const int* W, const int* off, const long long* row0,
                  int count, _Float16* dst, int kp, const char* label) {
  ExpandList l;
  LF_TRY(expand_add_packed(ctx, l, views, W, off, row0, count, dst, kp, label));
  return expand_flush(ctx, l, label);
}

// dst = (f16) (scale * src), n elements; with tq > 0 every [tq][tq] plane is transposed.
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float* src, _Float16* dst, long long n, int tq,
                                                         float scale, int rowlen, int ld) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    long long s = i;
    if (tq > 0) {
      const long long plane = (long long)tq * tq, pl = i / plane, r = i % plane;
      s = pl * plane + (r % tq) * tq + r / tq;
    }
    const long long o = ld > 0 ? (i / rowlen) * ld + i % rowlen : i;
    dst[o] = (_Float16)(scale * src[s]);
  }
}

int f32_to_f16(lf_context* ctx, const float* src, _Float16* dst, long long n, int tq, float scale, int rowlen,
               int ld) {
  LaunchScope ls(ctx, "convert.f16");
  const long long blocks = std::min<long long>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)std::max<long long>(blocks, 1)), dim3(256), 0, ctx->stream,
                     src, dst, n, tq, scale, rowlen, ld);
  return check_hip(hipGetLastError(), "f32_to_f16 launch");
}

size_t expanded_bytes(const WView& v) { return (size_t)v.N * ((v.K + 31) & ~31) * sizeof(_Float16); }

}  // namespace lf
