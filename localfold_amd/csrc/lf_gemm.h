// Shared MFMA tile machinery: weight staging into LDS (from an f16 expansion, or decoded from
// the stored codes inside the kernel) and the 16-row x (16*NT)-column wave tile over an
// LDS-resident A block.
//
// LDS layouts (f16, row stride padded by 8 halves so the 16-byte fragment reads of 16
// consecutive rows land in different banks):
//   A:  As[row][k]      rows of the block's activation tile, k contiguous
//   W:  Ws[n][k]        one column chunk of the logical weight matrix, k contiguous
// MFMA v_mfma_f32_16x16x32_f16: lane l supplies A[l%16][8*(l/16) .. +8) and
// B[8*(l/16) .. +8)[l%16]; the result lane l holds D[4*(l/16)+i][l%16], i = 0..3.
#pragma once
#include "lf_common.h"

namespace lf {

// Expanded weights: one matrix decoded to f16 as E[n][k] (k contiguous, row pitch kp,
// zero past K), written once per op call by expand_weights_kernel into the workspace;
// the GEMM blocks copy their column chunks from it with 16-byte loads.
struct WExp {
  const _Float16* p;
  int kp;   // row pitch = K rounded up to 32
  int N;    // valid columns
};

// Up to 8 matrices decoded per launch.  Matrix m's column n lands in destination row
// (n / W) * 64 + off + n % W with row pitch `kp` (plain expansion: W = N, off = 0); `ncols`
// columns are written, those >= N as zeros.
struct ExpandBatch {
  WView v[8];
  _Float16* dst[8];
  int kp[8];
  int W[8], off[8], ncols[8];
  float scale[8];   // multiplies the decoded value before the f16 rounding
  int count;
};

// ---- in-kernel dequantisation ----------------------------------------------------------
// A run is 8 stored weights adjacent in memory (WView::run): k..k+7 of column n (WRUN_K) or
// columns n..n+7 at k (WRUN_N).  wrun_fetch issues its loads -- codes and the group's scale
// and zero exactly as stored, no arithmetic on them, so a prefetch never waits -- and
// wrun_decode turns the words into 8 f16 values when they are written to LDS.  The decode is
// the reference's readTensorRange arithmetic (shared/weights/dtype.js:212-406): int8
// code * scale, int5 fma(code, scale, zero) with codes LSB-first at bit 5i, in f32, with the
// kernel's factor `mul` folded into scale and zero (1 for the reference's own weights),
// rounded once to f16.  f32 weights are converted at fetch (they are not a codec).
// Coordinates outside the view are clamped for the fetch and decode to zeros.
struct WRunAt {
  int flat;   // flat index of the run's first stored weight (clamped)
  int grp;    // its group (scale / zero index)
  bool ok;    // inside the view
};

__device__ __forceinline__ WRunAt wrun_at(const WView& w, int k, int n) {
  WRunAt r;
  r.ok = k < w.K && n < w.N;
  const int kc = k < w.K ? k : 0, nc = n < w.N ? n : 0;
  const int np = w.col_off + nc * w.col_stride;
  r.flat = kc * w.ld_k + np * w.ld_n;
  r.grp = w.group > 0 ? r.flat >> w.gshift : np;
  return r;
}

// Views without runs (interleaved columns, tiny or unaligned matrices): the 8 weights
// k..k+7 of column n decoded one by one at fetch (out of line: rare, and it keeps the
// generic decoder's code out of the kernels' loops).
__device__ __noinline__ u32x4 wrun_gather(WView w, int k, int n, float mul) {
  h8 h;
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = (_Float16)(mul * wdecode(w, k + j, n));
  u32x4 v;
  __builtin_memcpy(&v, &h, 16);
  return v;
}

// The fetch and decode of one stored dtype (a compile-time constant): straight-line code for
// callers that know every view they stage has that dtype.
template <int DT>
__device__ __forceinline__ u32x4 wrun_fetch_dt(const WView& w, const WRunAt& r, float mul) {
  u32x4 v;
  if constexpr (DT == DT_F32) {
    const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(w.data) + r.flat);
    const float4 a = src[0], b = src[1];
    h8 h;
    h[0] = (_Float16)(mul * a.x); h[1] = (_Float16)(mul * a.y); h[2] = (_Float16)(mul * a.z); h[3] = (_Float16)(mul * a.w);
    h[4] = (_Float16)(mul * b.x); h[5] = (_Float16)(mul * b.y); h[6] = (_Float16)(mul * b.z); h[7] = (_Float16)(mul * b.w);
    __builtin_memcpy(&v, &h, 16);
  } else if constexpr (DT == DT_F16 || DT == DT_BF16) {
    v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(w.data) + r.flat);
  } else if constexpr (DT == DT_I8) {
    const uint2 c = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(w.data) + r.flat);
    v = u32x4{c.x, c.y, (uint32_t)w.scales[r.grp], 0u};
  } else {   // int5: the run is the 5 bytes at 5 * flat / 8, inside two aligned words
    const uint8_t* b = static_cast<const uint8_t*>(w.data) + (((r.flat >> 3) * 5) & ~3);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(b);
    v = u32x4{q[0], q[1], (uint32_t)w.scales[r.grp], (uint32_t)w.zeros[r.grp]};
  }
  return v;
}

template <int DT>
__device__ __forceinline__ h8 wrun_decode_dt(const u32x4& v, const WRunAt& r, float mul) {
  h8 h;
  if constexpr (DT == DT_F32) {   // converted at fetch
    __builtin_memcpy(&h, &v, 16);
  } else if constexpr (DT == DT_F16) {
    __builtin_memcpy(&h, &v, 16);
    if (mul != 1.f) {
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = (_Float16)(mul * (float)h[j]);
    }
  } else if constexpr (DT == DT_BF16) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t word = v[j >> 1];
      h[j] = (_Float16)(mul * __uint_as_float((j & 1) ? (word & 0xffff0000u) : (word << 16)));
    }
  } else if constexpr (DT == DT_I8) {
    // `mul` folded into the scale (and zero): one product per run instead of per weight
    const float sc = mul * h2f((uint16_t)v.z);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int code = (int)(int8_t)(((j < 4 ? v.x : v.y) >> (8 * (j & 3))) & 0xffu);
      h[j] = (_Float16)((float)code * sc);
    }
  } else {
    const float sc = mul * h2f((uint16_t)v.z), zp = mul * h2f((uint16_t)v.w);
    const int sh = (((r.flat >> 3) * 5) & 3) * 8;
    const uint64_t x = (((uint64_t)v.y << 32) | v.x) >> sh;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (_Float16)fmaf((float)((uint32_t)(x >> (5 * j)) & 31u), sc, zp);
  }
  if (!r.ok) h = h8{0, 0, 0, 0, 0, 0, 0, 0};
  return h;
}

// GATHER = false: the caller guarantees w.run != WRUN_GATHER (kernels are instantiated
// without the out-of-line call, which costs registers even where it is never taken).
template <bool GATHER = true>
__device__ __forceinline__ u32x4 wrun_fetch(const WView& w, int k, int n, float mul) {
  if (GATHER && w.run == WRUN_GATHER) return wrun_gather(w, k, n, mul);
  const WRunAt r = wrun_at(w, k, n);
  switch (w.dtype) {
    case DT_F32: return wrun_fetch_dt<DT_F32>(w, r, mul);
    case DT_F16: return wrun_fetch_dt<DT_F16>(w, r, mul);
    case DT_BF16: return wrun_fetch_dt<DT_BF16>(w, r, mul);
    case DT_I8: return wrun_fetch_dt<DT_I8>(w, r, mul);
    default: return wrun_fetch_dt<DT_I5>(w, r, mul);
  }
}

template <bool GATHER = true>
__device__ __forceinline__ h8 wrun_decode(const WView& w, const u32x4& v, int k, int n, float mul) {
  const WRunAt r = wrun_at(w, k, n);
  switch (GATHER && w.run == WRUN_GATHER ? DT_F32 : w.dtype) {
    case DT_F32: return wrun_decode_dt<DT_F32>(v, r, mul);   // a gathered run is converted at fetch
    case DT_F16: return wrun_decode_dt<DT_F16>(v, r, mul);
    case DT_BF16: return wrun_decode_dt<DT_BF16>(v, r, mul);
    case DT_I8: return wrun_decode_dt<DT_I8>(v, r, mul);
    default: return wrun_decode_dt<DT_I5>(v, r, mul);
  }
}

// Writes a decoded run to Ws[n][k] (pitch ldw halves): one 16-byte store for a run along k
// at (n, k..k+7), eight 2-byte stores down the rows for a run along n at (n..n+7, k).
__device__ __forceinline__ void wrun_put(_Float16* Ws, int ldw, bool krun, int n, int k, const h8& h) {
  if (krun) {
    *reinterpret_cast<h8*>(Ws + n * ldw + k) = h;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) Ws[(n + j) * ldw + k] = h[j];
  }
}

// Ws[n][k] = mul * W[k][n_base + n] for n < ncols, k < kpad (zeros outside the view), decoded
// from the stored runs; ncols and kpad multiples of 8.  Runs are taken four at a time so their
// loads overlap.
__device__ __forceinline__ void stage_view(_Float16* Ws, int ldw, const WView& w, int ncols, int n_base, int kpad,
                                           float mul, int tid, int nthreads) {
  const bool krun = w.run != WRUN_N;
  const int runs = ncols * kpad / 8;
  const int per = krun ? kpad >> 3 : kpad;   // runs per LDS row (krun) or per 8-row band
  for (int i0 = tid; i0 < runs; i0 += 4 * nthreads) {
    u32x4 v[4];
    int nn[4], kk[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(i0 + u * nthreads, runs - 1);
      const int q = i / per, m = i - q * per;
      nn[u] = krun ? q : 8 * q;
      kk[u] = krun ? 8 * m : m;
      v[u] = wrun_fetch(w, kk[u], n_base + nn[u], mul);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i0 + u * nthreads < runs)
        wrun_put(Ws, ldw, krun, nn[u], kk[u], wrun_decode(w, v[u], kk[u], n_base + nn[u], mul));
    }
  }
}

// acc[r][t] += A[row0 + 16r .. +16][0..kloop) * Ws[16t .. +16][0..kloop)^T
template <int RF, int NT>
__device__ __forceinline__ void wave_tile_mfma(f4 (&acc)[RF][NT], const _Float16* As, int lda, int row0,
                                               const _Float16* Ws, int ldw, int kloop, int lane) {
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  for (int kk = 0; kk < kloop; kk += 32) {
    h8 a[RF];
#pragma unroll
    for (int r = 0; r < RF; ++r) a[r] = *reinterpret_cast<const h8*>(As + (row0 + r * 16 + r16) * lda + kk + kq);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const h8 b = *reinterpret_cast<const h8*>(Ws + (t * 16 + r16) * ldw + kk + kq);
#pragma unroll
      for (int r = 0; r < RF; ++r) acc[r][t] = mfma16(a[r], b, acc[r][t]);
    }
  }
}

template <int RF, int NT>
__device__ __forceinline__ void zero_acc(f4 (&acc)[RF][NT]) {
#pragma unroll
  for (int r = 0; r < RF; ++r)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[r][t] = f4{0.f, 0.f, 0.f, 0.f};
}

}  // namespace lf
