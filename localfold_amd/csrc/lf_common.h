// Device-side building blocks shared by every localfold HIP kernel (gfx950 / CDNA4).
//
//  * activation storage types (f32 / f16 / bf16) and their conversions
//  * the weight view: one (stored) weight tensor seen as a logical K x N matrix, decoded
//    element by element from f32 / f16 / bf16 / int8 (symmetric, fp16 scale) / int5
//    (asymmetric, LSB-first packed, fp16 scale + zero) - the codecs of
//    shared/weights/dtype.js:212-406 - with either the flat group map
//    (group = flat_index / block) or one group per stored output column
//  * wave-wide reductions, the LayerNorm row helper and the 16x16x32 f16 MFMA tile loop
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lf {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum DType { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_I8 = 3, DT_I5 = 4 };

constexpr int WAVE = 64;

__device__ __forceinline__ float h2f(uint16_t bits) {
  _Float16 h;
  __builtin_memcpy(&h, &bits, 2);
  return (float)h;
}

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Round-to-nearest-even float -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float load_act(const void* p, int dt, size_t i) {
  if (dt == DT_F32) return static_cast<const float*>(p)[i];
  if (dt == DT_F16) return (float)static_cast<const _Float16*>(p)[i];
  return bf2f(static_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ void store_act(void* p, int dt, size_t i, float v) {
  if (dt == DT_F32) static_cast<float*>(p)[i] = v;
  else if (dt == DT_F16) static_cast<_Float16*>(p)[i] = (_Float16)v;
  else static_cast<uint16_t*>(p)[i] = f2bf(v);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// A stored weight tensor seen as a logical matrix W[k][n], k < K, n < N.
// flat stored index = k*ld_k + nphys*ld_n, nphys = col_off + n*col_stride.
struct WView {
  const void* data;
  const uint16_t* scales;   // fp16 bits, one per group
  const uint16_t* zeros;    // fp16 bits, one per group (int5)
  int dtype;
  int group;                // > 0: flat group size; 0: one group per stored output column (nphys)
  int ld_k, ld_n;
  int col_off, col_stride;
  int K, N;
};

__device__ __forceinline__ float wdecode(const WView& w, int k, int n) {
  if (k >= w.K || n >= w.N) return 0.f;
  const int np = w.col_off + n * w.col_stride;
  const long idx = (long)k * w.ld_k + (long)np * w.ld_n;
  switch (w.dtype) {
    case DT_F32: return static_cast<const float*>(w.data)[idx];
    case DT_F16: return (float)static_cast<const _Float16*>(w.data)[idx];
    case DT_BF16: return bf2f(static_cast<const uint16_t*>(w.data)[idx]);
    case DT_I8: {
      const long g = w.group > 0 ? idx / w.group : np;
      return (float)static_cast<const int8_t*>(w.data)[idx] * h2f(w.scales[g]);
    }
    default: {  // DT_I5: code i starts at bit 5*i; two bytes always cover it (one slack byte).
      const long g = w.group > 0 ? idx / w.group : np;
      const uint8_t* b = static_cast<const uint8_t*>(w.data);
      const long bit = idx * 5;
      const uint32_t pair = (uint32_t)b[bit >> 3] | ((uint32_t)b[(bit >> 3) + 1] << 8);
      const float code = (float)((pair >> (bit & 7)) & 31u);
      return fmaf(code, h2f(w.scales[g]), h2f(w.zeros[g]));
    }
  }
}

// True when consecutive k of one logical column are adjacent in storage.
__device__ __forceinline__ bool wview_k_contiguous(const WView& w) { return w.ld_k == 1; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}


__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// LayerNorm of one row of C <= 256 channels by one wave; writes f16 to dst[0..KPAD)
// (zero past C).  Two-pass statistics (mean, then mean squared deviation) as
// webgpu/kernels/triangle/cpu-reference.js:5-29, or E[x^2]-E[x]^2 when fast_var
// (cpu/af3/trunk/pairformer.js:68-87).
template <int KPAD>
__device__ __forceinline__ void ln_row_to_lds(_Float16* dst, const void* src, int dt, size_t base, int C,
                                              const float* gamma, const float* beta, float eps, bool fast_var,
                                              int lane) {
  constexpr int PER = (KPAD + WAVE - 1) / WAVE;
  float v[PER];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = lane + j * WAVE;
    v[j] = c < C ? load_act(src, dt, base + c) : 0.f;
    s += v[j];
  }
  s = wave_sum(s);
  const float mean = s / (float)C;
  float q = 0.f;
  if (fast_var) {
#pragma unroll
    for (int j = 0; j < PER; ++j) q += v[j] * v[j];
    q = wave_sum(q);
    q = q / (float)C - mean * mean;
  } else {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = lane + j * WAVE;
      const float d = c < C ? v[j] - mean : 0.f;
      q += d * d;
    }
    q = wave_sum(q) / (float)C;
  }
  const float inv = 1.0f / sqrtf(q + eps);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = lane + j * WAVE;
    if (c < KPAD) {
      float o = 0.f;
      if (c < C) o = (v[j] - mean) * inv * (gamma ? gamma[c] : 1.f) + (beta ? beta[c] : 0.f);
      dst[c] = (_Float16)o;
    }
  }
}

}  // namespace lf
