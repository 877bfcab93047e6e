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
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));   // register words (arrays of it stay in VGPRs)

enum DType { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_I8 = 3, DT_I5 = 4 };

constexpr int WAVE = 64;

__device__ __forceinline__ float h2f(uint16_t bits) {
  _Float16 h;
  __builtin_memcpy(&h, &bits, 2);
  return (float)h;
}

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Round-to-nearest-even float -> bf16 (gfx950's v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f2bf(float f) {
  const __bf16 h = (__bf16)f;
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
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

// sigmoid with the hardware exp and reciprocal (v_exp_f32, v_rcp_f32: ~1 ulp each)
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// 1/sqrt(x) with v_rsq_f32 (~1 ulp)
__device__ __forceinline__ float rsqrt_(float x) { return __builtin_amdgcn_rsqf(x); }

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
  // How the kernels fetch and decode the weights themselves, 8 at a time (set by make_view):
  // WRUN_K when 8 consecutive k of one column are adjacent in storage ((out,in) layout), WRUN_N
  // when 8 consecutive columns of one k are ((in,out) layout) -- one vector load of codes and
  // one scale per run -- and WRUN_GATHER, element by element, when neither holds with the
  // alignment the vector loads need (interleaved columns, widths not a multiple of 8).
  int run;
  int gshift;               // log2(group) for flat groups (a power of two, multiple of 8)
};
enum { WRUN_GATHER = 0, WRUN_K = 1, WRUN_N = 2 };

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
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}


// 16x16x16 f16 MFMA: lane l supplies A[l%16][4(l/16)+j] and B[4(l/16)+j][l%16], j < 4.
__device__ __forceinline__ f4 mfma16k16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Compile-time activation storage: loads and stores are straight-line code, so a wave can
// keep many of them in flight (a runtime dtype switch puts every load in its own basic
// block and the compiler then waits for each one before the next).
template <int ACT> struct Act;
template <> struct Act<DT_F32> {
  typedef float T;
  static __device__ __forceinline__ float ld(const T* p) { return *p; }
  static __device__ __forceinline__ void st(T* p, float v) { *p = v; }
};
template <> struct Act<DT_F16> {
  typedef _Float16 T;
  static __device__ __forceinline__ float ld(const T* p) { return (float)*p; }
  static __device__ __forceinline__ void st(T* p, float v) { *p = (_Float16)v; }
};
template <> struct Act<DT_BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float ld(const T* p) { return bf2f(*p); }
  static __device__ __forceinline__ void st(T* p, float v) { *p = f2bf(v); }
};

// Sum over the 4 lanes of a quad (lanes 4q..4q+3) with two DPP quad permutes (VALU only).
__device__ __forceinline__ float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));  // [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));  // [2,3,0,1]
  return v;
}

// A tile of 16 activation rows held in registers by one wave, 4 lanes per row: lane l owns
// row l/4 and the CPL = KPAD/4 consecutive channels (l%4)*CPL.  A tile of row-major rows is
// one contiguous block of memory, so the 16-byte loads of a wave are fully coalesced, and
// a row's statistics need only a 4-lane (DPP) reduction.  The words are kept RAW until the
// tile is normalised, so loads issued for the next tile stay in flight meanwhile.
template <int ACT, int KPAD>
struct RowTile {
  typedef typename Act<ACT>::T T;
  static constexpr int CPL = KPAD / 4;
  static constexpr int VEC = 16 / (int)sizeof(T);   // elements per 16-byte load
  static constexpr int NV = CPL / VEC;
  static_assert(CPL % VEC == 0, "a lane's channels must be whole 16-byte vectors");
  uint4 raw[NV];
  __device__ __forceinline__ float get(int j) const {
    const T* e = reinterpret_cast<const T*>(raw);
    return Act<ACT>::ld(e + j);
  }
};

// Row r = lane/4 reads src[(row0 + r) * C + c]; rows >= nvalid and channels >= C come from a
// clamped (valid) address and are discarded when the tile is normalised.
template <int ACT, int KPAD>
__device__ __forceinline__ void tile_load(RowTile<ACT, KPAD>& t, const void* src, size_t row0, int nvalid, int C,
                                          int lane) {
  typedef RowTile<ACT, KPAD> RT;
  typedef typename RT::T T;
  const T* s = static_cast<const T*>(src);
  const int r = lane >> 2, c0 = (lane & 3) * RT::CPL;
  const size_t base = (row0 + (r < nvalid ? r : 0)) * (size_t)C;
  if (C == KPAD) {
#pragma unroll
    for (int v = 0; v < RT::NV; ++v) t.raw[v] = *reinterpret_cast<const uint4*>(s + base + c0 + v * RT::VEC);
  } else {
    T* e = reinterpret_cast<T*>(t.raw);
#pragma unroll
    for (int j = 0; j < RT::CPL; ++j) {
      const int c = c0 + j;
      e[j] = s[base + (c < C ? c : 0)];
    }
  }
}

// LayerNorm of the tile's rows written as f16 to dst[r*lda + c], c < KPAD (zero past C and
// for rows >= nvalid).  gamma/beta: KPAD floats (LDS), 1/0 past C.  Two-pass statistics
// (mean, then mean squared deviation) as webgpu/kernels/triangle/cpu-reference.js:5-29, or
// E[x^2]-E[x]^2 when fast_var (cpu/af3/trunk/pairformer.js:68-87).
template <int ACT, int KPAD>
__device__ __forceinline__ void tile_ln_store(const RowTile<ACT, KPAD>& t, _Float16* dst, int lda, int nvalid, int C,
                                              const float* gamma, const float* beta, float eps, bool fast_var,
                                              int lane) {
  constexpr int CPL = RowTile<ACT, KPAD>::CPL;
  const int r = lane >> 2, c0 = (lane & 3) * CPL;
  const bool full = C == KPAD;
  float x[CPL];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    x[j] = (full || c0 + j < C) ? t.get(j) : 0.f;
    s += x[j];
  }
  const float invC = 1.0f / (float)C;
  const float mean = quad_sum(s) * invC;
  float q = 0.f;
  if (fast_var) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) q += x[j] * x[j];
    q = quad_sum(q) * invC - mean * mean;
  } else {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float d = (full || c0 + j < C) ? x[j] - mean : 0.f;
      q += d * d;
    }
    q = quad_sum(q) * invC;
  }
  const float inv = rsqrt_(q + eps);
  const bool ok = r < nvalid;
  _Float16* d = dst + r * lda + c0;
#pragma unroll
  for (int v = 0; v < CPL / 8; ++v) {
    h8 o;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = v * 8 + k;
      o[k] = (_Float16)((ok && (full || c0 + j < C)) ? (x[j] - mean) * inv * gamma[c0 + j] + beta[c0 + j] : 0.f);
    }
    *reinterpret_cast<h8*>(d + v * 8) = o;
  }
}

// LayerNorm, in place, of each of the 16 rows of an f16 LDS tile X[r*ld + c] over its first
// C of KPAD columns (4 lanes per row, as tile_ln_store).  Rows >= nvalid become zero.
template <int KPAD>
__device__ __forceinline__ void lds_ln_inplace(_Float16* X, int ld, int nvalid, int C, const float* gamma,
                                               const float* beta, float eps, bool fast_var, int lane) {
  constexpr int CPL = KPAD / 4;
  const int r = lane >> 2, c0 = (lane & 3) * CPL;
  _Float16* row = X + r * ld + c0;
  float x[CPL];
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < CPL / 8; ++v) {
    const h8 h = *reinterpret_cast<const h8*>(row + v * 8);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x[v * 8 + k] = (c0 + v * 8 + k < C) ? (float)h[k] : 0.f;
      s += x[v * 8 + k];
    }
  }
  const float invC = 1.0f / (float)C;
  const float mean = quad_sum(s) * invC;
  float q = 0.f;
  if (fast_var) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) q += x[j] * x[j];
    q = quad_sum(q) * invC - mean * mean;
  } else {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float d = c0 + j < C ? x[j] - mean : 0.f;
      q += d * d;
    }
    q = quad_sum(q) * invC;
  }
  const float inv = rsqrt_(q + eps);
  const bool ok = r < nvalid;
#pragma unroll
  for (int v = 0; v < CPL / 8; ++v) {
    h8 o;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = v * 8 + k;
      o[k] = (_Float16)((ok && c0 + j < C) ? (x[j] - mean) * inv * gamma[c0 + j] + beta[c0 + j] : 0.f);
    }
    *reinterpret_cast<h8*>(row + v * 8) = o;
  }
}

// ---- MFMA A-fragment row tiles ---------------------------------------------------------
// For v_mfma_f32_16x16x32_f16 over K = 32*KS in KS k-steps, lane l supplies row l%16 and
// channels 32*j + 8*(l/16) .. +8 at k-step j.  A FragTile loads a 16-row activation tile
// straight into that layout (one 16-byte load per k-step for 16-bit storage, two for f32),
// so LayerNorm'd rows never touch LDS: a row's channels sit in lanes l, l^16, l^32, l^48
// and its statistics take two cross-lane shuffles for all 16 rows at once.
template <int ACT, int KS = 4>
struct FragTile {
  typedef typename Act<ACT>::T T;
  static constexpr int NV = (int)sizeof(T) * 8 / 16;   // 16-byte words per 8 elements
  u32x4 raw[KS][NV];
  // element e (< 8) of k-step j, decoded with shifts (no address-taken locals)
  __device__ __forceinline__ float get(int j, int e) const {
    if constexpr (ACT == DT_F32) {
      const u32x4 q = raw[j][e >> 2];
      const uint32_t w = (e & 3) == 0 ? q.x : (e & 3) == 1 ? q.y : (e & 3) == 2 ? q.z : q.w;
      return __uint_as_float(w);
    } else {
      const u32x4 q = raw[j][0];
      const uint32_t w = (e >> 1) == 0 ? q.x : (e >> 1) == 1 ? q.y : (e >> 1) == 2 ? q.z : q.w;
      const uint16_t hbits = (uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu));
      if constexpr (ACT == DT_BF16) return bf2f(hbits);
      else return h2f(hbits);
    }
  }
};

// Lane loads its row (storage row `srow`, already clamped to a valid row) at channels
// 32j + 8*(lane/16) + e; channels >= C read as zero.
template <int ACT, int KS>
__device__ __forceinline__ void frag_load_row(FragTile<ACT, KS>& t, const void* src, size_t srow, int C, int lane) {
  typedef typename FragTile<ACT, KS>::T T;
  const T* s = static_cast<const T*>(src) + srow * (size_t)C;
  const int g = lane >> 4;
  if (C == 32 * KS) {
    // one per-lane base, then compile-time offsets (immediates of the loads): with the lane
    // term inside each address the compiler kept a 64-bit address per load live and spilled
    const T* sg = s + 8 * g;
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int v = 0; v < FragTile<ACT, KS>::NV; ++v)
        t.raw[j][v] = *reinterpret_cast<const u32x4*>(sg + 32 * j + v * (16 / (int)sizeof(T)));
  } else {
    // C not a multiple of 32: when rows stay 16-byte aligned, whole 8-channel groups below C
    // take the vector loads and the group that straddles C (one lane group of one k-step)
    // reads element by element, zero past C; otherwise every group reads element by element
    const T* sg = s + 8 * g;
    const bool vec = (C * (int)sizeof(T)) % 16 == 0;
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const int c0 = 32 * j + 8 * g;
      if (vec && c0 + 8 <= C) {
#pragma unroll
        for (int v = 0; v < FragTile<ACT, KS>::NV; ++v)
          t.raw[j][v] = *reinterpret_cast<const u32x4*>(sg + 32 * j + v * (16 / (int)sizeof(T)));
      } else {
        uint32_t w[4 * FragTile<ACT, KS>::NV];
        if constexpr (ACT == DT_F32) {
#pragma unroll
          for (int k = 0; k < 8; ++k) w[k] = c0 + k < C ? __float_as_uint(s[c0 + k]) : 0u;
          t.raw[j][0] = u32x4{w[0], w[1], w[2], w[3]};
          t.raw[j][1] = u32x4{w[4], w[5], w[6], w[7]};
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int c = c0 + 2 * k;
            const uint16_t lo = c < C ? __builtin_bit_cast(uint16_t, s[c]) : (uint16_t)0;
            const uint16_t hi = c + 1 < C ? __builtin_bit_cast(uint16_t, s[c + 1]) : (uint16_t)0;
            w[k] = (uint32_t)lo | ((uint32_t)hi << 16);
          }
          t.raw[j][0] = u32x4{w[0], w[1], w[2], w[3]};
        }
      }
    }
  }
}

// Row r16 = lane%16 of the tile reads src[(row0 + r16) * C + ...]; rows >= nvalid read row0.
template <int ACT, int KS = 4>
__device__ __forceinline__ void frag_load(FragTile<ACT, KS>& t, const void* src, size_t row0, int nvalid, int C,
                                          int lane) {
  const int r = lane & 15;
  frag_load_row(t, src, row0 + (r < nvalid ? r : 0), C, lane);
}

// 8 floats -> the storage words of 8 activations (bit operations only, so the words stay
// in registers).
template <int ACT>
__device__ __forceinline__ void pack8(const float (&v)[8], uint4 (&o)[FragTile<ACT>::NV]) {
  if constexpr (ACT == DT_F32) {
    o[0] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
    o[1] = make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7]));
  } else if constexpr (ACT == DT_BF16) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = (uint32_t)f2bf(v[2 * k]) | ((uint32_t)f2bf(v[2 * k + 1]) << 16);
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const h2 hh = h2{(_Float16)v[2 * k], (_Float16)v[2 * k + 1]};
      w[k] = __builtin_bit_cast(uint32_t, hh);
    }
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Reductions over lanes l, l^16, l^32, l^48 with gfx950's VALU lane swaps (no LDS round
// trip).  With the same register as both operands, v_permlane16_swap pairs row 0 with row 1
// and row 2 with row 3 (rows of 16 lanes), and v_permlane32_swap the lower half with the
// upper half: combining the two results gives every lane the pair's reduction.
__device__ __forceinline__ float lanes4_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float lanes4_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Four consecutive activations at element index idx (8-/16-byte aligned).
template <int ACT>
__device__ __forceinline__ void ld4v(const void* base, size_t idx, float (&v)[4]) {
  if constexpr (ACT == DT_F32) {
    const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else if constexpr (ACT == DT_F16) {
    const h4 q = *reinterpret_cast<const h4*>(static_cast<const _Float16*>(base) + idx);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)q[i];
  } else {
    const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
    v[0] = __uint_as_float(q.x << 16); v[1] = __uint_as_float(q.x & 0xffff0000u);
    v[2] = __uint_as_float(q.y << 16); v[3] = __uint_as_float(q.y & 0xffff0000u);
  }
}

// Four activations as their storage words: loaded early, taken into registers (touch) at a
// chosen point, converted when used.
template <int ACT>
struct Raw4v {
  typedef uint2 T;
  __device__ static T load(const void* base, size_t idx) {
    return *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
  }
  __device__ static void touch(T& q) { asm volatile("" : "+v"(q.x), "+v"(q.y)); }
  __device__ static void unpack(const T& q, float (&v)[4]) {
    if constexpr (ACT == DT_F16) {
      const h4 h = __builtin_bit_cast(h4, q);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (float)h[i];
    } else {
      v[0] = __uint_as_float(q.x << 16); v[1] = __uint_as_float(q.x & 0xffff0000u);
      v[2] = __uint_as_float(q.y << 16); v[3] = __uint_as_float(q.y & 0xffff0000u);
    }
  }
};
template <>
struct Raw4v<DT_F32> {
  typedef float4 T;
  __device__ static T load(const void* base, size_t idx) {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
  }
  __device__ static void touch(T& q) { asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w)); }
  __device__ static void unpack(const T& q, float (&v)[4]) { v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w; }
};

template <int ACT>
__device__ __forceinline__ void st4v(void* base, size_t idx, const float (&v)[4]) {
  if constexpr (ACT == DT_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + idx) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (ACT == DT_F16) {
    h4 q;
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = (_Float16)v[i];
    *reinterpret_cast<h4*>(static_cast<_Float16*>(base) + idx) = q;
  } else {
    uint2 q;
    q.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
    q.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + idx) = q;
  }
} 

// (float)h + c, with h the f16 in half HI of the dword w, as one mixed-precision FMA
// (h * 1.0 + c: exact widening, one rounding, the same value as a convert then an add).
template <int HI>
__device__ __forceinline__ float f16_add(uint32_t w, float c) {
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(c));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(c));
  return r;
}

// LayerNorm of the 16 rows held as values x[j][e] (channel 32j + 8*(lane/16) + e, zero past
// C) into f16 A fragments.  gamma/beta: 32*KS floats (LDS).  Rows with !ok give zeros.
template <int KS>
__device__ __forceinline__ void frag_ln(const float (&x)[KS][8], h8 (&a)[KS], bool ok, int C, const float* gamma,
                                        const float* beta, float eps, bool fast_var, int lane) {
  const int g = lane >> 4;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < KS; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += x[j][e];
  const float invC = 1.0f / (float)C;
  const float mean = lanes4_sum(s) * invC;
  float q = 0.f;
  if (fast_var) {
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) q += x[j][e] * x[j][e];
    q = lanes4_sum(q) * invC - mean * mean;
  } else {
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = (32 * j + 8 * g + e < C) ? x[j][e] - mean : 0.f;
        q += d * d;
      }
    q = lanes4_sum(q) * invC;
  }
  const float inv = rsqrt_(q + eps);
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    const float4 g0 = *reinterpret_cast<const float4*>(gamma + 32 * j + 8 * g);
    const float4 g1 = *reinterpret_cast<const float4*>(gamma + 32 * j + 8 * g + 4);
    const float4 b0 = *reinterpret_cast<const float4*>(beta + 32 * j + 8 * g);
    const float4 b1 = *reinterpret_cast<const float4*>(beta + 32 * j + 8 * g + 4);
    const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool valid = ok && (32 * j + 8 * g + e < C);
      a[j][e] = (_Float16)(valid ? (x[j][e] - mean) * inv * gg[e] + bb[e] : 0.f);
    }
  }
}

// Keeps the compiler from carrying values decoded from a raw tile from one pass to the
// next (the packed words stay live; the decoded floats would cost 8x the registers).
template <int ACT, int KS>
__device__ __forceinline__ void launder(FragTile<ACT, KS>& t) {
#pragma unroll
  for (int j = 0; j < KS; ++j)
#pragma unroll
    for (int v = 0; v < FragTile<ACT, KS>::NV; ++v)
      asm volatile("" : "+v"(t.raw[j][v].x), "+v"(t.raw[j][v].y), "+v"(t.raw[j][v].z), "+v"(t.raw[j][v].w));
}

// Row statistics of a raw tile whose channels >= C hold zeros (frag_load_row): values are
// decoded on the fly, one k-step at a time, so only the packed words stay live.  The padding
// channels add (32*KS - C) * mean^2 to the centred sum, which is subtracted.
template <int ACT, int KS>
__device__ __forceinline__ void frag_stats_raw(FragTile<ACT, KS>& t, int C, float eps, bool fast_var, float& mean,
                                               float& inv) {
  float s = 0.f, q = 0.f;
#pragma unroll
  for (int j = 0; j < KS; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = t.get(j, e);
      s += v;
      q += v * v;
    }
    __builtin_amdgcn_sched_barrier(0);   // decode one k-step at a time
  }
  const float invC = 1.0f / (float)C;
  mean = lanes4_sum(s) * invC;
  if (fast_var) {
    q = lanes4_sum(q) * invC - mean * mean;
  } else {
    launder(t);
    q = 0.f;
#pragma unroll
    for (int j = 0; j < KS; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = t.get(j, e) - mean;
        q += d * d;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    q = (lanes4_sum(q) - (float)(32 * KS - C) * mean * mean) * invC;
  }
  inv = rsqrt_(q + eps);
  launder(t);
}

// LayerNorm of two raw tiles into MFMA fragments, gamma/beta read once per k-step for both.
// Padding channels normalise to finite values that meet zero weight rows; rows past the end
// are normalised too (their outputs are never stored).
template <int ACT, int KS>
__device__ __forceinline__ void frag_ln_raw2(FragTile<ACT, KS>& t0, FragTile<ACT, KS>& t1, h8 (&a0)[KS],
                                             h8 (&a1)[KS], int C, const float* gamma, const float* beta,
                                             float eps, bool fast_var, int lane) {
  const int g = lane >> 4;
  float m0, i0, m1, i1;
  frag_stats_raw(t0, C, eps, fast_var, m0, i0);
  frag_stats_raw(t1, C, eps, fast_var, m1, i1);
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    const float4 g0 = *reinterpret_cast<const float4*>(gamma + 32 * j + 8 * g);
    const float4 g1 = *reinterpret_cast<const float4*>(gamma + 32 * j + 8 * g + 4);
    const float4 b0 = *reinterpret_cast<const float4*>(beta + 32 * j + 8 * g);
    const float4 b1 = *reinterpret_cast<const float4*>(beta + 32 * j + 8 * g + 4);
    const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a0[j][e] = (_Float16)((t0.get(j, e) - m0) * i0 * gg[e] + bb[e]);
      a1[j][e] = (_Float16)((t1.get(j, e) - m1) * i1 * gg[e] + bb[e]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int ACT, int KS>
__device__ __forceinline__ void frag_ln_given(FragTile<ACT, KS>& t0, h8 (&a0)[KS], const float* gamma,
                                              const float* beta, float m0, float i0, int lane);

// LayerNorm of one raw tile into MFMA fragments (frag_ln_raw2 for a single tile).
template <int ACT, int KS>
__device__ __forceinline__ void frag_ln_raw1(FragTile<ACT, KS>& t0, h8 (&a0)[KS], int C, const float* gamma,
                                             const float* beta, float eps, bool fast_var, int lane) {
  float m0, i0;
  frag_stats_raw(t0, C, eps, fast_var, m0, i0);
  frag_ln_given(t0, a0, gamma, beta, m0, i0, lane);
}

// The normalisation of frag_ln_raw1 with a row's mean m0 and 1/std i0 already known (the
// triangle output kernel reads them from the project kernel).
template <int ACT, int KS>
__device__ __forceinline__ void frag_ln_given(FragTile<ACT, KS>& t0, h8 (&a0)[KS], const float* gamma,
                                              const float* beta, float m0, float i0, int lane) {
  const int g = lane >> 4;
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    const float4 g0 = *reinterpret_cast<const float4*>(gamma + 32 * j + 8 * g);
    const float4 g1 = *reinterpret_cast<const float4*>(gamma + 32 * j + 8 * g + 4);
    const float4 b0 = *reinterpret_cast<const float4*>(beta + 32 * j + 8 * g);
    const float4 b1 = *reinterpret_cast<const float4*>(beta + 32 * j + 8 * g + 4);
    const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) a0[j][e] = (_Float16)((t0.get(j, e) - m0) * i0 * gg[e] + bb[e]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// dst[i] = v[i] when v is non-null and i < n, else dflt; i < cap (block-cooperative).
__device__ __forceinline__ void stage_vec(float* dst, const float* v, int n, float dflt, int cap, int tid,
                                          int nthreads) {
  for (int i = tid; i < cap; i += nthreads) dst[i] = (v && i < n) ? v[i] : dflt;
}

}  // namespace lf
