// AF2 input and recycling embedder before the template branch (InputEmbedderGpu.run /
// encodeInputEmbedder, webgpu/af2/evoformer/input-embedder.js:160-231).
//
//   msa[s, r]   = target[r] W1d + b1d + msa_feat[s, r] Wmsa + bmsa, + LN(prev_msa[r]) on s = 0
//                 (MSA_SHADER, :61-83)
//   pair[i, j]  = target[i] Wl + bl + target[j] Wr + br + bpos + Wpos[dgram bin of the
//                 pseudo-beta distance] + LN(prev_pair[i, j]) + brel + Wrel[clip(ri - rj + 32)]
//                 (PAIR_SHADER, :99-137)
//   extra[s, r] = bext + Wext[code] + has_deletion Wext[23] + deletion_value Wext[24]
//                 (EXTRA_SHADER, :85-97)
//
// All of it is gather / elementwise work bound by HBM: the per-residue terms (target[r] W1d,
// target[i] Wl, target[j] Wr) are computed once into a small f32 table, then one wave per
// msa or pair row reads its row once, normalises the recycled row in registers and writes
// the embedding once.  Layer norms are two-pass with eps 1e-5 (:197-204).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "lf_common.h"
#include "lf_context.h"
#include "lf_ops.h"

namespace lf {

namespace {

constexpr int EMB_MAXV = 8;   // channels per lane: C <= 512
constexpr int EMB_BINS = 15;
constexpr float EMB_MIN_BIN = 3.25f, EMB_MAX_BIN = 20.75f;
constexpr int EMB_MAX_REL = 32;

// per residue r: single[r] = target[r] W1d + b1d + bmsa (cM), left[r] = target[r] Wl + bl,
// right[r] = target[r] Wr + br (cZ each)
__global__ __launch_bounds__(256) void embed_single_kernel(const float* target, int Ct, int cM, int cZ,
                                                           lf_input_embedder_weights w, float* single,
                                                           float* left, float* right) {
  const int r = blockIdx.x;
  const float* t = target + (size_t)r * Ct;
  for (int c = threadIdx.x; c < cM + 2 * cZ; c += 256) {
    const float* W;
    float acc;
    int col, ld;
    float* dst;
    if (c < cM) {
      W = w.preprocess_1d_w, col = c, ld = cM, acc = w.preprocess_1d_b[c] + w.preprocess_msa_b[c];
      dst = single + (size_t)r * cM + c;
    } else if (c < cM + cZ) {
      col = c - cM, W = w.left_w, ld = cZ, acc = w.left_b[col];
      dst = left + (size_t)r * cZ + col;
    } else {
      col = c - cM - cZ, W = w.right_w, ld = cZ, acc = w.right_b[col];
      dst = right + (size_t)r * cZ + col;
    }
    for (int k = 0; k < Ct; ++k) acc += t[k] * W[(size_t)k * ld + col];
    *dst = acc;
  }
}

// lane values v[k] = row[lane + 64 k] (zeros past C), normalised in place (two-pass)
__device__ __forceinline__ void wave_ln(float (&v)[EMB_MAXV], int C, int lane, const float* scale,
                                        const float* offset, float eps) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < EMB_MAXV; ++k) s += v[k];
  const float mean = wave_sum(s) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < EMB_MAXV; ++k) {
    const int c = lane + 64 * k;
    const float d = c < C ? v[k] - mean : 0.f;
    q += d * d;
  }
  const float inv = 1.f / sqrtf(wave_sum(q) / (float)C + eps);
#pragma unroll
  for (int k = 0; k < EMB_MAXV; ++k) {
    const int c = lane + 64 * k;
    if (c < C) v[k] = (v[k] - mean) * inv * scale[c] + offset[c];
  }
}

__device__ __forceinline__ void wave_row_load(float (&v)[EMB_MAXV], const void* src, int dt, size_t base, int C,
                                              int lane) {
#pragma unroll
  for (int k = 0; k < EMB_MAXV; ++k) {
    const int c = lane + 64 * k;
    v[k] = (src != nullptr && c < C) ? load_act(src, dt, base + c) : 0.f;
  }
}

// One wave per EMB_ROWS msa rows: a lane holds one feature of each row (feature j = lane, up to
// 64 per pass), broadcast through readlane, and the channels lane + 64 k of every row, so each
// weight value Wmsa[j][c] (L1/L2-resident) is loaded once for EMB_ROWS rows.  The f32 FMAs
// bound it (S L cM Cf of them); staging Wmsa in LDS measured slower (fewer waves per CU).
constexpr int EMB_ROWS = 8;
__global__ __launch_bounds__(256) void embed_msa_kernel(const float* msa_feat, int S, int L, int Cf, int cM,
                                                        const float* single, const float* wmsa, const void* prev,
                                                        int prev_dt, const float* ln_s, const float* ln_o,
                                                        float eps, void* out, int out_dt) {
  const long long rows = (long long)S * L;
  const long long row0 = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * EMB_ROWS;
  if (row0 >= rows) return;
  const int lane = threadIdx.x & 63;
  const int nk = (cM + 63) / 64;
  float acc[EMB_ROWS][EMB_MAXV];
#pragma unroll
  for (int r = 0; r < EMB_ROWS; ++r)
#pragma unroll
    for (int k = 0; k < EMB_MAXV; ++k) acc[r][k] = 0.f;
  for (int j0 = 0; j0 < Cf; j0 += 64) {
    float fv[EMB_ROWS];
#pragma unroll
    for (int r = 0; r < EMB_ROWS; ++r) {
      const long long row = min(row0 + r, rows - 1);
      fv[r] = j0 + lane < Cf ? msa_feat[row * Cf + j0 + lane] : 0.f;
    }
    const int jn = min(64, Cf - j0);
    for (int j = 0; j < jn; ++j) {
      float wj[EMB_MAXV];
#pragma unroll
      for (int k = 0; k < EMB_MAXV; ++k) {
        const int c = lane + 64 * k;
        wj[k] = (k < nk && c < cM) ? wmsa[(size_t)(j0 + j) * cM + c] : 0.f;
      }
#pragma unroll
      for (int r = 0; r < EMB_ROWS; ++r) {
        const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fv[r]), j));
#pragma unroll
        for (int k = 0; k < EMB_MAXV; ++k) acc[r][k] += x * wj[k];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < EMB_ROWS; ++r) {
    const long long row = row0 + r;
    if (row >= rows) break;
    const int res = (int)(row % L);
    float v[EMB_MAXV];
    if (row < L) {   // sequence 0: the recycled first row, normalised
      wave_row_load(v, prev, prev_dt, (size_t)res * cM, cM, lane);
      wave_ln(v, cM, lane, ln_s, ln_o, eps);
    } else {
#pragma unroll
      for (int k = 0; k < EMB_MAXV; ++k) v[k] = 0.f;
    }
#pragma unroll
    for (int k = 0; k < EMB_MAXV; ++k) {
      const int c = lane + 64 * k;
      if (c < cM) store_act(out, out_dt, (size_t)row * cM + c, acc[r][k] + single[(size_t)res * cM + c] + v[k]);
    }
  }
}

__device__ __forceinline__ void pseudo_beta(const float* pos, const float* aatype, int r, float (&x)[3]) {
  const int atom = (int)aatype[r] == 7 ? 1 : 3;
#pragma unroll
  for (int c = 0; c < 3; ++c) x[c] = pos ? pos[((size_t)r * 37 + atom) * 3 + c] : 0.f;
}

// one wave per pair row (i, j)
__global__ __launch_bounds__(256) void embed_pair_kernel(int L, int cZ, const float* left, const float* right,
                                                         const float* pos, const float* aatype,
                                                         const float* residue_index, lf_input_embedder_weights w,
                                                         const void* prev, int prev_dt, float eps, void* out,
                                                         int out_dt) {
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (long long)L * L) return;
  const int lane = threadIdx.x & 63;
  const int i = (int)(row / L), j = (int)(row % L);
  float v[EMB_MAXV];
  wave_row_load(v, prev, prev_dt, (size_t)row * cZ, cZ, lane);
  wave_ln(v, cZ, lane, w.prev_pair_norm_scale, w.prev_pair_norm_offset, eps);
  // distogram bin of the recycled pseudo-beta distance (:110-129); at or below 3.25 A none
  float a[3], b[3];
  pseudo_beta(pos, aatype, i, a);
  pseudo_beta(pos, aatype, j, b);
  float d2 = 0.f;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float d = a[c] - b[c];
    d2 += d * d;
  }
  const float width = (EMB_MAX_BIN - EMB_MIN_BIN) / (float)(EMB_BINS - 1);
  int bin = -1;
  for (int k = 0; k < EMB_BINS; ++k) {
    const float lower = EMB_MIN_BIN + (float)k * width;
    const float upper = k + 1 < EMB_BINS ? EMB_MIN_BIN + (float)(k + 1) * width : EMB_MAX_BIN + width;
    if (d2 > lower * lower && (k + 1 == EMB_BINS || d2 < upper * upper)) bin = k;
  }
  const int off = (int)residue_index[i] - (int)residue_index[j] + EMB_MAX_REL;
  const int rel = min(max(off, 0), 2 * EMB_MAX_REL);
#pragma unroll
  for (int k = 0; k < EMB_MAXV; ++k) {
    const int c = lane + 64 * k;
    if (c >= cZ) break;
    float acc = left[(size_t)i * cZ + c] + right[(size_t)j * cZ + c] + w.prev_pos_b[c];
    if (bin >= 0) acc += w.prev_pos_w[(size_t)bin * cZ + c];
    acc += v[k];
    acc += w.relpos_b[c] + w.relpos_w[(size_t)rel * cZ + c];
    store_act(out, out_dt, (size_t)row * cZ + c, acc);
  }
}

// one thread per extra-MSA element
__global__ __launch_bounds__(256) void embed_extra_kernel(const float* codes, const float* has_del,
                                                          const float* del_val, long long rows, int cE,
                                                          const float* W, const float* bias, void* out, int out_dt) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * cE) return;
  const long long row = rows * cE < (1LL << 31) ? (long long)((int)idx / cE) : idx / cE;
  const int c = (int)(idx - row * cE);
  const int code = min(max((int)codes[row], 0), 22);   // 23 residue classes; keeps a bad code in bounds
  float acc = bias[c] + W[(size_t)code * cE + c];
  acc += has_del[row] * W[23 * (size_t)cE + c];
  acc += del_val[row] * W[24 * (size_t)cE + c];
  store_act(out, out_dt, (size_t)idx, acc);
}

}  // namespace

int input_embedder(lf_context* ctx, const lf_input_embedder_args& a) {
  LF_REQUIRE(a.w != nullptr, "input embedder: weights are NULL");
  const lf_input_embedder_weights& w = *a.w;
  const int L = a.length, S = a.msa_sequences, Se = a.extra_sequences;
  LF_REQUIRE(L > 0 && S > 0 && Se >= 0 && a.target_channels > 0 && a.msa_feature_channels > 0,
             "input embedder dimensions must be positive");
  LF_REQUIRE(a.c_m > 0 && a.c_m <= 64 * EMB_MAXV && a.c_z > 0 && a.c_z <= 64 * EMB_MAXV && a.c_e > 0,
             "input embedder: channels must be 1..512");
  LF_REQUIRE(act_dtype_ok(a.msa_dtype) && act_dtype_ok(a.pair_dtype) && act_dtype_ok(a.extra_dtype),
             "input embedder: dtypes must be f32, f16 or bf16");
  LF_REQUIRE(a.target_feat && a.msa_feat && a.residue_index && a.aatype && a.msa && a.pair,
             "input embedder: NULL feature or output");
  LF_REQUIRE(Se == 0 || (a.extra_msa && a.extra_has_deletion && a.extra_deletion_value && a.extra),
             "input embedder: NULL extra-MSA feature or output");
  LF_REQUIRE(w.preprocess_1d_w && w.preprocess_1d_b && w.preprocess_msa_w && w.preprocess_msa_b && w.left_w &&
                 w.left_b && w.right_w && w.right_b && w.prev_pos_w && w.prev_pos_b && w.prev_msa_norm_scale &&
                 w.prev_msa_norm_offset && w.prev_pair_norm_scale && w.prev_pair_norm_offset && w.relpos_w &&
                 w.relpos_b && (Se == 0 || (w.extra_w && w.extra_b)),
             "input embedder: NULL weight");
  LF_REQUIRE((long long)L * L < (1LL << 31) && (long long)S * L < (1LL << 31), "input embedder: too many rows");
  const float eps = a.epsilon > 0.f ? a.epsilon : 1e-5f;
  size_t sizes[3] = {(size_t)L * a.c_m * sizeof(float), (size_t)L * a.c_z * sizeof(float),
                     (size_t)L * a.c_z * sizeof(float)};
  void* bufs[3];
  LF_TRY(workspace(ctx, sizes, bufs, 3));
  float *single = (float*)bufs[0], *left = (float*)bufs[1], *right = (float*)bufs[2];
  {
    LaunchScope ls(ctx, "embed.single");
    hipLaunchKernelGGL(embed_single_kernel, dim3(L), dim3(256), 0, ctx->stream, a.target_feat, a.target_channels,
                       a.c_m, a.c_z, w, single, left, right);
  }
  LF_TRY(check_hip(hipGetLastError(), "embed single launch"));
  {
    LaunchScope ls(ctx, "embed.msa");
    const long long groups = ((long long)S * L + EMB_ROWS - 1) / EMB_ROWS;
    hipLaunchKernelGGL(embed_msa_kernel, dim3((unsigned)((groups + 3) / 4)), dim3(256), 0, ctx->stream,
                       a.msa_feat, S, L, a.msa_feature_channels, a.c_m, single, w.preprocess_msa_w,
                       a.prev_msa_first_row, a.msa_dtype, w.prev_msa_norm_scale, w.prev_msa_norm_offset, eps, a.msa,
                       a.msa_dtype);
  }
  LF_TRY(check_hip(hipGetLastError(), "embed msa launch"));
  {
    LaunchScope ls(ctx, "embed.pair");
    hipLaunchKernelGGL(embed_pair_kernel, dim3((unsigned)(((long long)L * L + 3) / 4)), dim3(256), 0, ctx->stream,
                       L, a.c_z, left, right, a.prev_positions, a.aatype, a.residue_index, w, a.prev_pair,
                       a.pair_dtype, eps, a.pair, a.pair_dtype);
  }
  LF_TRY(check_hip(hipGetLastError(), "embed pair launch"));
  if (Se > 0) {
    const long long n = (long long)Se * L * a.c_e;
    LaunchScope ls(ctx, "embed.extra");
    hipLaunchKernelGGL(embed_extra_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream,
                       a.extra_msa, a.extra_has_deletion, a.extra_deletion_value, (long long)Se * L, a.c_e,
                       w.extra_w, w.extra_b, a.extra, a.extra_dtype);
  }
  LF_TRY(check_hip(hipGetLastError(), "embed extra launch"));
  return LF_OK;
}

}  // namespace lf
