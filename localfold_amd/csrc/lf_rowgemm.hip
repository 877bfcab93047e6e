// Generic row GEMMs (see lf_rowgemm.h): lnproj (LayerNorm + grouped projections) and
// rowgemm (f16 rows x streamed weights + bias / ReLU / row denominator / residual).
#include <algorithm>

#include "lf_rowgemm.h"

namespace lf {

constexpr int RG_WAVES = 8;            // 8 waves x 16 rows = 128 rows per block
constexpr int RG_ROWS = RG_WAVES * 16;

__device__ __forceinline__ long long dst_rowpart(const Dst& d, int row) {
  return (long long)(row / d.Q) * d.sB + (long long)(row % d.Q) * d.sN;
}
__device__ __forceinline__ long long dst_colpart(const Dst& d, int col) {
  return (long long)(col / d.D) * d.sH + (long long)(col % d.D) * d.sD;
}

__device__ __forceinline__ void dst_store(const Dst& d, long long idx, float v) {
  if (d.dtype == DT_F32) static_cast<float*>(d.ptr)[idx] = v;
  else if (d.dtype == DT_F16) static_cast<_Float16*>(d.ptr)[idx] = (_Float16)v;
  else static_cast<uint16_t*>(d.ptr)[idx] = f2bf(v);
}

__device__ __forceinline__ float dst_load(const void* ptr, int dtype, long long idx) {
  if (dtype == DT_F32) return static_cast<const float*>(ptr)[idx];
  if (dtype == DT_F16) return (float)static_cast<const _Float16*>(ptr)[idx];
  return bf2f(static_cast<const uint16_t*>(ptr)[idx]);
}

// Chunk `ci` of an lnproj launch -> (group, first logical column, columns per half)
__device__ __forceinline__ void chunk_of(const LnProjParams& p, int ci, int& gi, int& c0) {
  gi = 0;
  c0 = 0;
  for (int g = 0; g < p.ngroups; ++g) {
    const int w = p.g[g].op == OP_SWIGLU ? 32 : 64;
    const int n = (p.g[g].ncols + w - 1) / w;
    if (ci < n) {
      gi = g;
      c0 = ci * w;
      return;
    }
    ci -= n;
  }
}

// Loads chunk ci's weights ([64][KP] f16: 64 columns of w0, or 32 of w0 then 32 of w1) into
// registers (`regs`, NREG 16-byte words per thread), to be stored into LDS later.
template <int KP, int NREG>
__device__ __forceinline__ void chunk_load(const LnProjParams& p, int ci, uint4 (&regs)[NREG], int tid) {
  int gi, c0;
  chunk_of(p, ci, gi, c0);
  const Group& G = p.g[gi];
  const bool paired = G.op == OP_SWIGLU;
  constexpr int SEGS = KP / 8;
#pragma unroll
  for (int r = 0; r < NREG; ++r) {
    const int i = tid + r * 512;
    const int n = i / SEGS, seg = i - n * SEGS;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (n < 64) {
      const WExp& w = (paired && n >= 32) ? G.w1 : G.w0;
      const int col = paired ? c0 + (n & 31) : c0 + n;
      if (col < w.N && seg * 8 < w.kp) v = *reinterpret_cast<const uint4*>(w.p + (size_t)col * w.kp + seg * 8);
    }
    regs[r] = v;
  }
}

template <int KP, int NREG>
__device__ __forceinline__ void chunk_store(_Float16* Ws, const uint4 (&regs)[NREG], int tid) {
  constexpr int SEGS = KP / 8, LDW = KP + 8;
#pragma unroll
  for (int r = 0; r < NREG; ++r) {
    const int i = tid + r * 512;
    const int n = i / SEGS, seg = i - n * SEGS;
    if (n < 64) *reinterpret_cast<uint4*>(Ws + n * LDW + seg * 8) = regs[r];
  }
}

template <int ACT, int KS>
__global__ __launch_bounds__(512) void lnproj_kernel(LnProjParams p) {
  constexpr int KP = KS * 32, LDW = KP + 8;
  constexpr int NREG = (64 * KP / 8 + 511) / 512;
  __shared__ __attribute__((aligned(16))) _Float16 Ws[2][64 * LDW];
  __shared__ __attribute__((aligned(16))) float Gs[2 * KP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  stage_vec(Gs, p.ln_s, p.C, 1.f, KP, tid, 512);
  stage_vec(Gs + KP, p.ln_o, p.C, 0.f, KP, tid, 512);

  int nchunks = 0;
  for (int g = 0; g < p.ngroups; ++g) {
    const int w = p.g[g].op == OP_SWIGLU ? 32 : 64;
    nchunks += (p.g[g].ncols + w - 1) / w;
  }
  uint4 regs[NREG];
  chunk_load<KP, NREG>(p, 0, regs, tid);

  // this wave's 16 logical rows, LayerNorm'd into A fragments
  const int row0 = blockIdx.x * RG_ROWS + wave * 16;
  const int myrow = row0 + r16;
  const bool rvalid = myrow < p.rows;
  const int lrow = rvalid ? myrow : 0;
  const int srow = p.rmB > 0 ? (lrow % p.rmQ) * p.rmB + lrow / p.rmQ : lrow;
  h8 a[KS];
  {
    FragTile<ACT, KS> t;
    frag_load_row(t, p.x, (size_t)srow, p.C, lane);
    float x[KS][8];
    frag_values(t, x, p.C, lane);
    chunk_store<KP, NREG>(Ws[0], regs, tid);
    __syncthreads();  // Gs and chunk 0 staged
    frag_ln<KS>(x, a, rvalid, p.C, Gs, Gs + KP, p.eps, p.fast_var, lane);
  }
  // storage rows of the 4 output rows this lane holds (for OP_ROWMASK)
  int orow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) orow[i] = row0 + g4 * 4 + i;

  for (int ci = 0; ci < nchunks; ++ci) {
    const _Float16* W = Ws[ci & 1];
    if (ci + 1 < nchunks) chunk_load<KP, NREG>(p, ci + 1, regs, tid);
    f4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc[t] = mfma16(a[j], *reinterpret_cast<const h8*>(W + (t * 16 + r16) * LDW + 32 * j + kq), acc[t]);
    }
    int gi, c0;
    chunk_of(p, ci, gi, c0);
    const Group& G = p.g[gi];
    long long rp[4];
    float rm[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int lr = orow[i] < p.rows ? orow[i] : 0;
      rp[i] = dst_rowpart(G.dst, lr);
      rm[i] = 1.f;
      if (G.op == OP_ROWMASK) rm[i] = p.rowmask[p.rmB > 0 ? (lr % p.rmQ) * p.rmB + lr / p.rmQ : lr];
    }
    if (G.op == OP_SWIGLU) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int col = c0 + t * 16 + r16;
        if (col >= G.ncols) continue;
        const float b0 = G.bias0 ? G.bias0[col] : 0.f, b1 = G.bias1 ? G.bias1[col] : 0.f;
        const long long cp = dst_colpart(G.dst, col);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (orow[i] >= p.rows) continue;
          const float gt = (acc[t][i] + b0) * G.scale, vl = (acc[t + 2][i] + b1) * G.scale;
          dst_store(G.dst, rp[i] + cp, gt * sigmoidf_(gt) * vl);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int col = c0 + t * 16 + r16;
        if (col >= G.ncols) continue;
        const float b0 = G.bias0 ? G.bias0[col] : 0.f;
        const long long cp = dst_colpart(G.dst, col);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (orow[i] >= p.rows) continue;
          float v = (acc[t][i] + b0) * G.scale;
          if (G.op == OP_SIGMOID) v = sigmoidf_(v);
          else if (G.op == OP_RELU) v = fmaxf(v, 0.f);
          v *= rm[i];
          dst_store(G.dst, rp[i] + cp, v);
        }
      }
    }
    if (ci + 1 < nchunks) {
      chunk_store<KP, NREG>(Ws[(ci + 1) & 1], regs, tid);
      __syncthreads();
    }
  }
}

int launch_lnproj(lf_context* ctx, const LnProjParams& p, int act, const char* label) {
  if (p.C > 384) return set_error(LF_ERR_INVALID, std::string(label) + ": LayerNorm width above 384");
  if (p.rows <= 0) return LF_OK;
  const int ks = p.C <= 32 ? 1 : p.C <= 64 ? 2 : p.C <= 128 ? 4 : p.C <= 256 ? 8 : 12;
  dim3 grid((p.rows + RG_ROWS - 1) / RG_ROWS);
  LaunchScope ls(ctx, label);
#define LF_LP(A, K) hipLaunchKernelGGL((lnproj_kernel<A, K>), grid, dim3(512), 0, ctx->stream, p)
#define LF_LPK(A)            \
  if (ks == 1) LF_LP(A, 1);  \
  else if (ks == 2) LF_LP(A, 2); \
  else if (ks == 4) LF_LP(A, 4); \
  else if (ks == 8) LF_LP(A, 8); \
  else LF_LP(A, 12);
  if (act == DT_F32) { LF_LPK(DT_F32) }
  else if (act == DT_F16) { LF_LPK(DT_F16) }
  else { LF_LPK(DT_BF16) }
#undef LF_LPK
#undef LF_LP
  return check_hip(hipGetLastError(), label);
}

// ---------------------------------------------------------------------------------------

constexpr int RGK = 128;             // K slice per LDS stage
constexpr int RG_LDW = RGK + 8;

template <int DACT>
__global__ __launch_bounds__(512) void rowgemm_kernel(RowGemmParams p) {
  __shared__ __attribute__((aligned(16))) _Float16 Ws[2][64 * RG_LDW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  const int row0 = blockIdx.x * RG_ROWS + wave * 16;
  const int myrow = row0 + r16;
  const _Float16* arow = p.A + (size_t)(myrow < p.rows ? myrow : 0) * p.K;
  const int nks = (p.K + RGK - 1) / RGK, ncs = (p.N + 63) / 64, nst = nks * ncs;
  const bool kvec = (p.K & 7) == 0;

  // stage s = (column chunk s / nks, K slice s % nks): [64 cols][128 k] of the expanded weights
  auto wload = [&](int s, uint4 (&regs)[2]) {
    const int cc = s / nks, kc = s - cc * nks;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int i = tid + r * 512, n = i >> 4, seg = i & 15;
      const int col = cc * 64 + n, k = kc * RGK + seg * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (col < p.w.N && k < p.w.kp) v = *reinterpret_cast<const uint4*>(p.w.p + (size_t)col * p.w.kp + k);
      regs[r] = v;
    }
  };
  auto wstore = [&](_Float16* W, const uint4 (&regs)[2]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int i = tid + r * 512, n = i >> 4, seg = i & 15;
      *reinterpret_cast<uint4*>(W + n * RG_LDW + seg * 8) = regs[r];
    }
  };
  uint4 regs[2];
  wload(0, regs);
  wstore(Ws[0], regs);
  __syncthreads();

  f4 acc[4];
  for (int s = 0; s < nst; ++s) {
    const int cc = s / nks, kc = s - cc * nks;
    if (kc == 0)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    // this slice's A fragments first, then the next stage's weights: the MFMAs wait only
    // for the A loads (loads complete in issue order)
    h8 a[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = kc * RGK + 32 * j + kq;
      if (kvec) {
        a[j] = *reinterpret_cast<const h8*>(arow + (k + 8 <= p.K ? k : 0));
        if (k + 8 > p.K) a[j] = h8{0, 0, 0, 0, 0, 0, 0, 0};
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) a[j][e] = arow[k + e < p.K ? k + e : 0];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (k + e >= p.K) a[j][e] = (_Float16)0.f;
      }
    }
    if (s + 1 < nst) wload(s + 1, regs);
    const _Float16* W = Ws[s & 1];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc[t] = mfma16(a[j], *reinterpret_cast<const h8*>(W + (t * 16 + r16) * RG_LDW + 32 * j + kq), acc[t]);
    }
    if (kc == nks - 1) {
      long long rp[4], cp[4];
      float den[4], res[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + g4 * 4 + i;
        rp[i] = dst_rowpart(p.dst, row < p.rows ? row : 0);
        den[i] = p.rowden ? p.rowden[row < p.rows ? row : 0] : 1.f;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int col = cc * 64 + t * 16 + r16;
        cp[t] = dst_colpart(p.dst, col < p.N ? col : 0);
      }
      if (p.resid) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) res[t][i] = dst_load(p.resid, DACT, rp[i] + cp[t]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int col = cc * 64 + t * 16 + r16;
        if (col >= p.N) continue;
        const float b = p.bias ? p.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + g4 * 4 + i;
          if (row >= p.rows) continue;
          float v = acc[t][i] + b;
          if (p.op == OP_RELU) v = fmaxf(v, 0.f);
          if (p.rowden) v = v / den[i];
          if (p.resid) v += res[t][i];
          dst_store(p.dst, rp[i] + cp[t], v);
        }
      }
    }
    if (s + 1 < nst) {
      wstore(Ws[(s + 1) & 1], regs);
      __syncthreads();
    }
  }
}

int launch_rowgemm(lf_context* ctx, const RowGemmParams& p, const char* label) {
  if (p.rows <= 0) return LF_OK;
  dim3 grid((p.rows + RG_ROWS - 1) / RG_ROWS);
  LaunchScope ls(ctx, label);
  if (p.dst.dtype == DT_F32) hipLaunchKernelGGL(rowgemm_kernel<DT_F32>, grid, dim3(512), 0, ctx->stream, p);
  else if (p.dst.dtype == DT_F16) hipLaunchKernelGGL(rowgemm_kernel<DT_F16>, grid, dim3(512), 0, ctx->stream, p);
  else hipLaunchKernelGGL(rowgemm_kernel<DT_BF16>, grid, dim3(512), 0, ctx->stream, p);
  return check_hip(hipGetLastError(), label);
}

}  // namespace lf
