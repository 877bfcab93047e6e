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

// Loads chunk ci of the packed weights (a contiguous [64][KP] f16 block) into registers
// (NREG 16-byte words per thread), to be stored into LDS later.
template <int KP, int NREG>
__device__ __forceinline__ void chunk_load(const LnProjParams& p, int ci, uint4 (&regs)[NREG], int tid) {
  const uint4* src = reinterpret_cast<const uint4*>(p.wpk + (size_t)ci * 64 * KP);
#pragma unroll
  for (int r = 0; r < NREG; ++r) {
    const int i = tid + r * 512;
    regs[r] = i < 64 * KP / 8 ? src[i] : make_uint4(0, 0, 0, 0);
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

// lnproj: 8 waves x 32 rows (two 16-row tiles) = 256 rows per block.  The LayerNorm'd rows
// stay in registers as MFMA B fragments for the whole launch; the weights stream through
// double-buffered LDS in 64-column chunks, and every weight fragment read from LDS feeds two
// MFMAs (one per row tile).  The weights are the A operand, so a lane ends up holding four
// consecutive output columns of one row: stores are 8-byte vectors wherever the destination
// keeps those columns contiguous.  Destinations are f16 with 32-bit element offsets.
constexpr int LP_ROWS = RG_WAVES * 32;

__device__ __forceinline__ int dst_row32(const Dst& d, int row) {
  const unsigned q = (unsigned)d.Q;
  const unsigned b = (unsigned)row / q, n = (unsigned)row - b * q;
  return (int)b * (int)d.sB + (int)n * (int)d.sN;
}
__device__ __forceinline__ int dst_col32(const Dst& d, int col) {
  const unsigned dd = (unsigned)d.D;
  const unsigned h = (unsigned)col / dd, e = (unsigned)col - h * dd;
  return (int)h * (int)d.sH + (int)e * (int)d.sD;
}

// Four consecutive columns cb..cb+3 of one row: one 8-byte store when they are contiguous in
// the destination, else element stores (columns >= ncols are dropped).
__device__ __forceinline__ void store_cols4(const Group& G, int rowpart, int cb, const float (&v)[4]) {
  _Float16* out = static_cast<_Float16*>(G.dst.ptr);
  const unsigned dd = (unsigned)G.dst.D;
  const unsigned e0 = (unsigned)cb % dd;
  if (G.dst.sD == 1 && cb + 3 < G.ncols && e0 + 3 < dd && ((rowpart + dst_col32(G.dst, cb)) & 3) == 0) {
    h4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (_Float16)v[i];
    *reinterpret_cast<h4*>(out + rowpart + dst_col32(G.dst, cb)) = o;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (cb + i < G.ncols) out[rowpart + dst_col32(G.dst, cb + i)] = (_Float16)v[i];
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

  // this wave's two 16-row tiles, LayerNorm'd into B fragments
  const int rbase = blockIdx.x * LP_ROWS + wave * 32;
  h8 xb[2][KS];
  int srow[2];
  bool rvalid[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int myrow = rbase + tt * 16 + r16;
    rvalid[tt] = myrow < p.rows;
    const int lrow = rvalid[tt] ? myrow : 0;
    srow[tt] = p.rmB > 0 ? (lrow % p.rmQ) * p.rmB + lrow / p.rmQ : lrow;
  }
  {
    FragTile<ACT, KS> t0, t1;
    frag_load_row(t0, p.x, (size_t)srow[0], p.C, lane);
    frag_load_row(t1, p.x, (size_t)srow[1], p.C, lane);
    chunk_store<KP, NREG>(Ws[0], regs, tid);
    __syncthreads();  // Gs and chunk 0 staged
    frag_ln_raw2(t0, t1, xb[0], xb[1], p.C, Gs, Gs + KP, p.eps, p.fast_var, lane);
  }
  float rm[2] = {1.f, 1.f};
  if (p.rowmask) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) rm[tt] = p.rowmask[srow[tt]];
  }

  for (int ci = 0; ci < nchunks; ++ci) {
    const _Float16* W = Ws[ci & 1];
    if (ci + 1 < nchunks) chunk_load<KP, NREG>(p, ci + 1, regs, tid);
    f4 acc[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[tt][t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      h8 w[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) w[t] = *reinterpret_cast<const h8*>(W + (t * 16 + r16) * LDW + 32 * j + kq);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc[0][t] = mfma16(w[t], xb[0][j], acc[0][t]);
        acc[1][t] = mfma16(w[t], xb[1][j], acc[1][t]);
      }
      __builtin_amdgcn_sched_barrier(0);   // one k-step's weight fragments live at a time
    }
    int gi, c0;
    chunk_of(p, ci, gi, c0);
    const Group& G = p.g[gi];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      if (!rvalid[tt]) continue;
      const int rowpart = dst_row32(G.dst, rbase + tt * 16 + r16);
      if (G.op == OP_SWIGLU) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int cb = c0 + t * 16 + 4 * g4;
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int c = cb + i < G.ncols ? cb + i : 0;
            const float gt = (acc[tt][t][i] + (G.bias0 ? G.bias0[c] : 0.f)) * G.scale;
            const float vl = (acc[tt][t + 2][i] + (G.bias1 ? G.bias1[c] : 0.f)) * G.scale;
            v[i] = gt * sigmoidf_(gt) * vl;
          }
          if (cb < G.ncols) store_cols4(G, rowpart, cb, v);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int cb = c0 + t * 16 + 4 * g4;
          if (cb >= G.ncols) continue;
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int c = cb + i < G.ncols ? cb + i : 0;
            float y = (acc[tt][t][i] + (G.bias0 ? G.bias0[c] : 0.f)) * G.scale;
            if (G.op == OP_SIGMOID) y = sigmoidf_(y);
            else if (G.op == OP_RELU) y = fmaxf(y, 0.f);
            else if (G.op == OP_ROWMASK) y *= rm[tt];
            v[i] = y;
          }
          store_cols4(G, rowpart, cb, v);
          __builtin_amdgcn_sched_barrier(0);   // one column tile's epilogue at a time
        }
      }
    }
    if (ci + 1 < nchunks) {
      chunk_store<KP, NREG>(Ws[(ci + 1) & 1], regs, tid);
      __syncthreads();
    }
  }
}

static int lnproj_ks(int C) { return C <= 32 ? 1 : C <= 64 ? 2 : C <= 128 ? 4 : C <= 256 ? 8 : 12; }

static int lnproj_chunks(const LnProjParams& p) {
  int n = 0;
  for (int g = 0; g < p.ngroups; ++g) {
    const int w = p.g[g].op == OP_SWIGLU ? 32 : 64;
    n += (p.g[g].ncols + w - 1) / w;
  }
  return n;
}

size_t lnproj_packed_bytes(const LnProjParams& p) {
  return (size_t)lnproj_chunks(p) * 64 * 32 * lnproj_ks(p.C) * sizeof(_Float16);
}

int launch_lnproj(lf_context* ctx, LnProjParams p, int act, void* packed, const char* label, bool decode) {
  if (p.C > 384) return set_error(LF_ERR_INVALID, std::string(label) + ": LayerNorm width above 384");
  if (p.rows <= 0) return LF_OK;
  if (!packed) return set_error(LF_ERR_INVALID, std::string(label) + ": no packed-weight workspace");
  for (int g = 0; g < p.ngroups; ++g) {
    const Dst& d = p.g[g].dst;
    if (d.dtype != DT_F16) return set_error(LF_ERR_INVALID, std::string(label) + ": lnproj writes f16 only");
    const long long span = (long long)((p.rows - 1) / d.Q) * d.sB + (long long)std::min(p.rows - 1, d.Q - 1) * d.sN +
                           (long long)((p.g[g].ncols - 1) / d.D) * d.sH +
                           (long long)std::min(p.g[g].ncols - 1, d.D - 1) * d.sD;
    if (span >= (1LL << 31)) return set_error(LF_ERR_INVALID, std::string(label) + ": destination above 2^31 elements");
  }
  // decode every group's weights into chunk order
  const int KP = 32 * lnproj_ks(p.C);
  WView views[2 * MAX_GROUPS];
  int W[2 * MAX_GROUPS], off[2 * MAX_GROUPS];
  long long row0[2 * MAX_GROUPS];
  int nv = 0;
  long long rows_done = 0;
  for (int g = 0; g < p.ngroups; ++g) {
    const Group& G = p.g[g];
    const bool paired = G.op == OP_SWIGLU;
    const int w = paired ? 32 : 64;
    views[nv] = G.w0;
    W[nv] = w;
    off[nv] = 0;
    row0[nv++] = rows_done;
    if (paired) {
      views[nv] = G.w1;
      W[nv] = 32;
      off[nv] = 32;
      row0[nv++] = rows_done;
    }
    rows_done += (long long)(G.ncols + w - 1) / w * 64;
  }
  p.wpk = static_cast<const _Float16*>(packed);
  if (decode)
    LF_TRY(expand_packed(ctx, views, W, off, row0, nv, static_cast<_Float16*>(packed), KP,
                       (std::string(label) + ".expand").c_str()));
  const int ks = lnproj_ks(p.C);
  dim3 grid((p.rows + LP_ROWS - 1) / LP_ROWS);
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
