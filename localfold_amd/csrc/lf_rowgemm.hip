// Generic row GEMMs (see lf_rowgemm.h): lnproj (LayerNorm + grouped projections) and
// rowgemm (f16 rows x streamed weights + bias / ReLU / row denominator / residual).
#include <algorithm>

#include "lf_rowgemm.h"

namespace lf {

constexpr int LP_ROWS = 8 * 32;         // 8 waves x 32 rows

// Loads chunk ci of the packed weights (a contiguous [64][KP] f16 block) into registers
// (NREG 16-byte words per thread), to be stored into LDS later.
template <int KP, int NREG>
__device__ __forceinline__ void chunk_load(const LnProjParams& p, int ci, u32x4 (&regs)[NREG], int tid) {
  const u32x4* src = reinterpret_cast<const u32x4*>(p.wpk + (size_t)ci * 64 * KP);
#pragma unroll
  for (int r = 0; r < NREG; ++r) {
    const int i = tid + r * 512;
    regs[r] = i < 64 * KP / 8 ? src[i] : u32x4{0u, 0u, 0u, 0u};
  }
}

template <int KP, int NREG>
__device__ __forceinline__ void chunk_store(_Float16* Ws, const u32x4 (&regs)[NREG], int tid) {
  constexpr int SEGS = KP / 8, LDW = KP + 8;
#pragma unroll
  for (int r = 0; r < NREG; ++r) {
    const int i = tid + r * 512;
    const int n = i / SEGS, seg = i - n * SEGS;
    if (n < 64) *reinterpret_cast<u32x4*>(Ws + n * LDW + seg * 8) = regs[r];
  }
}

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

// Per-chunk epilogue table: destination column offsets (-1 past the group's columns) and
// scaled biases of the chunk's logical columns (64, or 32 gate/value pairs for SwiGLU).  Every
// wave loads the next chunk's biases with the weight prefetch (so the one wait for that
// prefetch covers them) and wave 0 writes the table.
struct ChunkTab {
  int cofs[64];
  float b0[64];
  float b1[64];
};

__device__ __forceinline__ void chunk_tab_load(const LnProjParams& p, int g, int c0, int lane, float& b0, float& b1) {
  const Group& G = p.g[g];
  const int c = min(c0 + lane, G.ncols - 1);
  b0 = G.bias0 ? G.bias0[c] : 0.f;
  b1 = G.bias1 ? G.bias1[c] : 0.f;
}

__device__ __forceinline__ void chunk_tab_put(ChunkTab& T, const LnProjParams& p, int g, int c0, int lane, float b0,
                                              float b1) {
  const Group& G = p.g[g];
  const int c = c0 + lane;
  const bool ok = c < G.ncols;
  T.cofs[lane] = ok ? dst_col32(G.dst, c) : -1;
  T.b0[lane] = ok ? b0 * G.scale : 0.f;
  T.b1[lane] = ok ? b1 * G.scale : 0.f;
}

// Round-to-nearest-even f16 of 4 floats (two v_cvt_pk_f16_f32).
__device__ __forceinline__ h4 pack_h4(const float (&v)[4]) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const h2 lo = __builtin_convertvector((f2){v[0], v[1]}, h2);
  const h2 hi = __builtin_convertvector((f2){v[2], v[3]}, h2);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
}

// Four consecutive logical columns of one row.  When every lane of the wave has its four
// columns valid, contiguous and 8-byte aligned in the destination (the usual case) all
// lanes take one vector store, decided by a wave-uniform vote; otherwise each lane stores
// its valid elements.
__device__ __forceinline__ void store4(_Float16* out, int rowpart, int4 co, bool row_ok, const float (&v)[4]) {
  const bool vec = row_ok && co.x >= 0 && co.y == co.x + 1 && co.z == co.x + 2 && co.w == co.x + 3 &&
                   ((rowpart + co.x) & 3) == 0;
  if (__all(vec)) {
    *reinterpret_cast<h4*>(out + rowpart + co.x) = pack_h4(v);
  } else if (row_ok) {
    if (co.x >= 0) out[rowpart + co.x] = (_Float16)v[0];
    if (co.y >= 0) out[rowpart + co.y] = (_Float16)v[1];
    if (co.z >= 0) out[rowpart + co.z] = (_Float16)v[2];
    if (co.w >= 0) out[rowpart + co.w] = (_Float16)v[3];
  }
}

// Four consecutive rows of one logical column (the transposed tile): one vector store when
// every lane's rows are valid, contiguous and 8-byte aligned in the destination.
__device__ __forceinline__ void store4t(_Float16* out, int4 rp, int co, int nrow, const float (&v)[4]) {
  const bool vec = nrow == 4 && co >= 0 && rp.y == rp.x + 1 && rp.z == rp.x + 2 && rp.w == rp.x + 3 &&
                   ((rp.x + co) & 3) == 0;
  if (__all(vec)) {
    *reinterpret_cast<h4*>(out + rp.x + co) = pack_h4(v);
  } else if (co >= 0) {
    if (nrow > 0) out[rp.x + co] = (_Float16)v[0];
    if (nrow > 1) out[rp.y + co] = (_Float16)v[1];
    if (nrow > 2) out[rp.z + co] = (_Float16)v[2];
    if (nrow > 3) out[rp.w + co] = (_Float16)v[3];
  }
}

// Half a chunk's GEMM for both row tiles: acc[tt][u] is the 16x16 tile of row tile tt and
// column tile tb + u*ts -- tiles 2th, 2th+1 (adjacent columns, so a half writes whole 64-byte
// runs of a destination row and no line is left half-written for the other half), or th, th+2
// for SwiGLU (gate and value).  TR puts the activation rows first (lane: rows 4*g4+i of column
// r16), else the weight columns.
template <int KS, bool TR>
__device__ __forceinline__ void lnproj_mma(f4 (&acc)[2][2], const _Float16* W, const h8 (&xb)[2][KS], int tb, int ts,
                                           int r16, int kq) {
  constexpr int LDW = KS * 32 + 8;
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    h8 w[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
      w[u] = *reinterpret_cast<const h8*>(W + ((tb + ts * u) * 16 + r16) * LDW + 32 * j + kq);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        acc[tt][u] = TR ? mfma16(xb[tt][j], w[u], acc[tt][u]) : mfma16(w[u], xb[tt][j], acc[tt][u]);
    }
  }
}

// Half a chunk's epilogue for a wave: y = op(acc * scale + bias) for column tiles 2th and 2th+1
// (SwiGLU: tile th = gate, th + 2 = value, one output tile), stored as f16.
// The op and the tile orientation are template parameters, dispatched once per chunk.
struct EpiArgs {
  _Float16* out;
  const int* Rp;        // destination row offsets of the block rows
  const float* Rm;      // OP_ROWMASK multipliers of the block rows
  const ChunkTab* T;
  float scale;
  int rows_left;        // rows of the block that exist (may exceed LP_ROWS)
  int wrow;             // the wave's first block row
  int r16, g4;
};

template <int OP>
__device__ __forceinline__ float lnproj_op(float y, float value, float rmul) {
  if (OP == OP_SWIGLU) return y * sigmoidf_(y) * value;
  if (OP == OP_SIGMOID) return sigmoidf_(y);
  if (OP == OP_RELU) return fmaxf(y, 0.f);
  if (OP == OP_ROWMASK) return y * rmul;
  return y;
}

template <int OP, bool TR, bool FAST>
__device__ __forceinline__ void lnproj_epilogue(const f4 (&acc)[2][2], int th, const EpiArgs& a) {
  const ChunkTab& T = *a.T;
  {
#pragma unroll
    for (int u = 0; u < (OP == OP_SWIGLU ? 1 : 2); ++u) {
      const int t = OP == OP_SWIGLU ? th : 2 * th + u;
      if (TR) {
        const int col = t * 16 + a.r16, co = T.cofs[col];
        const float b0 = T.b0[col], b1 = T.b1[col];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int r0 = a.wrow + tt * 16 + 4 * a.g4;
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            v[i] = lnproj_op<OP>(fmaf(acc[tt][u][i], a.scale, b0), fmaf(acc[tt][1][i], a.scale, b1),
                                 OP == OP_ROWMASK ? a.Rm[r0 + i] : 1.f);
          if (FAST) *reinterpret_cast<h4*>(a.out + (uint32_t)(a.Rp[r0] + co)) = pack_h4(v);
          else store4t(a.out, *reinterpret_cast<const int4*>(&a.Rp[r0]), co, min(4, max(0, a.rows_left - r0)), v);
        }
      } else {
        const int cc = t * 16 + 4 * a.g4;
        const int4 co = *reinterpret_cast<const int4*>(&T.cofs[cc]);
        const float4 bb = *reinterpret_cast<const float4*>(&T.b0[cc]);
        const float b0s[4] = {bb.x, bb.y, bb.z, bb.w};
        float b1s[4] = {0.f, 0.f, 0.f, 0.f};
        if (OP == OP_SWIGLU) {
          const float4 bv = *reinterpret_cast<const float4*>(&T.b1[cc]);
          b1s[0] = bv.x; b1s[1] = bv.y; b1s[2] = bv.z; b1s[3] = bv.w;
        }
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int r = a.wrow + tt * 16 + a.r16;
          const float rmul = OP == OP_ROWMASK ? a.Rm[r] : 1.f;
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            v[i] = lnproj_op<OP>(fmaf(acc[tt][u][i], a.scale, b0s[i]),
                                 OP == OP_SWIGLU ? fmaf(acc[tt][1][i], a.scale, b1s[i]) : 0.f, rmul);
          if (FAST) *reinterpret_cast<h4*>(a.out + (uint32_t)(a.Rp[r] + co.x)) = pack_h4(v);
          else store4(a.out, a.Rp[r], co, r < a.rows_left, v);
        }
      }
      __builtin_amdgcn_sched_barrier(0);   // one column tile's epilogue at a time
    }
  }
}

// 512 threads = 8 waves x 32 rows; the accumulators cover half a chunk at a time and the two
// row tiles are LayerNorm'd one after the other.  With K <= 128 the kernel fits 128 VGPRs, so
// two blocks share a CU (the LDS holds two); wider rows keep 256 (one block), since at 128 the
// 64 registers of LayerNorm'd activations push the loop into spills.
template <int ACT, int KS>
__global__ __launch_bounds__(512, KS <= 4 ? 4 : 2) void lnproj_kernel(LnProjParams p) {
  constexpr int KP = KS * 32, LDW = KP + 8;
  constexpr int NREG = (64 * KP / 8 + 511) / 512;
  // NB chunks per LDS buffer, one block barrier per NB chunks: two at K = 256 (the block is
  // alone on its CU there, and two buffers of two chunks fit), one elsewhere
  constexpr int NB = KS == 8 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) _Float16 Ws[2][NB][64 * LDW];
  __shared__ __attribute__((aligned(16))) float Gs[2 * KP];
  __shared__ __attribute__((aligned(16))) ChunkTab Tab[2][NB];
  __shared__ int Rp[MAX_GROUPS][LP_ROWS];   // destination row offsets per group and block row
  __shared__ float Rm[LP_ROWS];             // OP_ROWMASK multipliers of the block rows
  __shared__ int Cg[MAX_CHUNKS], Cc[MAX_CHUNKS], Cf[MAX_CHUNKS];   // chunk -> group, first column, fast
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  stage_vec(Gs, p.ln_s, p.C, 1.f, KP, tid, 512);
  stage_vec(Gs + KP, p.ln_o, p.C, 0.f, KP, tid, 512);
  // blockIdx.y takes a contiguous range of the column chunks (few rows: more blocks)
  const int per = (p.nchunks + (int)gridDim.y - 1) / (int)gridDim.y;
  const int ci0 = (int)blockIdx.y * per, ci1 = min(p.nchunks, ci0 + per);
  if (ci0 >= ci1) return;
  for (int i = tid; i < p.nchunks; i += 512) {
    Cg[i] = p.chunk_group[i];
    Cc[i] = p.chunk_c0[i];
    Cf[i] = p.chunk_fast[i];
  }
  u32x4 regs[NREG];
  chunk_load<KP, NREG>(p, ci0, regs, tid);
  {
    const int g = __builtin_amdgcn_readfirstlane(p.chunk_group[ci0]);
    const int c0 = __builtin_amdgcn_readfirstlane(p.chunk_c0[ci0]);
    float b0, b1;
    chunk_tab_load(p, g, c0, lane, b0, b1);
    if (wave == 0) chunk_tab_put(Tab[0][0], p, g, c0, lane, b0, b1);
  }
  const int row_block = blockIdx.x * LP_ROWS;
  for (int i = tid; i < p.ngroups * LP_ROWS; i += 512) {
    const int g = i / LP_ROWS, r = i - g * LP_ROWS;
    Rp[g][r] = row_block + r < p.rows ? dst_row32(p.g[g].dst, row_block + r) : 0;
  }
  if (p.rowmask && tid < LP_ROWS) {
    const int r = row_block + tid;
    Rm[tid] = r < p.rows ? p.rowmask[p.rmB > 0 ? (r % p.rmQ) * p.rmB + r / p.rmQ : r] : 0.f;
  }

  // this wave's two 16-row tiles, LayerNorm'd into B fragments
  const int rbase = row_block + wave * 32;
  auto srow_of = [&](int r) { return p.rmB > 0 ? (r % p.rmQ) * p.rmB + r / p.rmQ : r; };
  h8 xb[2][KS];
  chunk_store<KP, NREG>(Ws[0][0], regs, tid);
  if constexpr (NB == 2) {   // the second chunk of the first pair (clamped)
    const int c2 = min(ci0 + 1, ci1 - 1);
    chunk_load<KP, NREG>(p, c2, regs, tid);
    const int g = __builtin_amdgcn_readfirstlane(p.chunk_group[c2]);
    const int c0 = __builtin_amdgcn_readfirstlane(p.chunk_c0[c2]);
    float b0, b1;
    chunk_tab_load(p, g, c0, lane, b0, b1);
    chunk_store<KP, NREG>(Ws[0][1], regs, tid);
    if (wave == 0) chunk_tab_put(Tab[0][1], p, g, c0, lane, b0, b1);
  }
  __syncthreads();  // Gs, the first chunks, their tables and the row offsets staged
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int myrow = rbase + tt * 16 + r16;
    FragTile<ACT, KS> t0;
    frag_load_row(t0, p.x, (size_t)srow_of(myrow < p.rows ? myrow : 0), p.C, lane);
    frag_ln_raw1(t0, xb[tt], p.C, Gs, Gs + KP, p.eps, p.fast_var, lane);
    // one raw tile live at a time: without the barrier the second tile's loads are hoisted
    // above the first tile's LayerNorm, and with f32 rows (64 VGPRs a tile at C = 256) the
    // prologue spilled to scratch
    __builtin_amdgcn_sched_barrier(0);
  }

  for (int ci = ci0; ci < ci1; ++ci) {
    // chunk ci in slot rel % NB of buffer (rel / NB) % 2; chunk ci + NB goes to the same slot
    // of the other buffer, which every wave left at the previous barrier
    const int rel = ci - ci0, kb = (rel / NB) & 1, sl = rel % NB;
    const _Float16* W = Ws[kb][sl];
    const ChunkTab& T = Tab[kb][sl];
    // unconditional (the last chunks reload the last one): with no branch around the
    // prefetch the compiler's wait before the LDS store counts only this iteration's stores
    const int cn = min(ci + NB, ci1 - 1);
    chunk_load<KP, NREG>(p, cn, regs, tid);
    // wave-uniform by construction; readfirstlane lets the compiler keep them in SGPRs
    const int gn = __builtin_amdgcn_readfirstlane(Cg[cn]), cn0 = __builtin_amdgcn_readfirstlane(Cc[cn]);
    float tb0, tb1;
    chunk_tab_load(p, gn, cn0, lane, tb0, tb1);
    const int gi = __builtin_amdgcn_readfirstlane(Cg[ci]);
    const Group& G = p.g[gi];
    const bool tr = __builtin_amdgcn_readfirstlane(G.tr) != 0;
    // whole-block, whole-chunk, vector-aligned: the epilogue stores without checks
    const bool fast = __builtin_amdgcn_readfirstlane(Cf[ci]) != 0 && p.rows - row_block >= LP_ROWS;
    _Float16* out = static_cast<_Float16*>(G.dst.ptr);
    const float scale = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(G.scale)));
    const int op = __builtin_amdgcn_readfirstlane(G.op);

    // per half: the GEMM, then (after half 0) the next chunk into the other LDS buffer -- its
    // loads are waited for before this chunk's first store, so that wait never covers this
    // chunk's stores -- then the half's epilogue
    const EpiArgs ea{out, Rp[gi], Rm, &T, scale, p.rows - row_block, wave * 32, r16, g4};
#pragma unroll
    for (int th = 0; th < 2; ++th) {
      f4 acc[2][2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) acc[tt][0] = acc[tt][1] = f4{0.f, 0.f, 0.f, 0.f};
      const int tb = op == OP_SWIGLU ? th : 2 * th, ts = op == OP_SWIGLU ? 2 : 1;
      if (tr) lnproj_mma<KS, true>(acc, W, xb, tb, ts, r16, kq);
      else lnproj_mma<KS, false>(acc, W, xb, tb, ts, r16, kq);
      if (th == 0) {
        chunk_store<KP, NREG>(Ws[kb ^ 1][sl], regs, tid);
        if (wave == 0) chunk_tab_put(Tab[kb ^ 1][sl], p, gn, cn0, lane, tb0, tb1);
      }
      __builtin_amdgcn_sched_barrier(0);
#define LF_EPI(OPV)                                                                          \
  if (fast) tr ? lnproj_epilogue<OPV, true, true>(acc, th, ea) : lnproj_epilogue<OPV, false, true>(acc, th, ea); \
  else tr ? lnproj_epilogue<OPV, true, false>(acc, th, ea) : lnproj_epilogue<OPV, false, false>(acc, th, ea);
      switch (op) {
        case OP_SIGMOID: LF_EPI(OP_SIGMOID) break;
        case OP_RELU: LF_EPI(OP_RELU) break;
        case OP_SWIGLU:
          tr ? lnproj_epilogue<OP_SWIGLU, true, false>(acc, th, ea) : lnproj_epilogue<OP_SWIGLU, false, false>(acc, th, ea);
          break;
        case OP_ROWMASK: LF_EPI(OP_ROWMASK) break;
        default: LF_EPI(OP_STORE) break;
      }
#undef LF_EPI
    }
    if (sl == NB - 1) __syncthreads();   // block-uniform
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

int lnproj_prepare(lf_context* ctx, LnProjParams& p, void* packed, ExpandList* xl, const char* label) {
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
    const bool cols_contig = d.D % 4 == 0 && d.sD == 1;
    const bool rows_contig = d.sN == 1 && d.Q % 4 == 0;
    p.g[g].tr = !cols_contig && rows_contig;
    const bool aligned8 = (reinterpret_cast<uintptr_t>(d.ptr) & 7) == 0 && d.sB % 4 == 0 && d.sH % 4 == 0;
    p.g[g].vec = aligned8 && (p.g[g].tr ? d.sD % 4 == 0 : cols_contig && d.sN % 4 == 0);
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
  p.nchunks = 0;
  for (int g = 0; g < p.ngroups; ++g) {
    const int w = p.g[g].op == OP_SWIGLU ? 32 : 64;
    for (int c0 = 0; c0 < p.g[g].ncols; c0 += w) {
      if (p.nchunks == MAX_CHUNKS) return set_error(LF_ERR_INVALID, std::string(label) + ": too many output columns");
      if (c0 > 32767) return set_error(LF_ERR_INVALID, std::string(label) + ": group wider than 32767 columns");
      p.chunk_group[p.nchunks] = g;
      p.chunk_fast[p.nchunks] = p.g[g].vec && c0 + w <= p.g[g].ncols;
      p.chunk_c0[p.nchunks++] = c0;
    }
  }
  if (xl)
    LF_TRY(expand_add_packed(ctx, *xl, views, W, off, row0, nv, static_cast<_Float16*>(packed), KP,
                             (std::string(label) + ".expand").c_str()));
  return LF_OK;
}

int lnproj_run(lf_context* ctx, const LnProjParams& p, int act, const char* label) {
  if (p.rows <= 0) return LF_OK;
  const int ks = lnproj_ks(p.C);
  // few row blocks (the single track): split the column chunks over grid.y so about two blocks
  // per CU run; each re-does the LayerNorm of its rows
  const int xb = (p.rows + LP_ROWS - 1) / LP_ROWS;
  const int ysplit = std::max(1, std::min(p.nchunks, (2 * ctx->num_cus) / xb));
  dim3 grid(xb, ysplit);
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

int launch_lnproj(lf_context* ctx, LnProjParams p, int act, void* packed, const char* label, bool decode) {
  if (p.rows <= 0) return LF_OK;
  ExpandList xl;
  LF_TRY(lnproj_prepare(ctx, p, packed, decode ? &xl : nullptr, label));
  LF_TRY(expand_flush(ctx, xl, (std::string(label) + ".expand").c_str()));
  return lnproj_run(ctx, p, act, label);
}

// ---------------------------------------------------------------------------------------

// rowgemm: block tile 128 rows x (32 * NT) columns; 8 waves = 4 row groups (32 rows, two
// 16-row tiles) x 2 column halves (16 * NT columns).  A rows are read from global straight
// into MFMA B fragments (each A element leaves HBM once; the other column half hits L2), one
// 64-deep K slice ahead; the weights stream through double-buffered LDS one K slice at a
// time.  The weights are the A operand, so a lane holds 4 consecutive output columns of one
// row and the epilogue (bias, ReLU, row denominator, residual) works on 4-element vectors.
constexpr int RB_K = 64, RB_LDW = RB_K + 8;

template <int DACT>
__device__ __forceinline__ void ld4(const void* base, int idx, float (&v)[4]) {
  if constexpr (DACT == DT_F32) {
    const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else if constexpr (DACT == DT_F16) {
    const h4 q = *reinterpret_cast<const h4*>(static_cast<const _Float16*>(base) + idx);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)q[i];
  } else {
    const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
    v[0] = __uint_as_float(q.x << 16); v[1] = __uint_as_float(q.x & 0xffff0000u);
    v[2] = __uint_as_float(q.y << 16); v[3] = __uint_as_float(q.y & 0xffff0000u);
  }
}

template <int DACT>
__device__ __forceinline__ void st4(void* base, int idx, const float (&v)[4]) {
  if constexpr (DACT == DT_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + idx) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (DACT == DT_F16) {
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

template <int DACT, int NT>
__global__ __launch_bounds__(512) void rowgemm_kernel(RowGemmParams p) {
  constexpr int BN = 32 * NT;                 // block columns
  constexpr int WREG = (BN * RB_K / 8 + 511) / 512;
  __shared__ __attribute__((aligned(16))) _Float16 Ws[2][BN * RB_LDW];
  __shared__ __attribute__((aligned(16))) float Bs[BN];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  const int wr = wave >> 1, wc = wave & 1;    // row group, column half
  const int col0 = blockIdx.y * BN;           // block's first output column
  const int rbase = blockIdx.x * 128 + wr * 32;
  const int nslices = (p.K + RB_K - 1) / RB_K;
  for (int i = tid; i < BN; i += 512) Bs[i] = (p.bias && col0 + i < p.N) ? p.bias[col0 + i] : 0.f;

  // weights of slice s: [BN cols][64 k] of the expanded E[n][kp]
  auto wload = [&](int sl, uint4 (&regs)[WREG]) {
#pragma unroll
    for (int r = 0; r < WREG; ++r) {
      const int i = tid + r * 512, n = i >> 3, seg = i & 7;
      const int col = col0 + n, k = sl * RB_K + seg * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (n < BN && col < p.w.N && k < p.w.kp) v = *reinterpret_cast<const uint4*>(p.w.p + (size_t)col * p.w.kp + k);
      regs[r] = v;
    }
  };
  auto wstore = [&](_Float16* W, const uint4 (&regs)[WREG]) {
#pragma unroll
    for (int r = 0; r < WREG; ++r) {
      const int i = tid + r * 512, n = i >> 3, seg = i & 7;
      if (n < BN) *reinterpret_cast<uint4*>(W + n * RB_LDW + seg * 8) = regs[r];
    }
  };
  // A fragments of slice s for both row tiles (rows past the end read row 0; K is a multiple
  // of 8, so an 8-element run is either inside K or wholly past it)
  const _Float16* arow[2];
  bool rvalid[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int row = rbase + tt * 16 + r16;
    rvalid[tt] = row < p.rows;
    arow[tt] = p.A + (size_t)(rvalid[tt] ? row : 0) * p.K;
  }
  auto aload = [&](int sl, h8 (&a)[2][2]) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int k = sl * RB_K + 32 * j + kq;
        a[tt][j] = k < p.K ? *reinterpret_cast<const h8*>(arow[tt] + k) : h8{0, 0, 0, 0, 0, 0, 0, 0};
      }
  };

  uint4 regs[WREG];
  h8 acur[2][2], anext[2][2];
  wload(0, regs);
  aload(0, acur);
  wstore(Ws[0], regs);
  __syncthreads();

  f4 acc[2][NT];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[tt][t] = f4{0.f, 0.f, 0.f, 0.f};

  for (int sl = 0; sl < nslices; ++sl) {
    if (sl + 1 < nslices) {
      aload(sl + 1, anext);
      wload(sl + 1, regs);
    }
    const _Float16* W = Ws[sl & 1] + (wc * 16 * NT) * RB_LDW;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const h8 w = *reinterpret_cast<const h8*>(W + (t * 16 + r16) * RB_LDW + 32 * j + kq);
        acc[0][t] = mfma16(w, acur[0][j], acc[0][t]);
        acc[1][t] = mfma16(w, acur[1][j], acc[1][t]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (sl + 1 < nslices) {
      wstore(Ws[(sl + 1) & 1], regs);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int j = 0; j < 2; ++j) acur[tt][j] = anext[tt][j];
      __syncthreads();
    }
  }

  // epilogue: lane holds columns c..c+3 (c = col0 + wc*16*NT + 16t + 4*g4) of row rbase + 16tt + r16.
  // Every row denominator and residual is loaded before the first store: the vector-memory
  // counter completes in order, so a load issued after stores would wait for them as well.
  int rowpart[2];
  float den[2];
  typename Raw4v<DACT>::T rr[2][NT];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int row = rvalid[tt] ? rbase + tt * 16 + r16 : 0;
    const unsigned q = (unsigned)p.dst.Q;
    const unsigned b = (unsigned)row / q, n = (unsigned)row - b * q;
    rowpart[tt] = (int)b * (int)p.dst.sB + (int)n * (int)p.dst.sN;
    den[tt] = p.rowden ? p.rowden[row] : 1.f;
    if (p.resid) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int c = min(col0 + wc * 16 * NT + t * 16 + 4 * g4, p.N - 4);   // clamped: never skipped
        rr[tt][t] = Raw4v<DACT>::load(p.resid, rowpart[tt] + c);
      }
    }
  }
  // take every loaded value into registers here, while only loads are outstanding (the
  // stores below are conditional, so the compiler cannot count them and would wait for all)
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    asm volatile("" : "+v"(den[tt]));
    if (p.resid) {
#pragma unroll
      for (int t = 0; t < NT; ++t) Raw4v<DACT>::touch(rr[tt][t]);
    }
  }
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    if (!rvalid[tt]) continue;
    const float inv = 1.f / den[tt];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int cl = wc * 16 * NT + t * 16 + 4 * g4;   // column within the block
      const int c = col0 + cl;
      if (c >= p.N) continue;
      const float4 bb = *reinterpret_cast<const float4*>(&Bs[cl]);
      const float bs[4] = {bb.x, bb.y, bb.z, bb.w};
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float y = acc[tt][t][i] + bs[i];
        if (p.op == OP_RELU) y = fmaxf(y, 0.f);
        v[i] = y * inv;
      }
      if (p.resid) {
        float r[4];
        Raw4v<DACT>::unpack(rr[tt][t], r);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += r[i];
      }
      st4<DACT>(p.dst.ptr, rowpart[tt] + c, v);
    }
  }
}

// Weight-resident form for K = 32 KS <= 256 and N = 64 NP <= 256 (the attention output
// projections): a block stages the whole W (N x K f16, up to 132 KB) in LDS once -- copied from
// the f16 expansion, or decoded from the stored codes (int8 / int5 / f16 runs, the codec
// arithmetic of lf_gemm.h) -- and
// each of its 8 waves then walks 16-row tiles w, w + nw, ... with no block barrier.  A tile's
// A fragments come straight from memory into registers (the next tile's are loaded during
// this one's MFMAs), its residual and row denominator are loaded at the top of the tile, and
// the columns run in passes of 64 (4 accumulator tiles), each followed by its epilogue.
// W is the MFMA A operand, so a lane holds 4 consecutive columns of one row: one 8- or
// 16-byte store per column tile.  Rows past the end are clamped for the loads and not stored.
template <int DACT, int KS, int NP, int NWV>
__global__ __launch_bounds__(64 * NWV) void rowgemm_res_kernel(RowGemmParams p) {
  constexpr int NT = 64 * NWV, K = 32 * KS, N = 64 * NP, LDW = K + 8;
  __shared__ __attribute__((aligned(16))) _Float16 Ws[N * LDW];
  __shared__ __attribute__((aligned(16))) float Bs[N];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  const int ntiles = (p.rows + 15) >> 4, nw = (int)gridDim.x * NWV;
  auto aload = [&](int tl, h8 (&a)[KS]) __attribute__((always_inline)) {
    const int row = min(tl * 16 + r16, p.rows - 1);
    const _Float16* ar = p.A + (size_t)row * p.K + kq;
#pragma unroll
    for (int j = 0; j < KS; ++j) a[j] = *reinterpret_cast<const h8*>(ar + 32 * j);
  };
  int tile = (int)blockIdx.x * NWV + wave;
  h8 a[KS];
  aload(tile < ntiles ? tile : 0, a);
  if (p.wview) {
    // the whole W decoded from its stored codes (zeros past the view's columns)
    stage_view(Ws, LDW, p.wv, N, 0, K, 1.f, tid, NT);
  } else {
    // the whole W, 16-byte pieces of E[n][k] (row pitch p.w.kp >= K)
    for (int i = tid; i < N * K / 8; i += NT) {
      const int n = i / (K / 8), k = (i - n * (K / 8)) * 8;
      const uint4 v = n < p.w.N ? *reinterpret_cast<const uint4*>(p.w.p + (size_t)n * p.w.kp + k) : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(Ws + n * LDW + k) = v;
    }
  }
  for (int i = tid; i < N; i += NT) Bs[i] = (p.bias && i < p.N) ? p.bias[i] : 0.f;
  __syncthreads();
  for (; tile < ntiles; tile += nw) {
    const int row = tile * 16 + r16;
    const bool valid = row < p.rows;
    const int rc = valid ? row : p.rows - 1;
    const unsigned q = (unsigned)p.dst.Q;
    const unsigned b = (unsigned)rc / q, nn = (unsigned)rc - b * q;
    const int rowpart = (int)b * (int)p.dst.sB + (int)nn * (int)p.dst.sN;
    typename Raw4v<DACT>::T rr[NP][4];
    if (p.resid) {
#pragma unroll
      for (int pp = 0; pp < NP; ++pp)
#pragma unroll
        for (int t = 0; t < 4; ++t) rr[pp][t] = Raw4v<DACT>::load(p.resid, rowpart + pp * 64 + t * 16 + 4 * g4);
    }
    const float inv = p.rowden ? 1.f / p.rowden[rc] : 1.f;
    // the next tile's A fragments (clamped, never skipped), after this tile's other loads
    const int nt = tile + nw < ntiles ? tile + nw : tile;
    h8 an[KS];
    aload(nt, an);
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      f4 acc[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KS; ++j) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const h8 w = *reinterpret_cast<const h8*>(Ws + (pp * 64 + t * 16 + r16) * LDW + 32 * j + kq);
          acc[t] = mfma16(w, a[j], acc[t]);
        }
        __builtin_amdgcn_sched_barrier(0);   // one k step's weight fragments live at a time
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int c = pp * 64 + t * 16 + 4 * g4;
        const float4 bb = *reinterpret_cast<const float4*>(&Bs[c]);
        const float bs[4] = {bb.x, bb.y, bb.z, bb.w};
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float y = acc[t][i] + bs[i];
          if (p.op == OP_RELU) y = fmaxf(y, 0.f);
          v[i] = y * inv;
        }
        if (p.resid) {
          float r[4];
          Raw4v<DACT>::unpack(rr[pp][t], r);
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] += r[i];
        }
        if (valid && c < p.N) st4<DACT>(p.dst.ptr, rowpart + c, v);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < KS; ++j) a[j] = an[j];
  }
}

// As many blocks as are resident at once (the tiles are dealt out by block id, so every
// launched block must be resident together).
template <int DACT, int KS, int NP>
static void launch_rowgemm_res(lf_context* ctx, const RowGemmParams& p) {
  constexpr int NWV = 8;   // 12 measured no faster in the N = 384 Evoformer block, 16 slower
  static const int per_cu = [] {
    int n = 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, rowgemm_res_kernel<DACT, KS, NP, NWV>, 64 * NWV, 0) !=
        hipSuccess)
      n = 1;
    return n < 1 ? 1 : n;
  }();
  const dim3 g((unsigned)std::min((p.rows + 16 * NWV - 1) / (16 * NWV), per_cu * ctx->num_cus));
  hipLaunchKernelGGL((rowgemm_res_kernel<DACT, KS, NP, NWV>), g, dim3(64 * NWV), 0, ctx->stream, p);
}

bool rowgemm_resident(const lf_context* ctx, int rows, int K, int N, const Dst& dst) {
  const int np = N / 64, ks = K / 32;
  return N % 64 == 0 && K % 32 == 0 && (np == 2 || np == 4) && (ks == 4 || ks == 8) && dst.D >= 64 * np &&
         (rows + 15) / 16 >= 8 * ctx->num_cus;
}

int launch_rowgemm(lf_context* ctx, const RowGemmParams& p, const char* label) {
  if (p.rows <= 0) return LF_OK;
  const std::string l(label);
  if (p.K % 8 != 0 || p.N % 4 != 0) return set_error(LF_ERR_INVALID, l + ": rowgemm needs K % 8 == 0 and N % 4 == 0");
  const Dst& d = p.dst;
  if (d.sD != 1 || d.D < p.N || d.sB % 4 != 0 || d.sN % 4 != 0)
    return set_error(LF_ERR_INVALID, l + ": rowgemm destination columns must be contiguous and 4-aligned");
  const long long span = (long long)((p.rows - 1) / d.Q) * d.sB + (long long)std::min(p.rows - 1, d.Q - 1) * d.sN + p.N;
  if (span >= (1LL << 31)) return set_error(LF_ERR_INVALID, l + ": destination above 2^31 elements");
  LaunchScope ls(ctx, label);
  // weight-resident form: the whole W in LDS, N and K whole multiples of the tiles
  const int np = p.N / 64, ks = p.K / 32;
  const bool resident = rowgemm_resident(ctx, p.rows, p.K, p.N, p.dst);
  if (p.wview && !resident) return set_error(LF_ERR_INVALID, l + ": stored weights need the weight-resident form");
  if (resident && (p.wview || p.w.kp >= p.K)) {
#define LF_RR(D, KS_, NP_) launch_rowgemm_res<D, KS_, NP_>(ctx, p)
#define LF_RRD(D)                                      \
  if (ks == 4 && np == 2) LF_RR(D, 4, 2);               \
  else if (ks == 4) LF_RR(D, 4, 4);                     \
  else if (np == 2) LF_RR(D, 8, 2);                     \
  else LF_RR(D, 8, 4);
    if (d.dtype == DT_F32) { LF_RRD(DT_F32) }
    else if (d.dtype == DT_F16) { LF_RRD(DT_F16) }
    else { LF_RRD(DT_BF16) }
#undef LF_RRD
#undef LF_RR
    return check_hip(hipGetLastError(), label);
  }
  const int nt = p.N <= 128 ? 4 : 8;
  dim3 grid((p.rows + 127) / 128, (p.N + 32 * nt - 1) / (32 * nt));
#define LF_RG(D, T) hipLaunchKernelGGL((rowgemm_kernel<D, T>), grid, dim3(512), 0, ctx->stream, p)
  if (d.dtype == DT_F32) { if (nt == 4) LF_RG(DT_F32, 4); else LF_RG(DT_F32, 8); }
  else if (d.dtype == DT_F16) { if (nt == 4) LF_RG(DT_F16, 4); else LF_RG(DT_F16, 8); }
  else { if (nt == 4) LF_RG(DT_BF16, 4); else LF_RG(DT_BF16, 8); }
#undef LF_RG
  return check_hip(hipGetLastError(), label);
}

}  // namespace lf
