// Outer product mean: z_ij += ((sum_s l_si (x) r_sj) W_out + b) / (norm_eps + sum_s m_si m_sj)
// with l = m * (LN(msa) Wl + bl), r likewise (AF2: webgpu/kernels/outer-product-mean.js:395-416,
// 595-610, 702-742; AF3: cpu/af3/trunk/msa.js:72-155, no projection biases, fast variance).
//
// Kernels:
//   lnproj    LN(msa) -> l, r stored [i][a][s] (sequence-contiguous: the contraction's K axis)
//   count     den[i*N + j] = norm_eps + sum_s m_si m_sj
//   outer     O[(i,j)][a*c + b] = sum_s l[i][a][s] r[j][b][s]: one NT GEMM of (N*c) x (N*c) x S on
//             MFMA, 256x256 tiles (128x128 when N*c is not a multiple of 256), written
//             pair-major f16 (the next GEMM's rows)
//   rowgemm   O W_out + b, / den, + pair residual
//   fused     (c_outer 32, c_z 128, whole 256 tiles) the outer tile kept in LDS and the output
//             GEMM, /den and residual run in the same kernel: O never reaches memory
#include <algorithm>
#include <cmath>

#include "lf_rowgemm.h"

namespace lf {

// The outer products: O[(i*N + j)][a*co + b] = sum_s L[i][a][s] R[j][b][s], i.e. the NT GEMM
// (N*co) x (N*co) x S of the rows m = i*co + a and n = j*co + b, stored pair-major f16.
struct OuterParams {
  const _Float16* L;   // [N*co][S]
  const _Float16* R;   // [N*co][S]
  _Float16* O;         // [N*N][co*co]
  int N, co, S;
};

constexpr int OT = 128, OT_BK = 64, OT_LD = OT_BK + 8;

struct OtRegs {
  h8 v[4];
};

// [128 rows][64 k] of a sequence-contiguous operand: global -> registers (issued a K step
// ahead) -> LDS.  Rows past M and k past S read as zero.
__device__ __forceinline__ void ot_fetch(OtRegs& r, const _Float16* src, int M, int S, int m0, int k0, int tid,
                                         bool vec) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int e = tid + it * 256, m = m0 + (e >> 3), k = k0 + (e & 7) * 8;
    if (vec) {
      r.v[it] = (m < M && k < S) ? *reinterpret_cast<const h8*>(src + (size_t)m * S + k) : h8{0, 0, 0, 0, 0, 0, 0, 0};
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) r.v[it][u] = (m < M && k + u < S) ? src[(size_t)m * S + k + u] : (_Float16)0.f;
    }
  }
}

__device__ __forceinline__ void ot_store(_Float16* Sm, const OtRegs& r, int tid) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int e = tid + it * 256;
    *reinterpret_cast<h8*>(Sm + (e >> 3) * OT_LD + (e & 7) * 8) = r.v[it];
  }
}

// One 128x128 tile per block (4 waves of 64x64).  The 1-D grid is remapped so that each XCD
// (block ids are dealt round-robin over 8) owns a contiguous band of row tiles; when the band
// is whole rows it is walked column by column, so the band's L tiles stay in the XCD's L2 and
// each R tile is read from memory once per XCD, not once per row tile.  R is the MFMA A operand, so a lane holds four
// consecutive b of one (i, a) row: 8-byte stores into the pair-major output.
// FULL: N*co a multiple of 128 and S of 64, so every fetch is a whole in-range 16-byte load
// from a per-thread base pointer.
template <bool FULL>
__global__ __launch_bounds__(256) void opm_outer_kernel(OuterParams p) {
  __shared__ __attribute__((aligned(16))) _Float16 As[2][OT * OT_LD];   // double-buffered K steps
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][OT * OT_LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = p.N * p.co, tm = (M + OT - 1) / OT;
  const int total = (int)gridDim.x, per = total >> 3;
  int lin = (int)blockIdx.x;
  int mt, nt;
  if (lin < per * 8) {
    const int x = lin & 7, q = lin >> 3;   // XCD x owns tiles [x*per, (x+1)*per) of row-major order
    if (per % tm == 0) {                   // whole row tiles: walk the band column-major
      const int rows = per / tm;
      mt = x * rows + q % rows;
      nt = q / rows;
    } else {
      const int t = x * per + q;
      mt = t / tm;
      nt = t % tm;
    }
  } else {
    mt = lin / tm;
    nt = lin % tm;
  }
  const int m0 = mt * OT, n0 = nt * OT;
  const bool vec = (p.S & 7) == 0;
  f4 acc[4][4];
  zero_acc(acc);
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  OtRegs ra, rb;
  // FULL: thread tid loads rows (tid >> 3) + 32*it of each tile, k pieces (tid & 7)*8 .. +8
  const _Float16* pa = p.L + (size_t)(m0 + (tid >> 3)) * p.S + (tid & 7) * 8;
  const _Float16* pb = p.R + (size_t)(n0 + (tid >> 3)) * p.S + (tid & 7) * 8;
  const size_t rstep = (size_t)32 * p.S;
  auto fetch = [&](int k0) __attribute__((always_inline)) {
    if constexpr (FULL) {
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        ra.v[it] = *reinterpret_cast<const h8*>(pa + it * rstep + k0);
        rb.v[it] = *reinterpret_cast<const h8*>(pb + it * rstep + k0);
      }
    } else {
      ot_fetch(ra, p.L, M, p.S, m0, k0, tid, vec);
      ot_fetch(rb, p.R, M, p.S, n0, k0, tid, vec);
    }
  };
  // one barrier per K step: the next step's tiles are fetched before this step's MFMAs and
  // written to the other buffer after them (every wave passed the barrier that ended that
  // buffer's last use)
  fetch(0);
  ot_store(As[0], ra, tid);
  ot_store(Bs[0], rb, tid);
  __syncthreads();
  for (int k0 = 0, kb = 0; k0 < p.S; k0 += OT_BK, kb ^= 1) {
    const bool more = k0 + OT_BK < p.S;
    if (more) fetch(k0 + OT_BK);
    const _Float16* Ak = As[kb];
    const _Float16* Bk = Bs[kb];
#pragma unroll
    for (int kk = 0; kk < OT_BK; kk += 32) {
      h8 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const h8*>(Ak + (wm * 64 + i * 16 + r16) * OT_LD + kk + kq);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const h8*>(Bk + (wn * 64 + j * 16 + r16) * OT_LD + kk + kq);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(b[j], a[i], acc[i][j]);
    }
    if (more) {
      ot_store(As[kb ^ 1], ra, tid);
      ot_store(Bs[kb ^ 1], rb, tid);
    }
    __syncthreads();
  }
  // acc[i][j][u]: row m = m0 + wm*64 + 16i + r16, columns n = n0 + wn*64 + 16j + 4g4 + u
  const unsigned co = (unsigned)p.co;
  const long long cc = (long long)p.co * p.co;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + wm * 64 + i * 16 + r16;
    if (m >= M) continue;
    const unsigned mi = (unsigned)m / co, ma = (unsigned)m - mi * co;
    const long long rowpart = (long long)mi * p.N * cc + (long long)ma * p.co;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + 4 * g4;
      if (n >= M) continue;
      const unsigned nj = (unsigned)n / co, nb = (unsigned)n - nj * co;
      h4 o;
#pragma unroll
      for (int u = 0; u < 4; ++u) o[u] = (_Float16)acc[i][j][u];
      *reinterpret_cast<h4*>(p.O + rowpart + (long long)nj * cc + nb) = o;
    }
  }
}

constexpr int OB = 256;
constexpr size_t OB_SMEM = (size_t)2 * 2 * OB * OT_LD * sizeof(_Float16);   // 147,456 bytes

// The XCD band order of the 256-tile grid: tile (mt, nt) of block blockIdx.x.
__device__ __forceinline__ void opm_big_order(const OuterParams& p, int& mt, int& nt) {
  const int M = p.N * p.co, tm = M / OB;
  const int total = (int)gridDim.x, per = total >> 3;
  const int lin = (int)blockIdx.x;
  if (lin < per * 8) {
    const int x = lin & 7, q = lin >> 3;
    if (per % tm == 0) {
      const int rows = per / tm;
      mt = x * rows + q % rows;
      nt = q / rows;
    } else {
      const int t = x * per + q;
      mt = t / tm;
      nt = t % tm;
    }
  } else {
    mt = lin / tm;
    nt = lin % tm;
  }
}

// The 256x256 tile at (m0, n0) accumulated into acc: lane holds rows m0 + wm*128 + 16i + r16,
// columns n0 + wn*64 + 16j + 4g4 + u (wm = wave / 4, wn = wave % 4).  Ends after a barrier,
// so the caller may reuse the LDS.
__device__ __forceinline__ void opm_big_tile(const OuterParams& p, int m0, int n0, f4 (&acc)[8][4], _Float16* obs) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  constexpr int STAGE = 2 * OB * OT_LD;
  // thread tid loads rows (tid >> 3) + 64*it of each tile, k pieces (tid & 7)*8 .. +8
  const _Float16* pa = p.L + (size_t)(m0 + (tid >> 3)) * p.S + (tid & 7) * 8;
  const _Float16* pb = p.R + (size_t)(n0 + (tid >> 3)) * p.S + (tid & 7) * 8;
  const size_t rstep = (size_t)64 * p.S;
  h8 ra[4], rb[4];
  auto fetch = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      ra[it] = *reinterpret_cast<const h8*>(pa + it * rstep + k0);
      rb[it] = *reinterpret_cast<const h8*>(pb + it * rstep + k0);
    }
  };
  auto put = [&](int buf) __attribute__((always_inline)) {
    _Float16* A = obs + buf * STAGE;
    _Float16* B = A + OB * OT_LD;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int r = (tid >> 3) + 64 * it, c = (tid & 7) * 8;
      *reinterpret_cast<h8*>(A + r * OT_LD + c) = ra[it];
      *reinterpret_cast<h8*>(B + r * OT_LD + c) = rb[it];
    }
  };
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  fetch(0);
  put(0);
  __syncthreads();
  for (int k0 = 0, kb = 0; k0 < p.S; k0 += OT_BK, kb ^= 1) {
    const bool more = k0 + OT_BK < p.S;
    if (more) fetch(k0 + OT_BK);
    const _Float16* A = obs + kb * STAGE;
    const _Float16* B = A + OB * OT_LD;
    // the A fragment of row tile i + 1 is read while row tile i's MFMAs run (the scheduling
    // barriers keep the compiler from sinking each read to its use, which exposed the LDS
    // latency once per 4 MFMAs)
#pragma unroll
    for (int kk = 0; kk < OT_BK; kk += 32) {
      h8 b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const h8*>(B + (wn * 64 + j * 16 + r16) * OT_LD + kk + kq);
      h8 acur = *reinterpret_cast<const h8*>(A + (wm * 128 + r16) * OT_LD + kk + kq);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const h8 anext = *reinterpret_cast<const h8*>(A + (wm * 128 + ((i + 1) & 7) * 16 + r16) * OT_LD + kk + kq);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(b[j], acur, acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
        acur = anext;
      }
    }
    if (more) put(kb ^ 1);
    __syncthreads();
  }
}

// The outer-product GEMM with 256x256 tiles for whole tiles (N*co a multiple of 256, S of
// 64): half the L2-to-CU operand traffic per flop of the 128x128 kernel, which the L2 latency
// at the bytes a CU keeps in flight otherwise bounds.  512 threads = 8 waves of 128x64
// (2 in m x 4 in n); K steps of 64 double-buffered in LDS (147 KB, one block per CU), the next
// step fetched into registers during the current one's MFMAs.  Same XCD band order as above.
__global__ __launch_bounds__(512) void opm_outer_big_kernel(OuterParams p) {
  extern __shared__ __attribute__((aligned(16))) _Float16 obs[];   // [2][A 256 x OT_LD | B 256 x OT_LD]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 2, wn = wave & 3, r16 = lane & 15, g4 = lane >> 4;
  int mt, nt;
  opm_big_order(p, mt, nt);
  const int m0 = mt * OB, n0 = nt * OB;
  f4 acc[8][4];
  opm_big_tile(p, m0, n0, acc, obs);
  const unsigned co = (unsigned)p.co;
  const long long cc = (long long)p.co * p.co;
  long long colpart[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned n = (unsigned)(n0 + wn * 64 + j * 16 + 4 * g4), nj = n / co, nb = n - nj * co;
    colpart[j] = (long long)nj * cc + nb;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const unsigned m = (unsigned)(m0 + wm * 128 + i * 16 + r16), mi = m / co, ma = m - mi * co;
    const long long rowpart = (long long)mi * p.N * cc + (long long)ma * p.co;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h4 o;
#pragma unroll
      for (int u = 0; u < 4; ++u) o[u] = (_Float16)acc[i][j][u];
      *reinterpret_cast<h4*>(p.O + rowpart + colpart[j]) = o;
    }
  }
}

// The whole OPM update for c_outer = 32, c_z = 128 in one kernel: the 256x256 outer-product
// tile above covers 8 x 8 residue pairs; instead of being stored, it goes to LDS as f16 rows
// [pair][a*32 + b] (132 KB, reusing the K-step buffers), and the block runs the output GEMM
// on it, D[c][pair] = sum_k W^T[c][k] O^T[k][pair], K = 1024: wave w owns all 64 pairs and
// the channels 16 w .. +16, its W^T fragments read straight from the expanded weights (256 KB,
// L2-resident, read once per block) a group of eight k steps ahead.  Epilogue as rowgemm's:
// (D + b) / den + residual, a lane storing 4 consecutive channels of one pair.  The 302 MB
// outer product at N = 384 never reaches memory.
constexpr int OF_LD = 1024 + 8;
struct OpmFusedParams {
  OuterParams o;
  const _Float16* W;    // expanded W_out: [c_z][1024], k contiguous
  int kp;
  const float* bias;    // [c_z] or null
  const float* den;     // [N*N]
  const void* resid;    // [N*N][c_z] or null
  void* out;
};

template <int ACT>
__global__ __launch_bounds__(512) void opm_fused_kernel(OpmFusedParams f) {
  extern __shared__ __attribute__((aligned(16))) _Float16 obs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 2, wn = wave & 3, r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  int mt, nt;
  opm_big_order(f.o, mt, nt);
  // the epilogue's normalisers and residual rows do not depend on the GEMMs: their loads are
  // issued first and land during the outer GEMM (lane: channels c .. c + 3 of pair 16 pt + r16)
  const int N = f.o.N;
  const int c = wave * 16 + 4 * g4;
  float inv[4], res[4][4];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
    const int pl = pt * 16 + r16;
    const size_t row = (size_t)(mt * 8 + (pl >> 3)) * N + nt * 8 + (pl & 7);
    inv[pt] = f.den[row];
    if (f.resid) ld4v<ACT>(f.resid, row * 128 + c, res[pt]);
    else res[pt][0] = res[pt][1] = res[pt][2] = res[pt][3] = 0.f;
  }
  {
    f4 acc[8][4];
    opm_big_tile(f.o, mt * OB, nt * OB, acc, obs);
    // tile row wm*128 + 16i + r16 = (residue, a), column wn*64 + 16j + 4g4 + u = (residue, b)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ml = wm * 128 + i * 16 + r16, ri = ml >> 5, a = ml & 31;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nl = wn * 64 + j * 16 + 4 * g4, rj = nl >> 5, b = nl & 31;
        *reinterpret_cast<h4*>(obs + (ri * 8 + rj) * OF_LD + a * 32 + b) =
            h4{(_Float16)acc[i][j][0], (_Float16)acc[i][j][1], (_Float16)acc[i][j][2], (_Float16)acc[i][j][3]};
      }
    }
  }
  __syncthreads();
  // wave w: all 64 pairs (4 tiles of 16) x channels 16 w .. +16, so each block reads W once
  const _Float16* wrow = f.W + (size_t)(wave * 16 + r16) * f.kp + kq;
  const _Float16* orow = obs + r16 * OF_LD + kq;
  f4 d[4];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) d[pt] = f4{0.f, 0.f, 0.f, 0.f};
  // W^T fragments in groups of 8 k steps, double-buffered: group g + 1's loads are issued
  // before group g's MFMAs, and scheduling barriers keep the compiler from sinking them
  // towards their use (which left two or three loads in flight)
  h8 wcur[8], wnext[8];
  auto wload = [&](int g, h8 (&w)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const h8*>(wrow + 256 * g + 32 * u);
  };
  wload(0, wcur);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    wload(g < 3 ? g + 1 : 3, wnext);   // the last group reloads itself: loads stay unconditional
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = 256 * g + 32 * u;
#pragma unroll
      for (int pt = 0; pt < 4; ++pt)
        d[pt] = mfma16(wcur[u], *reinterpret_cast<const h8*>(orow + pt * 16 * OF_LD + k), d[pt]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) wcur[u] = wnext[u];
  }
  // lane: channels c = 16 w + 4 g4 + i of pair 16 pt + r16 of the tile
  float bias[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bias[i] = f.bias ? f.bias[c + i] : 0.f;
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
    const int pl = pt * 16 + r16;
    const size_t row = (size_t)(mt * 8 + (pl >> 3)) * N + nt * 8 + (pl & 7);
    const float rinv = 1.f / inv[pt];
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (d[pt][i] + bias[i]) * rinv + res[pt][i];
    st4v<ACT>(f.out, row * 128 + c, v);
  }
}

// den[i*N + j] = eps + sum_s m[s][i] m[s][j]: a 16x16 tile per block, one output per thread
// (N = 384 gives 576 blocks), the mask columns staged through LDS 64 sequences at a time
// (reads of a staged row are broadcasts or conflict-free); sums run in sequence order.
constexpr int CT_S = 64;

__global__ __launch_bounds__(256) void opm_count_kernel(const float* mask, float* den, int S, int N, float eps) {
  __shared__ float Mi[CT_S][16], Mj[CT_S][16];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int i0 = blockIdx.y * 16, j0 = blockIdx.x * 16;
  float acc = 0.f;
  for (int s0 = 0; s0 < S; s0 += CT_S) {
    for (int e = tid; e < CT_S * 16; e += 256) {
      const int ss = e >> 4, c = e & 15, sg = s0 + ss;
      Mi[ss][c] = (sg < S && i0 + c < N) ? mask[(size_t)sg * N + i0 + c] : 0.f;
      Mj[ss][c] = (sg < S && j0 + c < N) ? mask[(size_t)sg * N + j0 + c] : 0.f;
    }
    __syncthreads();
#pragma unroll 16
    for (int ss = 0; ss < CT_S; ++ss) acc = fmaf(Mi[ss][ty], Mj[ss][tx], acc);
    __syncthreads();
  }
  const int i = i0 + ty, j = j0 + tx;
  if (i < N && j < N) den[(size_t)i * N + j] = eps + acc;
}

// The big kernels' dynamic LDS (above the 64 KB default) is opted into once per process.
static bool big_smem_ok(lf_context*) {
  auto opt = [](const void* k) {
    return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)OB_SMEM) == hipSuccess;
  };
  static const bool ok = opt(reinterpret_cast<const void*>(opm_outer_big_kernel)) &&
                         opt(reinterpret_cast<const void*>(opm_fused_kernel<DT_F32>)) &&
                         opt(reinterpret_cast<const void*>(opm_fused_kernel<DT_F16>)) &&
                         opt(reinterpret_cast<const void*>(opm_fused_kernel<DT_BF16>));
  return ok;
}

int outer_product_mean(lf_context* ctx, const lf_opm_args& a) {
  LF_REQUIRE(a.w != nullptr, "outer product mean: weights are NULL");
  LF_REQUIRE(a.sequences > 0 && a.length > 0 && a.c_m > 0 && a.c_outer > 0 && a.c_z > 0,
             "outer product mean dimensions must be positive safe integers");
  LF_REQUIRE(a.c_m <= 384, "outer product mean: c_m must be <= 384");
  LF_REQUIRE(a.c_outer <= 64 && a.c_outer % 4 == 0, "outer product mean: c_outer must be a multiple of 4, <= 64");
  LF_REQUIRE(act_dtype_ok(a.msa_dtype) && act_dtype_ok(a.pair_dtype), "outer product mean: bad activation dtype");
  LF_REQUIRE(a.msa && a.mask && a.out, "outer product mean: msa, mask and out must be device pointers");
  LF_REQUIRE(!a.accumulate || a.pair_in, "outer product mean: accumulate needs pair_in");
  LF_REQUIRE(a.epsilon > 0.f && a.norm_epsilon > 0.f, "outer product mean: epsilons must be positive");
  const lf_opm_weights& w = *a.w;
  const int S = a.sequences, N = a.length, co = a.c_outer, cz = a.c_z;
  const long long pairs = (long long)N * N, rows = (long long)S * N;
  WView views[3];
  LF_TRY(make_view(w.wl, a.c_m, co, "leftWeight", &views[0]));
  LF_TRY(make_view(w.wr, a.c_m, co, "rightWeight", &views[1]));
  LF_TRY(make_view(w.wo, co * co, cz, "outputWeight", &views[2]));
  // l, r = mask * (LN(msa) W + b), stored [i][a][s]
  LnProjParams pp{};
  pp.x = a.msa;
  pp.rows = (int)rows;
  pp.C = a.c_m;
  // logical row r = i*S + s reads MSA row s*N + i, so a wave's rows are consecutive sequences
  // of one residue: 16 lanes write 32 contiguous bytes of the sequence-contiguous l and r
  pp.rmQ = S;
  pp.rmB = N;
  pp.ln_s = w.norm_scale;
  pp.ln_o = w.norm_offset;
  pp.eps = a.epsilon;
  pp.fast_var = a.fast_variance;
  pp.rowmask = a.mask;
  pp.g[0] = Group{views[0], WView{}, co, OP_ROWMASK, 1.f, w.bl, nullptr, Dst{}};
  pp.g[1] = Group{views[1], WView{}, co, OP_ROWMASK, 1.f, w.br, nullptr, Dst{}};
  pp.ngroups = 2;

  const size_t lr = (size_t)N * co * S * sizeof(_Float16);
  // c_outer 32, c_z 128, whole 256 tiles: the output GEMM runs inside the outer-product kernel
  const bool fused = co == 32 && cz == 128 && (N * co) % OB == 0 && S % OT_BK == 0 && big_smem_ok(ctx);
  const size_t ob = fused ? 0 : (size_t)pairs * co * co * sizeof(_Float16);
  size_t sizes[6] = {lr, lr, ob, (size_t)pairs * sizeof(float), expanded_bytes(views[2]), lnproj_packed_bytes(pp)};
  void* bufs[6];
  LF_TRY(workspace(ctx, sizes, bufs, 6));
  _Float16 *L = (_Float16*)bufs[0], *R = (_Float16*)bufs[1], *O = (_Float16*)bufs[2];
  float* den = (float*)bufs[3];
  // the output projection and the l / r projections decoded in one launch
  ExpandList xl;
  WExp wo;
  LF_TRY(expand_add_plain(ctx, xl, views[2], bufs[4], &wo, 1.f, "opm.expand"));
  // logical row r = i*S + s, column a -> (i*co + a)*S + s
  pp.g[0].dst = Dst{L, DT_F16, S, (long long)co * S, 1, co, 0, S};
  pp.g[1].dst = Dst{R, DT_F16, S, (long long)co * S, 1, co, 0, S};
  LF_TRY(lnproj_prepare(ctx, pp, bufs[5], &xl, "opm.project"));
  LF_TRY(expand_flush(ctx, xl, "opm.expand"));
  LF_TRY(lnproj_run(ctx, pp, a.msa_dtype, "opm.project"));
  {  // the pair normalisers (inside a stack call, computed by the first block and reused)
    void* cached;
    bool filled;
    LF_TRY(mask_table(ctx, a.mask, 10, S, N, a.norm_epsilon, sizes[3], &cached, &filled));
    if (cached) den = static_cast<float*>(cached);
    if (!filled) {
      {
        LaunchScope ls(ctx, "opm.count");
        hipLaunchKernelGGL(opm_count_kernel, dim3((N + 15) / 16, (N + 15) / 16), dim3(256), 0, ctx->stream, a.mask,
                           den, S, N, a.norm_epsilon);
      }
      LF_TRY(check_hip(hipGetLastError(), "opm count launch"));
    }
  }
  if (fused) {
    OpmFusedParams f{OuterParams{L, R, nullptr, N, co, S}, wo.p, wo.kp, w.bo, den,
                     a.accumulate ? a.pair_in : nullptr, a.out};
    const int tb = N * co / OB;
    LaunchScope ls(ctx, "opm.fused");
    if (a.pair_dtype == LF_F32)
      hipLaunchKernelGGL(opm_fused_kernel<DT_F32>, dim3((unsigned)(tb * tb)), dim3(512), OB_SMEM, ctx->stream, f);
    else if (a.pair_dtype == LF_F16)
      hipLaunchKernelGGL(opm_fused_kernel<DT_F16>, dim3((unsigned)(tb * tb)), dim3(512), OB_SMEM, ctx->stream, f);
    else
      hipLaunchKernelGGL(opm_fused_kernel<DT_BF16>, dim3((unsigned)(tb * tb)), dim3(512), OB_SMEM, ctx->stream, f);
    return check_hip(hipGetLastError(), "opm fused launch");
  }
  {  // O[(i, j)][a*co + b] = sum_s l[i][a][s] r[j][b][s]
    OuterParams op{L, R, O, N, co, S};
    const int tm = (N * co + OT - 1) / OT;
    LaunchScope ls(ctx, "opm.outer");
    const bool full = (N * co) % OT == 0 && S % OT_BK == 0;
    const int tb = N * co / OB;
    if ((N * co) % OB == 0 && S % OT_BK == 0 && big_smem_ok(ctx)) {
      hipLaunchKernelGGL(opm_outer_big_kernel, dim3((unsigned)(tb * tb)), dim3(512), OB_SMEM, ctx->stream, op);
    } else if (full)
      hipLaunchKernelGGL(opm_outer_kernel<true>, dim3((unsigned)(tm * tm)), dim3(256), 0, ctx->stream, op);
    else
      hipLaunchKernelGGL(opm_outer_kernel<false>, dim3((unsigned)(tm * tm)), dim3(256), 0, ctx->stream, op);
  }
  LF_TRY(check_hip(hipGetLastError(), "opm outer launch"));
  {  // (O W_out + b) / den + residual
    RowGemmParams rp{};
    rp.A = O;
    rp.rows = (int)pairs;
    rp.K = co * co;
    rp.N = cz;
    rp.w = wo;
    rp.bias = w.bo;
    rp.op = OP_STORE;
    rp.rowden = den;
    rp.resid = a.accumulate ? a.pair_in : nullptr;
    rp.dst = dst_rowmajor(a.out, a.pair_dtype, (int)pairs, cz);
    LF_TRY(launch_rowgemm(ctx, rp, "opm.output"));
  }
  return LF_OK;
}

}  // namespace lf
