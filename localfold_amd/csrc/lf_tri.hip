// Triangle multiplicative update (AF2 and AF3 dialects), three kernels per direction:
//
//  project  LN(z) -> a, b = mask * (LN(z) Wp + bp) * sigmoid(LN(z) Wg + bg), stored
//           channel-major [cH][N*N] f16 (the layout the contraction reads).
//  contract X[h] = s * A[h] B[h]^T per channel h, 128x128 output tiles on MFMA; outgoing
//           reads a, b row-major, incoming reads them k-major (x_ij = sum_k a_kj b_ki).
//           X is stored channel-major f16, pre-scaled by s = 2^-ceil(log2(N)/2) so a
//           length-long sum stays inside f16's range.
//  output   LN_out(X) Wz + bz, gated by sigmoid(LN_in(z) Wg + bg), + z residual.  LN_in(z)
//           is recomputed from z rather than stored (one read of z instead of a write and
//           a read of the gate tensor).
//
// For c_z, c_hidden <= 128 (every AF2/AF3 pair width) project and output run as
// weight-resident persistent kernels: a block stages all of the op's f16 weights in LDS
// once and each wave streams 16-row tiles with no block barrier, prefetching the next
// tile's rows during the current tile's MFMA passes.  Wider channels use the chunked
// kernels, which re-stage 32/64-column weight chunks per 64-row block.
//
// The activation dtype is a template parameter so every load is straight-line code.
//
// Semantics: webgpu/kernels/triangle/cpu-reference.js:55-99 (AF2 outgoing),
// cpu/af3/trunk/pairformer.js:213-300 (AF3, both directions, interleaved split).
#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <type_traits>

#include "lf_gemm.h"
#include "lf_ops.h"

namespace lf {

// A weight operand of the triangle kernels: the stored view, decoded inside the kernels as
// they stage it into LDS, the factor applied to the decoded values before the f16 rounding,
// and kp = K rounded up to 32 (the k extent staged).
struct WSrc {
  WView v;
  float mul;
  int kp;
};

inline WSrc wsrc(const WView& v, float mul = 1.f) { return WSrc{v, mul, (v.K + 31) & ~31}; }

__device__ __forceinline__ void stage_src(_Float16* Ws, int ldw, const WSrc& s, int ncols, int n_base, int tid,
                                          int nthreads) {
  stage_view(Ws, ldw, s.v, ncols, n_base, s.kp, s.mul, tid, nthreads);
}

struct TriProjectParams {
  const void* z;
  const float* mask;
  const float *ln_s, *ln_o;
  float eps;
  int fast_var;
  int P, C, H;         // pairs, cZ, cHidden
  WSrc wp[2], wg[2];   // [0] -> a, [1] -> b
  const float *bp[2], *bg[2];
  _Float16* out[2];    // a, b: [H][P]
  int N;               // length (P = N * N)
  int kmajor_out;      // store each channel plane transposed: a[h][j][k] for pair (k, j)
  int split;           // AF3 in the resident kernels: wp[0] / wg[0] are the whole interleaved
                       // tensors (even stored columns -> a, odd -> b); wp[1] / wg[1] unused
  float2* stats;       // when not NULL (128-wide kernel only): LN_in (mean, 1/std) per pair, by z row
};

struct TriOutputParams {
  const _Float16* X;   // [H][P]
  const void* z;
  void* out;
  int accumulate;
  const float *ln_in_s, *ln_in_o, *ln_out_s, *ln_out_o;
  float eps, eps_x;    // eps_x: centre-norm epsilon on the stored (scaled) X
  int fast_var;
  int P, C, H;
  WSrc wz, wg;
  const float *bz, *bg;
  const float2* stats;  // when not NULL: LN_in (mean, 1/std) per pair, written by the project kernel
};

// ---------------------------------------------------------------------------------------
// Chunked kernels (any c_z, c_hidden <= 256)
// ---------------------------------------------------------------------------------------

constexpr int PJ_ROWS = 64;     // pairs per block (4 waves x 16)
constexpr int PJ_COLS = 32;     // hidden channels per chunk (32 projection + 32 gate columns)

template <int ACT, int KPAD>
__global__ __launch_bounds__(256) void tri_project_kernel(TriProjectParams p) {
  constexpr int LDA = KPAD + 8, LDW = KPAD + 8, LDO = PJ_ROWS + 8;
  __shared__ __attribute__((aligned(16))) _Float16 As[PJ_ROWS * LDA];
  __shared__ __attribute__((aligned(16))) _Float16 Ws[2 * PJ_COLS * LDW];
  __shared__ __attribute__((aligned(16))) _Float16 Os[PJ_COLS * LDO];
  __shared__ __attribute__((aligned(16))) float Gs[2 * KPAD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int p0 = blockIdx.x * PJ_ROWS;
  const int kloop = (p.C + 31) & ~31;
  stage_vec(Gs, p.ln_s, p.C, 1.f, KPAD, tid, 256);
  stage_vec(Gs + KPAD, p.ln_o, p.C, 0.f, KPAD, tid, 256);
  __syncthreads();
  {
    const int row0 = p0 + wave * 16;
    RowTile<ACT, KPAD> t;
    tile_load(t, p.z, (size_t)row0, min(16, p.P - row0), p.C, lane);
    tile_ln_store(t, As + wave * 16 * LDA, LDA, min(16, p.P - row0), p.C, Gs, Gs + KPAD, p.eps, p.fast_var, lane);
  }
  const int hchunks = (p.H + PJ_COLS - 1) / PJ_COLS;
  for (int chunk = 0; chunk < 2 * hchunks; ++chunk) {
    const int which = chunk / hchunks, h0 = (chunk % hchunks) * PJ_COLS;
    const WSrc& wpe = which ? p.wp[1] : p.wp[0];
    const WSrc& wge = which ? p.wg[1] : p.wg[0];
    __syncthreads();  // As ready / previous chunk done with Ws, Os
    stage_src(Ws, LDW, wpe, PJ_COLS, h0, tid, 256);
    stage_src(Ws + PJ_COLS * LDW, LDW, wge, PJ_COLS, h0, tid, 256);
    __syncthreads();
    f4 acc[1][4];
    zero_acc(acc);
    wave_tile_mfma<1, 4>(acc, As, LDA, wave * 16, Ws, LDW, kloop, lane);
    const float* bpv = which ? p.bp[1] : p.bp[0];
    const float* bgv = which ? p.bg[1] : p.bg[0];
    // tiles 0,1: projection columns h0 + 16t + lane%16; tiles 2,3: the gate of the same channel
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int hl = t * 16 + (lane & 15), h = h0 + hl, hc = h < p.H ? h : 0;
      const float bpp = bpv ? bpv[hc] : 0.f;
      const float bgg = bgv ? bgv[hc] : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wave * 16 + (lane >> 4) * 4 + i, pair = p0 + row;
        const float m = p.mask[pair < p.P ? pair : 0];
        const float v = (acc[0][t][i] + bpp) * (m * sigmoidf_(acc[0][t + 2][i] + bgg));
        Os[hl * LDO + row] = (_Float16)(pair < p.P ? v : 0.f);
      }
    }
    __syncthreads();
    _Float16* dst = which ? p.out[1] : p.out[0];
    if (p0 + PJ_ROWS <= p.P && (p.P & 7) == 0) {
      const int hl = tid >> 3, seg = tid & 7;
      if (h0 + hl < p.H)
        *reinterpret_cast<h8*>(dst + (size_t)(h0 + hl) * p.P + p0 + seg * 8) =
            *reinterpret_cast<const h8*>(Os + hl * LDO + seg * 8);
    } else {
      for (int e = tid; e < PJ_COLS * PJ_ROWS; e += 256) {
        const int hl = e / PJ_ROWS, row = e % PJ_ROWS;
        if (h0 + hl < p.H && p0 + row < p.P) dst[(size_t)(h0 + hl) * p.P + p0 + row] = Os[hl * LDO + row];
      }
    }
  }
}

constexpr int OT_ROWS = 64, OT_COLS = 64;

template <int ACT, int KZ, int KH>
__global__ __launch_bounds__(256) void tri_output_kernel(TriOutputParams p) {
  typedef typename Act<ACT>::T T;
  constexpr int LDX = KH + 8, LDZ = KZ + 8;
  __shared__ __attribute__((aligned(16))) _Float16 Xs[OT_ROWS * LDX];
  __shared__ __attribute__((aligned(16))) _Float16 Zs[OT_ROWS * LDZ];
  __shared__ __attribute__((aligned(16))) _Float16 Wzs[OT_COLS * LDX];
  __shared__ __attribute__((aligned(16))) _Float16 Wgs[OT_COLS * LDZ];
  __shared__ __attribute__((aligned(16))) float Gs[2 * KZ + 2 * KH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int p0 = blockIdx.x * OT_ROWS;
  const int kh = (p.H + 31) & ~31, kz = (p.C + 31) & ~31;

  // X tile, transposed into Xs[pair][h]
  for (int e = tid; e < KH * OT_ROWS; e += 256) {
    const int h = e / OT_ROWS, r = e % OT_ROWS;
    const size_t src = (size_t)(h < p.H ? h : 0) * p.P + (p0 + r < p.P ? p0 + r : 0);
    const _Float16 v = p.X[src];
    Xs[r * LDX + h] = (h < p.H && p0 + r < p.P) ? v : (_Float16)0.f;
  }
  stage_vec(Gs, p.ln_in_s, p.C, 1.f, KZ, tid, 256);
  stage_vec(Gs + KZ, p.ln_in_o, p.C, 0.f, KZ, tid, 256);
  stage_vec(Gs + 2 * KZ, p.ln_out_s, p.H, 1.f, KH, tid, 256);
  stage_vec(Gs + 2 * KZ + KH, p.ln_out_o, p.H, 0.f, KH, tid, 256);
  __syncthreads();
  // centre LN over h (in place, scaled-X epsilon) and LN_in of z rows
  {
    const int row0 = p0 + wave * 16, nvalid = min(16, p.P - row0);
    lds_ln_inplace<KH>(Xs + wave * 16 * LDX, LDX, nvalid, p.H, Gs + 2 * KZ, Gs + 2 * KZ + KH, p.eps_x, p.fast_var,
                       lane);
    RowTile<ACT, KZ> t;
    tile_load(t, p.z, (size_t)row0, nvalid, p.C, lane);
    tile_ln_store(t, Zs + wave * 16 * LDZ, LDZ, nvalid, p.C, Gs, Gs + KZ, p.eps, p.fast_var, lane);
  }
  const T* zin = static_cast<const T*>(p.z);
  T* out = static_cast<T*>(p.out);
  for (int c0 = 0; c0 < p.C; c0 += OT_COLS) {
    __syncthreads();
    stage_src(Wzs, LDX, p.wz, OT_COLS, c0, tid, 256);
    stage_src(Wgs, LDZ, p.wg, OT_COLS, c0, tid, 256);
    __syncthreads();
    f4 az[1][4], ag[1][4];
    zero_acc(az);
    zero_acc(ag);
    wave_tile_mfma<1, 4>(az, Xs, LDX, wave * 16, Wzs, LDX, kh, lane);
    wave_tile_mfma<1, 4>(ag, Zs, LDZ, wave * 16, Wgs, LDZ, kz, lane);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int c = c0 + t * 16 + (lane & 15);
      if (c >= p.C) continue;
      const float bz = p.bz ? p.bz[c] : 0.f, bg = p.bg ? p.bg[c] : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pair = p0 + wave * 16 + (lane >> 4) * 4 + i;
        if (pair >= p.P) continue;
        const size_t idx = (size_t)pair * p.C + c;
        float v = (az[0][t][i] + bz) * sigmoidf_(ag[0][t][i] + bg);
        if (p.accumulate) v += Act<ACT>::ld(zin + idx);
        Act<ACT>::st(out + idx, v);
      }
    }
  }
}

struct TriContractParams {
  const _Float16* L;  // [H][N][N]
  const _Float16* R;
  _Float16* X;        // [H][N][N]
  int N;
  float scale;
};

template <int TM, int BK, bool KMAJOR>
__device__ __forceinline__ void ct_load(_Float16* S, const _Float16* src, int N, int m0, int k0, int tid) {
  constexpr int LD = BK + 8;
  for (int e = tid; e < TM * BK; e += 256) {
    int m, k;
    if (!KMAJOR) {
      m = e / BK;
      k = e % BK;
    } else {
      k = e / TM;
      m = e % TM;
    }
    const int gm = m0 + m, gk = k0 + k;
    S[m * LD + k] = (gm < N && gk < N) ? src[KMAJOR ? (size_t)gk * N + gm : (size_t)gm * N + gk] : (_Float16)0.f;
  }
}

// Vector form (N % 8 == 0) split in two: global -> registers (issued before the current K
// step's MFMAs so the loads are in flight during them) and registers -> LDS.  PER = TM / 32
// 16-byte pieces per thread and operand.
// The piece it of a thread: its (m, k) origin in the [TM x 64] slice at (m0, k0).
template <int TM, int BK, bool KMAJOR>
__device__ __forceinline__ void ct_piece(int it, int tid, int m0, int k0, int& gm, int& gk) {
  if (!KMAJOR) {
    const int e = tid + it * 256;
    gm = m0 + e / (BK / 8);
    gk = k0 + (e % (BK / 8)) * 8;
  } else {
    const int e = tid + it * 256;
    gk = k0 + e % BK;
    gm = m0 + (e / BK) * 8;
  }
}

// Branch-free: a clamped address always loads and an out-of-range piece is zeroed when it is
// written to LDS (ct_store), not here: a select on the loaded value at this point would make
// the compiler wait for the loads before the MFMAs they are meant to overlap, and a branch
// per load lets it serialise them with vmcnt(0) waits.
template <int TM, int BK, bool KMAJOR>
__device__ __forceinline__ void ct_fetch(h8 (&r)[TM * BK / 2048], const _Float16* src, int N, int m0, int k0, int tid) {
#pragma unroll
  for (int it = 0; it < TM * BK / 2048; ++it) {
    int gm, gk;
    ct_piece<TM, BK, KMAJOR>(it, tid, m0, k0, gm, gk);
    const bool ok = gm < N && gk < N;
    const int cm = ok ? gm : 0, ck = ok ? gk : 0;
    r[it] = *reinterpret_cast<const h8*>(src + (KMAJOR ? (size_t)ck * N + cm : (size_t)cm * N + ck));
  }
}

template <int TM, int BK, bool KMAJOR>
__device__ __forceinline__ void ct_store(_Float16* S, const h8 (&r)[TM * BK / 2048], int N, int m0, int k0, int tid) {
  constexpr int LD = BK + 8;
#pragma unroll
  for (int it = 0; it < TM * BK / 2048; ++it) {
    int gm, gk;
    ct_piece<TM, BK, KMAJOR>(it, tid, m0, k0, gm, gk);
    const h8 v = (gm < N && gk < N) ? r[it] : h8{0, 0, 0, 0, 0, 0, 0, 0};
    if (!KMAJOR) {
      *reinterpret_cast<h8*>(S + (gm - m0) * LD + (gk - k0)) = v;
    } else {
      // lane -> k, so the eight 2-byte LDS stores of a wave hit consecutive k
#pragma unroll
      for (int j = 0; j < 8; ++j) S[(gm - m0 + j) * LD + (gk - k0)] = v[j];
    }
  }
}

// One TM x TM tile of X[h] per block of 4 waves (2 x 2, a (TM/2)-square each), K in steps
// of BK through one LDS stage, the next step's loads in registers during the current step's
// MFMAs.  MINW waves per SIMD bound the registers (three: 12 waves a CU).  Measured at
// N = 384 (128 channels): 128-wide tiles with 64-wide K steps beat 192-wide tiles (fewer,
// longer blocks hide less latency), 32-wide K steps and 8-wave blocks.  The 1-D grid is
// remapped so that consecutive logical blocks (the tiles of one channel, which share their
// A rows and B rows) run on the same XCD: the hardware deals block ids round-robin over the
// 8 XCDs, each with its own L2.
template <int TM, int BK, int MINW, bool KMAJOR, bool VEC>
__global__ __launch_bounds__(256, MINW) void tri_contract_kernel(TriContractParams p) {
  constexpr int FM = TM / 32, WT = TM / 2, CT_LD = BK + 8, PER = TM * BK / 2048;
  __shared__ __attribute__((aligned(16))) _Float16 Ls[TM * CT_LD];
  __shared__ __attribute__((aligned(16))) _Float16 Rs[TM * CT_LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = (p.N + TM - 1) / TM, tiles = tm * tm;
  const int total = (int)gridDim.x, per = total >> 3;
  int lin = (int)blockIdx.x;
  if (lin < per * 8) lin = (lin & 7) * per + (lin >> 3);
  const int h = lin / tiles, t = lin - h * tiles;
  const int m0 = (t / tm) * TM, n0 = (t % tm) * TM;
  const size_t plane = (size_t)p.N * p.N;
  const _Float16* L = p.L + h * plane;
  const _Float16* R = p.R + h * plane;
  f4 acc[FM][FM];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  h8 rl[PER], rr[PER];
  if (VEC) {
    ct_fetch<TM, BK, KMAJOR>(rl, L, p.N, m0, 0, tid);
    ct_fetch<TM, BK, KMAJOR>(rr, R, p.N, n0, 0, tid);
  }
  for (int k0 = 0; k0 < p.N; k0 += BK) {
    __syncthreads();
    if (VEC) {
      ct_store<TM, BK, KMAJOR>(Ls, rl, p.N, m0, k0, tid);
      ct_store<TM, BK, KMAJOR>(Rs, rr, p.N, n0, k0, tid);
    } else {
      ct_load<TM, BK, KMAJOR>(Ls, L, p.N, m0, k0, tid);
      ct_load<TM, BK, KMAJOR>(Rs, R, p.N, n0, k0, tid);
    }
    __syncthreads();
    if (VEC && k0 + BK < p.N) {
      ct_fetch<TM, BK, KMAJOR>(rl, L, p.N, m0, k0 + BK, tid);
      ct_fetch<TM, BK, KMAJOR>(rr, R, p.N, n0, k0 + BK, tid);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      h8 a[FM], b[FM];
#pragma unroll
      for (int i = 0; i < FM; ++i) a[i] = *reinterpret_cast<const h8*>(Ls + (wm * WT + i * 16 + r16) * CT_LD + kk + kq);
#pragma unroll
      for (int j = 0; j < FM; ++j) b[j] = *reinterpret_cast<const h8*>(Rs + (wn * WT + j * 16 + r16) * CT_LD + kk + kq);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(b[j], a[i], acc[i][j]);
    }
  }
  // acc[i][j][r] = X[m0 + wm*WT + 16i + r16][n0 + wn*WT + 16j + 4*g4 + r]: four consecutive
  // columns of one row per lane, stored as one 8-byte piece (16 rows x 32 bytes a store)
  _Float16* X = p.X + h * plane;
  const int g4 = lane >> 4;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int gm = m0 + wm * WT + i * 16 + r16;
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int gn = n0 + wn * WT + j * 16 + 4 * g4;
      h4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = (_Float16)(acc[i][j][r] * p.scale);
      if (VEC) {
        if (gm < p.N && gn < p.N) *reinterpret_cast<h4*>(X + (size_t)gm * p.N + gn) = o;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (gm < p.N && gn + r < p.N) X[(size_t)gm * p.N + gn + r] = o[r];
      }
    }
  }
}

// The outgoing-layout contraction (k contiguous in both operands) when N is a multiple of BK:
// TM x TM tiles (TM = 128 or 96), K steps of BK double-buffered in LDS and filled by direct global -> LDS
// loads (16 bytes a lane, no register staging), one barrier a step, the next step's loads in
// flight during the current step's MFMAs.  A wave's load instruction fills 1 KB of LDS
// contiguously, so the 16-byte chunks of a row are XOR-swizzled by the row (chunk c of row r
// sits in slot c ^ swz(r)) to keep the MFMA fragment reads of 16 rows off a single bank group.
// Rows past N are clamped to row N - 1: they only feed output rows or columns that are never
// stored.
// At TM = 128 the two 32 KB stages hold the LDS at two blocks (8 waves) per CU, at TM = 96
// (24 KB stages) three.  Measured at N = 384 the 128-row kernel beats the register-staged
// kernel above (30.9 against 33.1 us), and 8-wave blocks or 32-wide K steps with four blocks
// per CU were no faster.
template <int BK>
__device__ __forceinline__ int ct_swz(int r) {
  return BK == 64 ? (r & 7) : ((r >> 1) & 3);
}

template <int BK, int TM>
__global__ __launch_bounds__(256, TM == 128 ? 2 : 3) void tri_contract_dma_kernel(TriContractParams p) {
  constexpr int NT = 256, FM = TM / 32, FN = TM / 32, WT = TM / 2, WTN = TM / 2, CH = BK / 8,
                PER = TM * CH / NT, STAGE = TM * BK;
  static_assert(TM % 32 == 0 && (TM * CH) % NT == 0, "tile rows must split into whole load rounds");
  __shared__ __attribute__((aligned(16))) _Float16 S[2][2][STAGE];   // [stage][L, R][row][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = (p.N + TM - 1) / TM, tiles = tm * tm;
  const int total = (int)gridDim.x, per = total >> 3;
  int lin = (int)blockIdx.x;
  if (lin < per * 8) lin = (lin & 7) * per + (lin >> 3);
  const int h = lin / tiles, t = lin - h * tiles;
  const int m0 = (t / tm) * TM, n0 = (t % tm) * TM;
  const size_t plane = (size_t)p.N * p.N;
  const _Float16* L = p.L + h * plane;
  const _Float16* R = p.R + h * plane;
  // this thread's pieces: LDS slot q = it * 256 + tid holds row q / CH, chunk (q % CH) ^ swz
  const _Float16* gl[PER];
  const _Float16* gr[PER];
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int q = it * NT + tid, r = q / CH, c = (q % CH) ^ ct_swz<BK>(r);
    gl[it] = L + (size_t)min(m0 + r, p.N - 1) * p.N + c * 8;
    gr[it] = R + (size_t)min(n0 + r, p.N - 1) * p.N + c * 8;
  }
  auto issue = [&](int k0, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int base = (it * NT + wave * 64) * 8;
#if __HIP_DEVICE_COMPILE__   // a target builtin: the host pass, which only emits the launch stub, lacks it
      __builtin_amdgcn_global_load_lds(gl[it] + k0, &S[st][0][base], 16, 0, 0);
      __builtin_amdgcn_global_load_lds(gr[it] + k0, &S[st][1][base], 16, 0, 0);
#endif
    }
  };
  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, g4 = lane >> 4;
  issue(0, 0);
  const int nk = p.N / BK;
  for (int ks = 0; ks < nk; ++ks) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();   // step ks in LDS for every wave; every wave done with the other stage
    if (ks + 1 < nk) issue((ks + 1) * BK, (ks + 1) & 1);
    const _Float16* Ls = S[ks & 1][0];
    const _Float16* Rs = S[ks & 1][1];
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      h8 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * WT + i * 16 + r16;
        a[i] = *reinterpret_cast<const h8*>(Ls + row * BK + ((kk * 4 + g4) ^ ct_swz<BK>(row)) * 8);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn * WTN + j * 16 + r16;
        b[j] = *reinterpret_cast<const h8*>(Rs + row * BK + ((kk * 4 + g4) ^ ct_swz<BK>(row)) * 8);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(b[j], a[i], acc[i][j]);
    }
  }
  _Float16* X = p.X + h * plane;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int gm = m0 + wm * WT + i * 16 + r16;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int gn = n0 + wn * WTN + j * 16 + 4 * g4;
      h4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = (_Float16)(acc[i][j][r] * p.scale);
      if (gm < p.N && gn < p.N) *reinterpret_cast<h4*>(X + (size_t)gm * p.N + gn) = o;
    }
  }
}

// Large N (a multiple of 64, at least 768, when whole 256-row tiles add at most 10% to the
// work of 128-row ones; rows past N clamped as above): 256 x 256 tiles, 8 waves in a 2 x 4 grid, each
// wave 128 x 64 (32 accumulator tiles), the same direct-to-LDS double buffering as above in
// two 64 KB stages (one block per CU).  A wave's K step reads 384 bytes of LDS per MFMA
// instead of the 64 x 64 tile's 512.  Measured at N = 1024 (same box,
// alternating runs): 0.373 -> 0.306 ms per contraction.  Four 32-wide stages in the same LDS
// measured 0.38 ms (twice the barriers).


template <int BK>
__global__ __launch_bounds__(512) void tri_contract_big_kernel(TriContractParams p) {
  constexpr int TM = 256, NT = 512, FM = 8, FN = 4, WT = 128, WTN = 64, CH = BK / 8, PER = TM * CH / NT,
                STAGE = TM * BK;
  static_assert((TM * CH) % NT == 0, "tile rows must split into whole load rounds");
  __shared__ __attribute__((aligned(16))) _Float16 S[2][2][STAGE];   // [stage][L, R][row][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int tm = (p.N + TM - 1) / TM, tiles = tm * tm;
  const int total = (int)gridDim.x, per = total >> 3;
  int lin = (int)blockIdx.x;
  if (lin < per * 8) lin = (lin & 7) * per + (lin >> 3);
  const int h = lin / tiles, t = lin - h * tiles;
  const int m0 = (t / tm) * TM, n0 = (t % tm) * TM;
  const size_t plane = (size_t)p.N * p.N;
  const _Float16* L = p.L + h * plane;
  const _Float16* R = p.R + h * plane;
  const _Float16* gl[PER];
  const _Float16* gr[PER];
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int q = it * NT + tid, r = q / CH, c = (q % CH) ^ ct_swz<BK>(r);
    gl[it] = L + (size_t)min(m0 + r, p.N - 1) * p.N + c * 8;
    gr[it] = R + (size_t)min(n0 + r, p.N - 1) * p.N + c * 8;
  }
  auto issue = [&](int k0, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int base = (it * NT + wave * 64) * 8;
#if __HIP_DEVICE_COMPILE__
      __builtin_amdgcn_global_load_lds(gl[it] + k0, &S[st][0][base], 16, 0, 0);
      __builtin_amdgcn_global_load_lds(gr[it] + k0, &S[st][1][base], 16, 0, 0);
#endif
    }
  };
  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, g4 = lane >> 4;
  const int nk = p.N / BK;
  issue(0, 0);
  for (int ks = 0; ks < nk; ++ks) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();   // step ks in LDS for every wave; every wave done with the other stage
    if (ks + 1 < nk) issue((ks + 1) * BK, (ks + 1) & 1);
    const _Float16* Ls = S[ks & 1][0];
    const _Float16* Rs = S[ks & 1][1];
    // every fragment of the step is read before the first MFMA (the scheduling barrier keeps
    // the compiler from interleaving them in small groups, each waiting for its reads)
    constexpr int KK = BK / 32;
    h8 a[KK][FM], b[KK][FN];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn * WTN + j * 16 + r16;
        b[kk][j] = *reinterpret_cast<const h8*>(Rs + row * BK + ((kk * 4 + g4) ^ ct_swz<BK>(row)) * 8);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * WT + i * 16 + r16;
        a[kk][i] = *reinterpret_cast<const h8*>(Ls + row * BK + ((kk * 4 + g4) ^ ct_swz<BK>(row)) * 8);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(b[kk][j], a[kk][i], acc[i][j]);
  }
  _Float16* X = p.X + h * plane;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int gm = m0 + wm * WT + i * 16 + r16;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int gn = n0 + wn * WTN + j * 16 + 4 * g4;
      h4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = (_Float16)(acc[i][j][r] * p.scale);
      if (gm < p.N && gn < p.N) *reinterpret_cast<h4*>(X + (size_t)gm * p.N + gn) = o;
    }
  }
}

template <int TM, int BK = 64, int MINW = 1>
static void launch_contract(lf_context* ctx, const TriContractParams& cp, int H, bool kmajor) {
  const int tm = (cp.N + TM - 1) / TM;
  const dim3 grid((unsigned)(tm * tm * H));
  const bool vec = (cp.N % 8) == 0;
  if (!kmajor) {
    const long long t256 = (cp.N + 255) / 256, t128 = (cp.N + 127) / 128;
    if (TM == 128 && cp.N % 64 == 0 && cp.N >= 768 && t256 * t256 * 65536 * 10 <= t128 * t128 * 16384 * 11) {
      hipLaunchKernelGGL((tri_contract_big_kernel<64>), dim3((unsigned)(t256 * t256 * H)), dim3(512), 0, ctx->stream,
                         cp);
      return;
    }
    if (TM == 128 && cp.N % 64 == 0) {
      // 128-row tiles at two blocks per CU, or, when the grid is only a few waves of blocks
      // and the last one would run mostly empty, 96-row tiles at three per CU.  Measured: at
      // N = 384 (1152 tiles of 128 in 512 slots: 2.25 waves) the 96-row kernel is 3-4%
      // faster; at N = 1024 (16 full waves) it is 11% slower, its operands re-read more often.
      const long long slots = 2LL * ctx->num_cus;
      const int t96 = (cp.N + 95) / 96;
      const long long b128 = (long long)tm * tm * H, b96 = (long long)t96 * t96 * H;
      const double w128 = (double)((b128 + slots - 1) / slots);
      const double w96 = (double)((b96 + slots * 3 / 2 - 1) / (slots * 3 / 2)) * (96.0 * 96.0) / (128.0 * 128.0);
      if (b128 <= 4 * slots && w96 < 0.85 * w128)
        hipLaunchKernelGGL((tri_contract_dma_kernel<64, 96>), dim3((unsigned)b96), dim3(256), 0, ctx->stream, cp);
      else
        hipLaunchKernelGGL((tri_contract_dma_kernel<64, 128>), grid, dim3(256), 0, ctx->stream, cp);
      return;
    }
    if (vec) hipLaunchKernelGGL((tri_contract_kernel<TM, BK, MINW, false, true>), grid, dim3(256), 0, ctx->stream, cp);
    else hipLaunchKernelGGL((tri_contract_kernel<TM, BK, MINW, false, false>), grid, dim3(256), 0, ctx->stream, cp);
  } else {
    if (vec) hipLaunchKernelGGL((tri_contract_kernel<TM, BK, MINW, true, true>), grid, dim3(256), 0, ctx->stream, cp);
    else hipLaunchKernelGGL((tri_contract_kernel<TM, BK, MINW, true, false>), grid, dim3(256), 0, ctx->stream, cp);
  }
}

// ---------------------------------------------------------------------------------------
// Weight-resident persistent kernels (c_z <= 128 and c_hidden <= 128)
// ---------------------------------------------------------------------------------------

constexpr int RS_LD = 136;

// 128 + 8 halves: 16-byte fragment reads of 16 rows hit distinct banks

// The weights of a resident kernel: COUNT matrices of up to 128 x 128 (k, n < 128) into dst[m]
// as [n][k] rows of pitch RS_LD, decoded from the stored codes.  SPLIT: each view is an AF3
// interleaved tensor of 256 stored columns, column c going to row c / 2 of dst[m] (c even) or
// of dst2[m] (c odd).  Every run's loads are issued before the first decode, so the whole
// stage waits for memory once.
// DT >= 0: every view is stored as DT with runs (no gathered view), so the fetches and
// decodes are straight-line code; DT < 0: each run dispatches on its view's dtype and run.
template <int COUNT, int NT, bool SPLIT, int DT>
__device__ __forceinline__ void stage_resident_as(_Float16* const (&dst)[COUNT], const WSrc* const (&src)[COUNT],
                                                  int tid, _Float16* const (&dst2)[COUNT]) {
  constexpr int COLS = SPLIT ? 256 : 128, RUNS = COLS * 128 / 8, PER = (RUNS + NT - 1) / NT;
  auto coords = [&](bool krun, int i, int& n, int& k) {
    if (krun) { n = i >> 4; k = (i & 15) * 8; }
    else { n = (i >> 7) * 8; k = i & 127; }
  };
  u32x4 v[COUNT][PER];
#pragma unroll
  for (int m = 0; m < COUNT; ++m) {
    const bool krun = src[m]->v.run != WRUN_N;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      int n, k;
      coords(krun, min(tid + u * NT, RUNS - 1), n, k);
      if constexpr (DT >= 0) v[m][u] = wrun_fetch_dt<DT>(src[m]->v, wrun_at(src[m]->v, k, n), src[m]->mul);
      else v[m][u] = wrun_fetch(src[m]->v, k, n, src[m]->mul);
    }
  }
#pragma unroll
  for (int m = 0; m < COUNT; ++m) {
    const bool krun = src[m]->v.run != WRUN_N;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      if (tid + u * NT >= RUNS) continue;
      int n, k;
      coords(krun, tid + u * NT, n, k);
      h8 h;
      if constexpr (DT >= 0) h = wrun_decode_dt<DT>(v[m][u], wrun_at(src[m]->v, k, n), src[m]->mul);
      else h = wrun_decode(src[m]->v, v[m][u], k, n, src[m]->mul);
      if (!SPLIT) {
        wrun_put(dst[m], RS_LD, krun, n, k, h);
      } else if (krun) {
        *reinterpret_cast<h8*>(((n & 1) ? dst2[m] : dst[m]) + (n >> 1) * RS_LD + k) = h;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) ((j & 1) ? dst2[m] : dst[m])[((n + j) >> 1) * RS_LD + k] = h[j];
      }
    }
  }
}

// The weights of a resident kernel: COUNT matrices of up to 128 x 128 (k, n < 128) into dst[m]
// as [n][k] rows of pitch RS_LD, decoded from the stored codes.  SPLIT: each view is an AF3
// interleaved tensor of 256 stored columns, column c going to row c / 2 of dst[m] (c even) or
// of dst2[m] (c odd).  Every run's loads are issued before the first decode, so the whole
// stage waits for memory once.  When all views share one stored dtype and none is gathered
// (the usual case: one codec per model), the stage runs as straight-line code for that dtype.
template <int COUNT, int NT, bool SPLIT = false>
__device__ __forceinline__ void stage_resident(_Float16* const (&dst)[COUNT], const WSrc* const (&src)[COUNT],
                                               int tid, _Float16* const (&dst2)[COUNT] = {}) {
  const int dt = src[0]->v.dtype;
  bool uniform = true;
#pragma unroll
  for (int m = 0; m < COUNT; ++m) uniform = uniform && src[m]->v.dtype == dt && src[m]->v.run != WRUN_GATHER;
  if (uniform) {
    switch (dt) {
      case DT_F32: stage_resident_as<COUNT, NT, SPLIT, DT_F32>(dst, src, tid, dst2); return;
      case DT_F16: stage_resident_as<COUNT, NT, SPLIT, DT_F16>(dst, src, tid, dst2); return;
      case DT_BF16: stage_resident_as<COUNT, NT, SPLIT, DT_BF16>(dst, src, tid, dst2); return;
      case DT_I8: stage_resident_as<COUNT, NT, SPLIT, DT_I8>(dst, src, tid, dst2); return;
      default: stage_resident_as<COUNT, NT, SPLIT, DT_I5>(dst, src, tid, dst2); return;
    }
  }
  stage_resident_as<COUNT, NT, SPLIT, -1>(dst, src, tid, dst2);
}

// The a/b projection and gate weights of the project kernels: blocks [a-proj, a-gate, b-proj,
// b-gate] of 128 rows from Ws.  AF3 (p.split): wp[0] and wg[0] are the whole interleaved
// projection and gate tensors.
template <int NT>
__device__ __forceinline__ void stage_project_weights(_Float16* Ws, const TriProjectParams& p, int tid) {
  if (p.split) {
    _Float16* const even[2] = {Ws, Ws + 128 * RS_LD};
    _Float16* const odd[2] = {Ws + 2 * 128 * RS_LD, Ws + 3 * 128 * RS_LD};
    const WSrc* const src[2] = {&p.wp[0], &p.wg[0]};
    stage_resident<2, NT, true>(even, src, tid, odd);
  } else {
    _Float16* const dst[4] = {Ws, Ws + 128 * RS_LD, Ws + 2 * 128 * RS_LD, Ws + 3 * 128 * RS_LD};
    const WSrc* const src[4] = {&p.wp[0], &p.wg[0], &p.wp[1], &p.wg[1]};
    stage_resident<4, NT>(dst, src, tid);
  }
}

// Weights of the a/b projections ([h][k] f16, padded rows) and a block of 8 waves; each
// wave LayerNorms its 16-row tiles straight into MFMA A fragments (FragTile), so LDS holds
// weights only.
constexpr int PR_WAVES = 8;

template <int ACT>
__global__ __launch_bounds__(512) void tri_project_resident_kernel(TriProjectParams p) {
  __shared__ __attribute__((aligned(16))) _Float16 Ws[4 * 128 * RS_LD];  // a-proj, a-gate, b-proj, b-gate as [h][k]
  __shared__ __attribute__((aligned(16))) float Bs[4 * 128];              // the four bias vectors
  __shared__ __attribute__((aligned(16))) float Gs[2 * 128];              // LN_in scale, offset
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  stage_project_weights<512>(Ws, p, tid);
  stage_vec(Bs, p.bp[0], p.H, 0.f, 128, tid, 512);
  stage_vec(Bs + 128, p.bg[0], p.H, 0.f, 128, tid, 512);
  stage_vec(Bs + 256, p.bp[1], p.H, 0.f, 128, tid, 512);
  stage_vec(Bs + 384, p.bg[1], p.H, 0.f, 128, tid, 512);
  stage_vec(Gs, p.ln_s, p.C, 1.f, 128, tid, 512);
  stage_vec(Gs + 128, p.ln_o, p.C, 0.f, 128, tid, 512);
  __syncthreads();

  const int r16 = lane & 15, g = lane >> 4, q4 = g * 4, kq = g * 8;
  const int ntiles = (p.P + 15) >> 4, stride = gridDim.x * PR_WAVES;
  const bool vec_store = (p.P & 3) == 0;
  // Loads for tile t+1 (rows and mask) are issued before tile t's stores: gfx9 counts loads
  // and stores on one in-order counter, so a wait on anything issued after a store would
  // also wait for the store.
  FragTile<ACT> t;
  float mnext[4];
  auto prefetch = [&](int tl) {
    const int r0 = tl * 16, nv = min(16, p.P - r0);
    frag_load(t, p.z, (size_t)r0, nv, p.C, lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) mnext[i] = p.mask[r0 + (q4 + i < nv ? q4 + i : 0)];
  };
  int tile = blockIdx.x * PR_WAVES + wave;
  if (tile < ntiles) prefetch(tile);
  for (; tile < ntiles; tile += stride) {
    const int row0 = tile * 16, nvalid = min(16, p.P - row0);
    h8 a[4];
    {
      float x[4][8];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[j][e] = (32 * j + kq + e < p.C) ? t.get(j, e) : 0.f;
      frag_ln<4>(x, a, r16 < nvalid, p.C, Gs, Gs + 128, p.eps, p.fast_var, lane);
    }
    float m[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) m[i] = q4 + i < nvalid ? mnext[i] : 0.f;
    const int next = tile + stride;
    if (next < ntiles) prefetch(next);
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
      const int which = pass >> 1, hh = (pass & 1) * 64;
      const _Float16* Wp = Ws + (which * 2) * 128 * RS_LD;
      const _Float16* Wg = Wp + 128 * RS_LD;
      f4 acc[8];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const h8 bp = *reinterpret_cast<const h8*>(Wp + (hh + t4 * 16 + r16) * RS_LD + kq);
        const h8 bg = *reinterpret_cast<const h8*>(Wg + (hh + t4 * 16 + r16) * RS_LD + kq);
        acc[t4] = mfma16(a[0], bp, f4{0.f, 0.f, 0.f, 0.f});
        acc[4 + t4] = mfma16(a[0], bg, f4{0.f, 0.f, 0.f, 0.f});
      }
#pragma unroll
      for (int j = 1; j < 4; ++j) {
        __builtin_amdgcn_sched_barrier(0);   // keep one k-step's fragments live at a time
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          const h8 bp = *reinterpret_cast<const h8*>(Wp + (hh + t4 * 16 + r16) * RS_LD + 32 * j + kq);
          const h8 bg = *reinterpret_cast<const h8*>(Wg + (hh + t4 * 16 + r16) * RS_LD + 32 * j + kq);
          acc[t4] = mfma16(a[j], bp, acc[t4]);
          acc[4 + t4] = mfma16(a[j], bg, acc[4 + t4]);
        }
      }
      _Float16* dst = which ? p.out[1] : p.out[0];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const int h = hh + t4 * 16 + r16;
        if (h >= p.H) continue;
        const float bpp = Bs[which * 256 + h], bgg = Bs[which * 256 + 128 + h];
        h4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (_Float16)((acc[t4][i] + bpp) * (m[i] * sigmoidf_(acc[4 + t4][i] + bgg)));
        _Float16* d = dst + (size_t)h * p.P + row0 + q4;
        if (vec_store && q4 + 4 <= nvalid) {
          *reinterpret_cast<h4*>(d) = o;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (q4 + i < nvalid) d[i] = o[i];
        }
      }
    }
  }
}

constexpr int OR_WAVES = 8;
constexpr int OR_SCR = 16 * 132;   // floats of per-wave scratch: X^T tile (f16) then the f32 update

template <int ACT>
__global__ __launch_bounds__(512) void tri_output_resident_kernel(TriOutputParams p) {
  typedef typename Act<ACT>::T T;
  __shared__ __attribute__((aligned(16))) _Float16 Wz[128 * RS_LD];   // [c][h]
  __shared__ __attribute__((aligned(16))) _Float16 Wg[128 * RS_LD];   // [c][k]
  __shared__ __attribute__((aligned(16))) float Scr[OR_WAVES * OR_SCR];
  __shared__ __attribute__((aligned(16))) float Vs[6 * 128];           // bz, bg, centre-norm scale/offset, LN_in scale/offset
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  {
    _Float16* const dst[2] = {Wz, Wg};
    const WSrc* const src[2] = {&p.wz, &p.wg};
    stage_resident<2, 512>(dst, src, tid);
  }
  stage_vec(Vs, p.bz, p.C, 0.f, 128, tid, 512);
  stage_vec(Vs + 128, p.bg, p.C, 0.f, 128, tid, 512);
  stage_vec(Vs + 256, p.ln_out_s, p.H, 1.f, 128, tid, 512);
  stage_vec(Vs + 384, p.ln_out_o, p.H, 0.f, 128, tid, 512);
  stage_vec(Vs + 512, p.ln_in_s, p.C, 1.f, 128, tid, 512);
  stage_vec(Vs + 640, p.ln_in_o, p.C, 0.f, 128, tid, 512);
  __syncthreads();

  const int r16 = lane & 15, g = lane >> 4, q4 = g * 4, kq = g * 8;
  const int ntiles = (p.P + 15) >> 4, stride = gridDim.x * OR_WAVES;
  _Float16* Xw = reinterpret_cast<_Float16*>(Scr + wave * OR_SCR);   // [16][RS_LD] f16
  float* Ow = Scr + wave * OR_SCR;                                    // [16][132] f32
  const bool vec_x = (p.P & 7) == 0;
  const T* zin = static_cast<const T*>(p.z);
  T* out = static_cast<T*>(p.out);
  // No cross-tile prefetch here: holding the next tile's X and z words across the two GEMMs
  // pushes this kernel past 256 VGPRs (spills); two waves per SIMD hide the loads instead.
  FragTile<ACT> t;
  for (int tile = blockIdx.x * OR_WAVES + wave; tile < ntiles; tile += stride) {
    const int row0 = tile * 16, nvalid = min(16, p.P - row0);
    // X tile [h][16 rows] -> Xw[row][h]; z rows into A-fragment layout
    frag_load(t, p.z, (size_t)row0, nvalid, p.C, lane);
    if (vec_x && nvalid == 16) {
      h8 xv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int idx = lane + 64 * j, h = idx >> 1, seg = idx & 1;
        xv[j] = *reinterpret_cast<const h8*>(p.X + (size_t)(h < p.H ? h : 0) * p.P + row0 + seg * 8);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int idx = lane + 64 * j, h = idx >> 1, seg = idx & 1;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) Xw[(seg * 8 + jj) * RS_LD + h] = h < p.H ? xv[j][jj] : (_Float16)0.f;
      }
    } else {
#pragma unroll 1
      for (int idx = lane; idx < 128 * 16; idx += 64) {
        const int h = idx >> 4, r = idx & 15;
        const _Float16 v = p.X[(size_t)(h < p.H ? h : 0) * p.P + row0 + (r < nvalid ? r : 0)];
        Xw[r * RS_LD + h] = (h < p.H && r < nvalid) ? v : (_Float16)0.f;
      }
    }
    // centre LN over h into A fragments (scaled-X epsilon); LN_in(z) into A fragments
    h8 ax[4], az[4];
    {
      float x[4][8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h8 v = *reinterpret_cast<const h8*>(Xw + r16 * RS_LD + 32 * j + kq);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[j][e] = (float)v[e];
      }
      frag_ln<4>(x, ax, r16 < nvalid, p.H, Vs + 256, Vs + 384, p.eps_x, p.fast_var, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[j][e] = (32 * j + kq + e < p.C) ? t.get(j, e) : 0.f;
      frag_ln<4>(x, az, r16 < nvalid, p.C, Vs + 512, Vs + 640, p.eps, p.fast_var, lane);
    }
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
      const int c0 = pass * 64;
      f4 accz[4], accg[4];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        accz[t4] = mfma16(ax[0], *reinterpret_cast<const h8*>(Wz + (c0 + t4 * 16 + r16) * RS_LD + kq),
                          f4{0.f, 0.f, 0.f, 0.f});
        accg[t4] = mfma16(az[0], *reinterpret_cast<const h8*>(Wg + (c0 + t4 * 16 + r16) * RS_LD + kq),
                          f4{0.f, 0.f, 0.f, 0.f});
      }
#pragma unroll
      for (int j = 1; j < 4; ++j) {
        __builtin_amdgcn_sched_barrier(0);   // keep one k-step's fragments live at a time
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          accz[t4] = mfma16(ax[j], *reinterpret_cast<const h8*>(Wz + (c0 + t4 * 16 + r16) * RS_LD + 32 * j + kq),
                            accz[t4]);
          accg[t4] = mfma16(az[j], *reinterpret_cast<const h8*>(Wg + (c0 + t4 * 16 + r16) * RS_LD + 32 * j + kq),
                            accg[t4]);
        }
      }
      // stage the gated update as f32 [row][c] (Xw is dead: its fragments are in registers)
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const int c = c0 + t4 * 16 + r16;
        const float bz = Vs[c], bg = Vs[128 + c];
#pragma unroll
        for (int i = 0; i < 4; ++i) Ow[(q4 + i) * 132 + c] = (accz[t4][i] + bz) * sigmoidf_(accg[t4][i] + bg);
      }
    }
    // lane: row r16, channels 32j + 8g .. +8; the residual rows are re-read (L2-resident: this
    // wave loaded them one tile ago) instead of being held in registers across the GEMMs.
    FragTile<ACT> zraw;
    if (p.accumulate) frag_load(zraw, p.z, (size_t)row0, nvalid, p.C, lane);
    if (r16 < nvalid) {
      T* orow = out + (size_t)(row0 + r16) * p.C;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 u0 = *reinterpret_cast<const float4*>(Ow + r16 * 132 + 32 * j + kq);
        const float4 u1 = *reinterpret_cast<const float4*>(Ow + r16 * 132 + 32 * j + kq + 4);
        const float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
        if (p.C == 128) {
          float w8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) w8[e] = p.accumulate ? u[e] + zraw.get(j, e) : u[e];
          uint4 o[FragTile<ACT>::NV];
          pack8<ACT>(w8, o);
#pragma unroll
          for (int v = 0; v < FragTile<ACT>::NV; ++v)
            *reinterpret_cast<uint4*>(orow + 32 * j + kq + v * (16 / (int)sizeof(T))) = o[v];
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int c = 32 * j + kq + e;
            if (c < p.C) Act<ACT>::st(orow + c, p.accumulate ? u[e] + Act<ACT>::ld(zin + (size_t)(row0 + r16) * p.C + c) : u[e]);
          }
        }
      }
    }
  }
}

// Project kernels for c_z = c_hidden = 128 (every AF2/AF3 pair width at production size),
// weights resident in LDS.  The gate weights and biases arrive pre-multiplied by -log2(e),
// so a gate is rcp(1 + exp2(acc)).  tri_project_v2_kernel (partial tiles) carries TPW 16-row
// tiles per wave, so with TPW = 2 every weight fragment read from LDS feeds two MFMAs; a wave
// walks tiles w, w + nw, w + 2nw, ... TPW at a time, the last step running only the tiles it
// has.  One tile per wave at 12 waves is what runs: two tiles need registers that leave two
// waves per SIMD, measured slower.
constexpr float TRI_NLOG2E = -1.4426950408889634f;
// waves per block and 16-row tiles per wave of the 128-wide project kernels (16 waves spill)
constexpr int TRI_P_NWV = 12, TRI_P_TPW = 1;
// waves per block of the output kernel: 12 (three per SIMD, one X buffer each) for 2-byte
// activations; f32 rows need more registers than three waves per SIMD leave, so 8 (two X
// buffers each).  Measured at N = 384: 43.9 -> 39.9 us with 12 waves for bf16, while f32 at
// 12 waves spills and is 4-7% slower than at 8.
template <int ACT>
constexpr int tri_o_nwv() { return ACT == DT_F32 ? 8 : 12; }

// The 16 pairs of a project tile: row r is pair src0 + r * sstride, stored at out0 + r of every
// channel plane, r < nvalid.  Tile t normally holds pairs 16t .. 16t + 15 in place.  With
// kmajor_out (the incoming direction) tile t = j * ceil(N/16) + kb holds the pairs (16kb + r, j)
// and stores them at j * N + 16kb + r: each plane then holds a^T (b^T), so the contraction
// reads both operands with k contiguous, as in the outgoing direction.
struct TileGeom {
  int src0, sstride, out0, nvalid;
};

__device__ __forceinline__ TileGeom tile_geom(const TriProjectParams& p, int tile) {
  if (!p.kmajor_out) {
    const int r0 = tile * 16;
    return TileGeom{r0, 1, r0, min(16, p.P - r0)};
  }
  const int nkb = (p.N + 15) >> 4, j = tile / nkb, kb = tile - j * nkb;
  return TileGeom{kb * 16 * p.N + j, p.N, j * p.N + kb * 16, min(16, p.N - kb * 16)};
}

template <int ACT>
__device__ __forceinline__ void tri_tile_load(FragTile<ACT, 4>& t, float (&m)[4], const TriProjectParams& p, int tile,
                                              int lane) {
  const TileGeom g = tile_geom(p, tile);
  const int r16 = lane & 15, q4 = (lane >> 4) * 4;
  frag_load_row(t, p.z, (size_t)g.src0 + (size_t)(r16 < g.nvalid ? r16 : 0) * g.sstride, 128, lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) m[i] = q4 + i < g.nvalid ? p.mask[g.src0 + (q4 + i) * g.sstride] : 0.f;
}

template <int ACT, int NWV, int TPW>
__global__ __launch_bounds__(64 * NWV) void tri_project_v2_kernel(TriProjectParams p) {
  constexpr int NT = 64 * NWV;
  __shared__ __attribute__((aligned(16))) _Float16 Ws[4 * 128 * RS_LD];  // a-proj, a-gate', b-proj, b-gate' [h][k]
  __shared__ __attribute__((aligned(16))) float Bs[4 * 128];              // the four bias vectors (gates scaled)
  __shared__ __attribute__((aligned(16))) float Gs[2 * 128];              // LN_in scale, offset
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  stage_project_weights<NT>(Ws, p, tid);
  for (int i = tid; i < 128; i += NT) {
    Bs[i] = p.bp[0] ? p.bp[0][i] : 0.f;
    Bs[128 + i] = p.bg[0] ? TRI_NLOG2E * p.bg[0][i] : 0.f;
    Bs[256 + i] = p.bp[1] ? p.bp[1][i] : 0.f;
    Bs[384 + i] = p.bg[1] ? TRI_NLOG2E * p.bg[1][i] : 0.f;
  }
  stage_vec(Gs, p.ln_s, 128, 1.f, 128, tid, NT);
  stage_vec(Gs + 128, p.ln_o, 128, 0.f, 128, tid, NT);

  const int r16 = lane & 15, g4 = lane >> 4, q4 = g4 * 4, kq = g4 * 8;
  const int ntiles = p.kmajor_out ? p.N * ((p.N + 15) >> 4) : (p.P + 15) >> 4, nw = gridDim.x * NWV;
  const bool vec_store = ((p.kmajor_out ? p.N : p.P) & 3) == 0;
  int tile = blockIdx.x * NWV + wave;
  FragTile<ACT, 4> t[TPW];
  float mk[TPW][4];
  if (tile < ntiles) {
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) tri_tile_load(t[tt], mk[tt], p, tile + tt * nw < ntiles ? tile + tt * nw : tile, lane);
  }
  __syncthreads();

  for (; tile < ntiles; tile += TPW * nw) {
    bool valid[TPW];
    int out0[TPW], nval[TPW];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      valid[tt] = tile + tt * nw < ntiles;   // wave-uniform
      const TileGeom g = tile_geom(p, valid[tt] ? tile + tt * nw : tile);
      out0[tt] = g.out0;
      nval[tt] = g.nvalid;
    }
    h8 xa[TPW][4];
    if constexpr (TPW == 2) frag_ln_raw2(t[0], t[1], xa[0], xa[1], 128, Gs, Gs + 128, p.eps, p.fast_var, lane);
    else frag_ln_raw1(t[0], xa[0], 128, Gs, Gs + 128, p.eps, p.fast_var, lane);
    float m[TPW][4];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) m[tt][i] = mk[tt][i];
    // loads of the next tiles are issued before this step's stores (one in-order counter)
    const int nt = tile + TPW * nw;
    if (nt < ntiles) {
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt) tri_tile_load(t[tt], mk[tt], p, nt + tt * nw < ntiles ? nt + tt * nw : nt, lane);
    }
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
      const int which = pass >> 1, hh = (pass & 1) * 64;
      const _Float16* Wp = Ws + (which * 2) * 128 * RS_LD;
      const _Float16* Wg = Wp + 128 * RS_LD;
      const float* bp = Bs + which * 256 + hh;
      const float* bg = bp + 128;
      f4 acc[TPW][8];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const float b0 = bp[t4 * 16 + r16], b1 = bg[t4 * 16 + r16];
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
          acc[tt][t4] = f4{b0, b0, b0, b0};
          acc[tt][4 + t4] = f4{b1, b1, b1, b1};
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h8 wb[8];
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          wb[t4] = *reinterpret_cast<const h8*>(Wp + (hh + t4 * 16 + r16) * RS_LD + 32 * j + kq);
          wb[4 + t4] = *reinterpret_cast<const h8*>(Wg + (hh + t4 * 16 + r16) * RS_LD + 32 * j + kq);
        }
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
          if (tt > 0 && !valid[tt]) break;
#pragma unroll
          for (int u = 0; u < 8; ++u) acc[tt][u] = mfma16(xa[tt][j], wb[u], acc[tt][u]);
        }
        __builtin_amdgcn_sched_barrier(0);   // one k-step's weight fragments live at a time
      }
      _Float16* dst = which ? p.out[1] : p.out[0];
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt) {
        if (tt > 0 && !valid[tt]) break;
        const int nvalid = nval[tt];
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          const int h = hh + t4 * 16 + r16;
          h4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            o[i] = (_Float16)(m[tt][i] * acc[tt][t4][i] *
                              __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(acc[tt][4 + t4][i])));
          _Float16* d = dst + (size_t)h * p.P + out0[tt] + q4;
          if (vec_store && q4 + 4 <= nvalid) {
            *reinterpret_cast<h4*>(d) = o;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (q4 + i < nvalid) d[i] = o[i];
          }
        }
      }
    }
  }
}

// Project kernel for c_z = c_hidden = 128 when every tile is whole (P % 16 == 0, or N % 16 == 0
// for the transposed incoming store): the v2 work as straight-line code.  The next tile's rows
// and mask are loaded at the top of a step (clamped, never skipped), the four passes are
// unrolled, and the next rows are taken into registers (an asm use forces the wait) after the
// last pass's MFMAs and before its stores: every wait on the in-order vector-memory counter
// then covers loads issued earlier in the same step, never the stores that follow them.
template <int ACT, int NWV, bool ST>
__global__ __launch_bounds__(64 * NWV) void tri_project_v3_kernel(TriProjectParams p) {
  constexpr int NT = 64 * NWV;
  __shared__ __attribute__((aligned(16))) _Float16 Ws[4 * 128 * RS_LD];  // a-proj, a-gate', b-proj, b-gate' [h][k]
  __shared__ __attribute__((aligned(16))) h4 Bt[4 * 128];                 // the four bias vectors (gates scaled), f16 hi + lo
  __shared__ __attribute__((aligned(16))) float Gs[2 * 128];              // LN_in scale, offset
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4, q4 = g4 * 4, kq = g4 * 8;
  // A operand of the bias MFMA: ones at k = 0, 1 (lanes 0-15 supply k 0..3), zeros elsewhere
  const _Float16 one = (_Float16)(g4 == 0 ? 1.f : 0.f);
  const h4 ones = h4{one, one, (_Float16)0.f, (_Float16)0.f};
  const int ntiles = p.kmajor_out ? p.N * (p.N >> 4) : p.P >> 4, nw = gridDim.x * NWV;
  auto fetch = [&](int tl, FragTile<ACT, 4>& t, float (&m)[4]) __attribute__((always_inline)) {
    const TileGeom g = tile_geom(p, tl);
    frag_load_row(t, p.z, (size_t)g.src0 + (size_t)r16 * g.sstride, 128, lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) m[i] = p.mask[g.src0 + (q4 + i) * g.sstride];
  };
  // the first tile's rows load while the weights are decoded into LDS (clamped, never skipped)
  int tile = blockIdx.x * NWV + wave;
  FragTile<ACT, 4> tc;
  float mc[4];
  fetch(tile < ntiles ? tile : 0, tc, mc);
  stage_project_weights<NT>(Ws, p, tid);
  // a bias b as the B operand of a 16x16x16 MFMA: k rows 0 and 1 hold hi = f16(b) and
  // lo = f16(b - hi), which the ones in the A operand sum back to b within 2^-22 relative
  auto split = [](float b) {
    const _Float16 hi = (_Float16)b;
    return h4{hi, (_Float16)(b - (float)hi), (_Float16)0.f, (_Float16)0.f};
  };
  for (int i = tid; i < 128; i += NT) {
    Bt[i] = split(p.bp[0] ? p.bp[0][i] : 0.f);
    Bt[128 + i] = split(p.bg[0] ? TRI_NLOG2E * p.bg[0][i] : 0.f);
    Bt[256 + i] = split(p.bp[1] ? p.bp[1][i] : 0.f);
    Bt[384 + i] = split(p.bg[1] ? TRI_NLOG2E * p.bg[1][i] : 0.f);
  }
  stage_vec(Gs, p.ln_s, 128, 1.f, 128, tid, NT);
  stage_vec(Gs + 128, p.ln_o, 128, 0.f, 128, tid, NT);
  __syncthreads();
  if (tile >= ntiles) return;
  for (; tile < ntiles; tile += nw) {
    const TileGeom tg = tile_geom(p, tile);
    const int out0 = tg.out0;
    const uint32_t lofs = ((uint32_t)r16 * (uint32_t)p.P + (uint32_t)(out0 + q4)) * (uint32_t)sizeof(_Float16);
    h8 xa[4];
    if constexpr (ST) {
      float m0, i0;
      frag_stats_raw(tc, 128, p.eps, p.fast_var, m0, i0);
      // the output kernel normalises the same z rows again for its gate: it reads these
      if (lane < 16) p.stats[tg.src0 + r16 * tg.sstride] = make_float2(m0, i0);
      frag_ln_given(tc, xa, Gs, Gs + 128, m0, i0, lane);
    } else {
      frag_ln_raw1(tc, xa, 128, Gs, Gs + 128, p.eps, p.fast_var, lane);
    }
    const int nt = tile + nw < ntiles ? tile + nw : tile;   // the last step reloads its own tile
    FragTile<ACT, 4> tn;
    float mn[4];
    fetch(nt, tn, mn);
    auto pass = [&](auto pass_tag) __attribute__((always_inline)) {
      constexpr int PS = decltype(pass_tag)::value, which = PS >> 1, hh = (PS & 1) * 64;
      const _Float16* Wp = Ws + (which * 2) * 128 * RS_LD;
      const _Float16* Wg = Wp + 128 * RS_LD;
      // the accumulators start at the biases, through the matrix core (no per-register moves)
      const h4* btp = Bt + which * 256 + hh + r16;
      f4 acc[8];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        acc[t4] = mfma16k16(ones, btp[t4 * 16], f4{0.f, 0.f, 0.f, 0.f});
        acc[4 + t4] = mfma16k16(ones, btp[128 + t4 * 16], f4{0.f, 0.f, 0.f, 0.f});
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h8 wb[8];
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          wb[t4] = *reinterpret_cast<const h8*>(Wp + (hh + t4 * 16 + r16) * RS_LD + 32 * j + kq);
          wb[4 + t4] = *reinterpret_cast<const h8*>(Wg + (hh + t4 * 16 + r16) * RS_LD + 32 * j + kq);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[u] = mfma16(xa[j], wb[u], acc[u]);
        __builtin_amdgcn_sched_barrier(0);   // one k-step's weight fragments live at a time
      }
      if constexpr (PS == 3) {
        launder(tn);
        asm volatile("" : "+v"(mn[0]), "+v"(mn[1]), "+v"(mn[2]), "+v"(mn[3]));
      }
      // a wave-uniform base per 16 channels plus one 32-bit lane offset (P < 2^27): scalar
      // base + vector offset stores, no 64-bit address arithmetic per store
      char* dst = reinterpret_cast<char*>(which ? p.out[1] : p.out[0]);
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        h4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = (_Float16)(mc[i] * acc[t4][i] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(acc[4 + t4][i])));
        *reinterpret_cast<h4*>(dst + (size_t)(hh + t4 * 16) * p.P * sizeof(_Float16) + lofs) = o;
      }
    };
    pass(std::integral_constant<int, 0>{});
    __builtin_amdgcn_sched_barrier(0);
    pass(std::integral_constant<int, 1>{});
    __builtin_amdgcn_sched_barrier(0);
    pass(std::integral_constant<int, 2>{});
    __builtin_amdgcn_sched_barrier(0);
    pass(std::integral_constant<int, 3>{});
    tc = tn;
#pragma unroll
    for (int i = 0; i < 4; ++i) mc[i] = mn[i];
  }
}

constexpr int O2_LD = 136;   // X patch pitch (halves)

// Xw[r][h] = X[h][row0 + r] for r < 16, element by element (rows past nvalid zero): the
// path for partial tiles and for P % 8 != 0
template <int ACT>
__device__ __forceinline__ void x_transpose(_Float16* Xw, const _Float16* X, int P, int row0, int nvalid, int lane) {
#pragma unroll 1
  for (int idx = lane; idx < 128 * 16; idx += 64) {
    const int h = idx >> 4, r = idx & 15;
    const _Float16 v = X[(size_t)h * P + row0 + (r < nvalid ? r : 0)];
    Xw[r * O2_LD + h] = r < nvalid ? v : (_Float16)0.f;
  }
}

// x_transpose for a whole tile with P % 8 == 0, in two halves: the 16-byte global loads
// (issued a tile ahead) and the transposing LDS stores.
__device__ __forceinline__ void x_fetch(h8 (&xv)[4], const _Float16* X, int P, int row0, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = lane + 64 * j, h = idx >> 1, seg = idx & 1;
    xv[j] = *reinterpret_cast<const h8*>(X + (size_t)h * P + row0 + seg * 8);
  }
}

__device__ __forceinline__ void x_put(_Float16* Xw, const h8 (&xv)[4], int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = lane + 64 * j, h = idx >> 1, seg = idx & 1;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) Xw[(seg * 8 + jj) * O2_LD + h] = xv[j][jj];
  }
}

// Output kernel for c_z = c_hidden = 128, one 16-pair tile per wave step.  The steady-state
// loop runs whole tiles as straight-line code: the next tile's z rows and X columns are loaded
// (clamped, never skipped) at the top of a step and transposed into the wave's other LDS
// buffer between the second pass's MFMAs and that pass's stores (two X buffers, 8 waves), or
// loaded between the two passes and transposed after the tile into its one buffer (12 waves,
// whose LDS and registers allow only that); the residual comes from the z rows already held.  Every wait on the in-order vector-memory counter then
// covers loads issued earlier in the same step and none of the stores issued after them.  A
// partial last tile (P % 16 pairs) runs once after the loop, masked, on the wave owning it.
// The weights are the MFMA A operand (resident in LDS), so a lane's accumulators hold four
// consecutive channels of one pair; the gate weights and bias arrive pre-multiplied by
// -log2(e): sigmoid = rcp(1 + exp2(acc)).
template <int ACT, int NWV, bool VECX, bool ZS>
__global__ __launch_bounds__(64 * NWV) void tri_output_v3_kernel(TriOutputParams p) {
  constexpr int NT = 64 * NWV;
  // X patch buffers per wave: two (the next tile's X is transposed during the current tile's
  // second pass) with 8 waves; one with more waves (it is transposed after the tile, into the
  // buffer the tile has finished with), which the LDS budget requires
  constexpr int XB = NWV <= 8 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) _Float16 Wz[128 * RS_LD];   // [c][h]
  __shared__ __attribute__((aligned(16))) _Float16 Wg[128 * RS_LD];   // [c][k], pre-scaled
  __shared__ __attribute__((aligned(16))) _Float16 Xs[NWV][XB][16 * O2_LD];
  __shared__ __attribute__((aligned(16))) float Vs[6 * 128];         // bz, bg', centre-norm s/o, LN_in s/o
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nfull = p.P >> 4, nw = gridDim.x * NWV;
  // the first tile's z rows and X columns load while the weights are decoded into LDS
  // (clamped, never skipped)
  int tile = blockIdx.x * NWV + wave;
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;
  FragTile<ACT, 4> zc;
  float2 zs = make_float2(0.f, 1.f);
  h8 xv[4];
  {
    const int t0 = tile < nfull ? tile : 0;
    frag_load(zc, p.z, (size_t)t0 * 16, 16, 128, lane);
    if constexpr (ZS) zs = p.stats[t0 * 16 + r16];
    if constexpr (VECX) x_fetch(xv, p.X, p.P, t0 * 16, lane);
  }
  // the biases and LayerNorm vectors (threads 0-127, one channel each) are loaded before the
  // weights, so their round trip overlaps the weight stage's instead of following it
  float vv[6] = {0.f, 0.f, 1.f, 0.f, 1.f, 0.f};
  if (tid < 128) {   // wave-uniform
    if (p.bz) vv[0] = p.bz[tid];
    if (p.bg) vv[1] = TRI_NLOG2E * p.bg[tid];
    if (p.ln_out_s) vv[2] = p.ln_out_s[tid];
    if (p.ln_out_o) vv[3] = p.ln_out_o[tid];
    if (p.ln_in_s) vv[4] = p.ln_in_s[tid];
    if (p.ln_in_o) vv[5] = p.ln_in_o[tid];
  }
  {
    _Float16* const dst[2] = {Wz, Wg};
    const WSrc* const src[2] = {&p.wz, &p.wg};
    stage_resident<2, NT>(dst, src, tid);
  }
  if (tid < 128) {
#pragma unroll
    for (int q = 0; q < 6; ++q) Vs[128 * q + tid] = vv[q];
  }
  __syncthreads();

  // One tile: LN_out of X (LDS buffer Xc) and LN_in of z (zc), then two passes of 64 output
  // channels.  A pass stages its f32 update in Xc (the X fragments are in registers by then)
  // and each lane writes its own pair r16, channels c0 + 32jj + 8*g4 .. +7: the layout of its
  // z fragment, which holds the residual.  `between` runs after the second pass's MFMAs.
  auto run_tile = [&](auto full_tag, const FragTile<ACT, 4>& zc, float2 zs, _Float16* Xc, int row0, int nval,
                      auto&& mid, auto&& between) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full_tag)::value;
    h8 ax[4], az[4];
    {
      FragTile<DT_F16, 4> x;
#pragma unroll
      for (int j = 0; j < 4; ++j) x.raw[j][0] = *reinterpret_cast<const u32x4*>(Xc + r16 * O2_LD + 32 * j + kq);
      frag_ln_raw1(x, ax, 128, Vs + 256, Vs + 384, p.eps_x, p.fast_var, lane);
    }
    {
      FragTile<ACT, 4> zl = zc;
      if constexpr (ZS) frag_ln_given(zl, az, Vs + 512, Vs + 640, zs.x, zs.y, lane);
      else frag_ln_raw1(zl, az, 128, Vs + 512, Vs + 640, p.eps, p.fast_var, lane);
    }
    float* Us = reinterpret_cast<float*>(Xc);   // [16 pairs][68] f32 (pitch 68: no bank conflicts)
    auto pass = [&](auto pass_tag) __attribute__((always_inline)) {
      constexpr int PS = decltype(pass_tag)::value, c0 = PS * 64;
      f4 accz[4], accg[4];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const float4 bz = *reinterpret_cast<const float4*>(Vs + c0 + t4 * 16 + 4 * g4);
        const float4 bg = *reinterpret_cast<const float4*>(Vs + 128 + c0 + t4 * 16 + 4 * g4);
        accz[t4] = f4{bz.x, bz.y, bz.z, bz.w};
        accg[t4] = f4{bg.x, bg.y, bg.z, bg.w};
      }
      // one k step's weight fragments live at a time (with one X buffer, the budget of three
      // waves per SIMD: half a k step's)
      constexpr int TH = XB == 2 ? 4 : 2;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int th = 0; th < 4; th += TH) {
          h8 wz[TH], wg[TH];
#pragma unroll
          for (int u = 0; u < TH; ++u) {
            wz[u] = *reinterpret_cast<const h8*>(Wz + (c0 + (th + u) * 16 + r16) * RS_LD + 32 * j + kq);
            wg[u] = *reinterpret_cast<const h8*>(Wg + (c0 + (th + u) * 16 + r16) * RS_LD + 32 * j + kq);
          }
#pragma unroll
          for (int u = 0; u < TH; ++u) {
            accz[th + u] = mfma16(wz[u], ax[j], accz[th + u]);
            accg[th + u] = mfma16(wg[u], az[j], accg[th + u]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        float4 v;
        v.x = accz[t4][0] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(accg[t4][0]));
        v.y = accz[t4][1] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(accg[t4][1]));
        v.z = accz[t4][2] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(accg[t4][2]));
        v.w = accz[t4][3] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(accg[t4][3]));
        *reinterpret_cast<float4*>(Us + r16 * 68 + t4 * 16 + 4 * g4) = v;
      }
      if constexpr (PS == 1 && XB == 2) between();
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const float4 u0 = *reinterpret_cast<const float4*>(Us + r16 * 68 + 32 * jj + 8 * g4);
        const float4 u1 = *reinterpret_cast<const float4*>(Us + r16 * 68 + 32 * jj + 8 * g4 + 4);
        float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
        if (p.accumulate) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] += zc.get(2 * PS + jj, e);
        }
        const size_t idx = (size_t)(row0 + r16) * 128 + c0 + 32 * jj + 8 * g4;
        const float lo[4] = {v[0], v[1], v[2], v[3]}, hi[4] = {v[4], v[5], v[6], v[7]};
        if (FULL || r16 < nval) {
          st4v<ACT>(p.out, idx, lo);
          st4v<ACT>(p.out, idx + 4, hi);
        }
      }
    };
    pass(std::integral_constant<int, 0>{});
    __builtin_amdgcn_sched_barrier(0);
    mid();
    pass(std::integral_constant<int, 1>{});
    if constexpr (XB == 1) between();
  };

  if (tile < nfull) {
    if constexpr (VECX) {
      x_put(Xs[wave][0], xv, lane);
    } else {
      x_transpose<ACT>(Xs[wave][0], p.X, p.P, tile * 16, 16, lane);
    }
    int cur = 0;
    for (; tile < nfull; tile += nw) {
      const int nt = tile + nw < nfull ? tile + nw : tile;   // the last step reloads its own tile
      FragTile<ACT, 4> zn;
      float2 zsn = zs;
      h8 xn[4];
      // the next tile's rows load at the top of the step (two X buffers), or between the two
      // passes (one buffer: fewer registers live through the first pass)
      auto fetch_next = [&]() __attribute__((always_inline)) {
        frag_load(zn, p.z, (size_t)nt * 16, 16, 128, lane);
        if constexpr (ZS) zsn = p.stats[nt * 16 + r16];
        if constexpr (VECX) x_fetch(xn, p.X, p.P, nt * 16, lane);
      };
      if constexpr (XB == 2) fetch_next();
      _Float16* Xn = Xs[wave][XB == 2 ? cur ^ 1 : 0];
      run_tile(std::true_type{}, zc, zs, Xs[wave][XB == 2 ? cur : 0], tile * 16, 16, [&]() __attribute__((always_inline)) {
        if constexpr (XB == 1) fetch_next();
      }, [&]() __attribute__((always_inline)) {
        if constexpr (VECX) x_put(Xn, xn, lane);
        else x_transpose<ACT>(Xn, p.X, p.P, nt * 16, 16, lane);
      });
      // take the next rows now (an asm use forces the wait here, within this step, where the
      // counter wait cannot cover this step's stores), not at their first use next step
      launder(zn);
      if constexpr (ZS) asm volatile("" : "+v"(zsn.x), "+v"(zsn.y));
      zc = zn;
      zs = zsn;
      if constexpr (XB == 2) cur ^= 1;
    }
  }
  if (tile == nfull && nfull * 16 < p.P) {
    const int row0 = nfull * 16, nval = p.P - row0;
    FragTile<ACT, 4> zc;
    frag_load(zc, p.z, (size_t)row0, nval, 128, lane);
    const float2 zt = ZS ? p.stats[row0 + (r16 < nval ? r16 : 0)] : make_float2(0.f, 1.f);
    x_transpose<ACT>(Xs[wave][0], p.X, p.P, row0, nval, lane);
    run_tile(std::false_type{}, zc, zt, Xs[wave][0], row0, nval, []() {}, []() {});
  }
}

template <int ACT>
static void launch_project(lf_context* ctx, const TriProjectParams& pp, bool resident, int kz) {
  const int P = pp.P;
  if (resident && pp.C == 128 && pp.H == 128) {
    const int tiles = (P + 15) / 16;
    dim3 g(std::max(1, std::min(ctx->num_cus, (tiles + TRI_P_NWV - 1) / TRI_P_NWV)));
    const bool whole = pp.kmajor_out ? pp.N % 16 == 0 : P % 16 == 0;
    if (whole && P < (1 << 27) && pp.stats)   // 32-bit per-lane store offsets
      hipLaunchKernelGGL((tri_project_v3_kernel<ACT, TRI_P_NWV, true>), g, dim3(64 * TRI_P_NWV), 0, ctx->stream, pp);
    else if (whole && P < (1 << 27))
      hipLaunchKernelGGL((tri_project_v3_kernel<ACT, TRI_P_NWV, false>), g, dim3(64 * TRI_P_NWV), 0, ctx->stream, pp);
    else
      hipLaunchKernelGGL((tri_project_v2_kernel<ACT, TRI_P_NWV, TRI_P_TPW>), g, dim3(64 * TRI_P_NWV), 0, ctx->stream, pp);
    return;
  }
  if (resident) {
    const int tiles = (P + 15) / 16;
    dim3 g(std::max(1, std::min(ctx->num_cus, (tiles + PR_WAVES - 1) / PR_WAVES)));
    hipLaunchKernelGGL(tri_project_resident_kernel<ACT>, g, dim3(512), 0, ctx->stream, pp);
    return;
  }
  dim3 grid((P + PJ_ROWS - 1) / PJ_ROWS);
  if (kz == 64) hipLaunchKernelGGL((tri_project_kernel<ACT, 64>), grid, dim3(256), 0, ctx->stream, pp);
  else if (kz == 128) hipLaunchKernelGGL((tri_project_kernel<ACT, 128>), grid, dim3(256), 0, ctx->stream, pp);
  else hipLaunchKernelGGL((tri_project_kernel<ACT, 256>), grid, dim3(256), 0, ctx->stream, pp);
}

template <int ACT>
static void launch_output(lf_context* ctx, const TriOutputParams& op, bool resident, int kz, int kh) {
  const int P = op.P;
  if (resident && op.C == 128 && op.H == 128) {
    constexpr int NWV = tri_o_nwv<ACT>();
    const int tiles = (P + 15) / 16;
    dim3 g(std::max(1, std::min(ctx->num_cus, (tiles + NWV - 1) / NWV)));
    // the z statistics come from the project kernel when it stored them (op.stats)
    if ((P & 7) == 0 && op.stats)
      hipLaunchKernelGGL((tri_output_v3_kernel<ACT, NWV, true, true>), g, dim3(64 * NWV), 0, ctx->stream, op);
    else if ((P & 7) == 0)
      hipLaunchKernelGGL((tri_output_v3_kernel<ACT, NWV, true, false>), g, dim3(64 * NWV), 0, ctx->stream, op);
    else if (op.stats)
      hipLaunchKernelGGL((tri_output_v3_kernel<ACT, NWV, false, true>), g, dim3(64 * NWV), 0, ctx->stream, op);
    else
      hipLaunchKernelGGL((tri_output_v3_kernel<ACT, NWV, false, false>), g, dim3(64 * NWV), 0, ctx->stream, op);
    return;
  }
  if (resident) {
    const int tiles = (P + 15) / 16;
    dim3 g(std::max(1, std::min(ctx->num_cus, (tiles + OR_WAVES - 1) / OR_WAVES)));
    hipLaunchKernelGGL(tri_output_resident_kernel<ACT>, g, dim3(512), 0, ctx->stream, op);
    return;
  }
  dim3 grid((P + OT_ROWS - 1) / OT_ROWS);
#define LF_TO(KZ_, KH_) \
  if (kz == KZ_ && kh == KH_) hipLaunchKernelGGL((tri_output_kernel<ACT, KZ_, KH_>), grid, dim3(256), 0, ctx->stream, op)
  LF_TO(64, 64);
  else LF_TO(64, 128);
  else LF_TO(64, 256);
  else LF_TO(128, 64);
  else LF_TO(128, 128);
  else LF_TO(128, 256);
  else LF_TO(256, 64);
  else LF_TO(256, 128);
  else LF_TO(256, 256);
#undef LF_TO
}

static int kpad_of(int c) { return c <= 64 ? 64 : (c <= 128 ? 128 : 256); }

// One triangle multiplicative update.  Its scratch (a, b, X planes and the expanded weights)
// comes from the context workspace, or, when `scratch` is not NULL, from that device buffer of
// `scratch_cap` bytes, in which case nothing is allocated.
static int tri_mult_impl(lf_context* ctx, const lf_tri_mult_args& a, void* scratch, size_t scratch_cap) {
  LF_REQUIRE(a.w != nullptr, "tri_mult: weights are NULL");
  LF_REQUIRE(a.length > 0 && a.c_z > 0 && a.c_hidden > 0, "tri_mult: length, c_z and c_hidden must be positive");
  LF_REQUIRE(a.c_z <= 256 && a.c_hidden <= 256, "tri_mult: c_z and c_hidden must be <= 256");
  LF_REQUIRE(a.direction == LF_OUTGOING || a.direction == LF_INCOMING, "tri_mult: direction must be outgoing or incoming");
  LF_REQUIRE(a.dialect == LF_AF2 || a.dialect == LF_AF3, "tri_mult: dialect must be LF_AF2 or LF_AF3");
  LF_REQUIRE(act_dtype_ok(a.act_dtype), "tri_mult: act_dtype must be f32, f16 or bf16");
  LF_REQUIRE(a.z && a.mask && a.out, "tri_mult: z, mask and out must be device pointers");
  LF_REQUIRE(a.epsilon > 0.f && std::isfinite(a.epsilon), "tri_mult: epsilon must be finite and positive");
  const lf_tri_mult_weights& w = *a.w;
  const int N = a.length, C = a.c_z, H = a.c_hidden;
  LF_REQUIRE((long long)N * N * std::max(C, H) < (1LL << 40), "tri_mult: tensor too large");
  const int P = N * N;

  TriProjectParams pp{};
  WView views[6];  // a-proj, a-gate, b-proj, b-gate, output, gate
  pp.z = a.z;
  pp.mask = a.mask;
  pp.ln_s = w.ln_in_scale;
  pp.ln_o = w.ln_in_offset;
  pp.eps = a.epsilon;
  pp.P = P;
  pp.N = N;
  pp.C = C;
  pp.H = H;
  TriOutputParams op{};
  if (a.dialect == LF_AF2) {
    LF_REQUIRE(w.ln_in_scale && w.ln_in_offset && w.ln_out_scale && w.ln_out_offset,
               "tri_mult: AF2 layer norms need scale and offset");
    LF_TRY(make_view(w.ap, C, H, "linearAPWeight", &views[0]));
    LF_TRY(make_view(w.ag, C, H, "linearAGWeight", &views[1]));
    LF_TRY(make_view(w.bp, C, H, "linearBPWeight", &views[2]));
    LF_TRY(make_view(w.bg, C, H, "linearBGWeight", &views[3]));
    pp.bp[0] = w.ap_bias;
    pp.bg[0] = w.ag_bias;
    pp.bp[1] = w.bp_bias;
    pp.bg[1] = w.bg_bias;
    pp.fast_var = 0;
  } else {
    LF_REQUIRE(H == C, "tri_mult: AF3 dialect needs c_hidden == c_z");
    LF_TRY(make_view(w.ap, C, C, "projection(a)", &views[0], 0, 2));
    LF_TRY(make_view(w.ag, C, C, "gate(a)", &views[1], 0, 2));
    LF_TRY(make_view(w.ap, C, C, "projection(b)", &views[2], 1, 2));
    LF_TRY(make_view(w.ag, C, C, "gate(b)", &views[3], 1, 2));
    pp.fast_var = 1;
  }
  LF_TRY(make_view(w.wz, H, C, "linearZWeight", &views[4]));
  LF_TRY(make_view(w.wg, C, C, "linearGWeight", &views[5]));

  // the 128-wide project kernel for whole 16-pair tiles (32-bit per-lane store offsets) also
  // stores each pair's LN_in statistics for the output kernel, for 16-bit activations; with
  // f32 activations the hand-over measured neutral (output kernel -3%, project kernel +3%:
  // its f32 tiles leave less room to hide the extra store), so f32 recomputes them
  const bool wide = C == 128 && H == 128 && N >= 16;
  const bool v3 = wide && a.act_dtype != LF_F32 && (a.direction != LF_OUTGOING ? N % 16 == 0 : P % 16 == 0) &&
                  P < (1 << 27);
  const size_t plane = (size_t)H * P * sizeof(_Float16);
  size_t sizes[4] = {plane, plane, plane, v3 ? (size_t)P * sizeof(float2) : 0};
  void* bufs[4] = {};
  const int nbufs = v3 ? 4 : 3;
  if (scratch) {
    size_t total = 0;
    for (int i = 0; i < nbufs; ++i) {
      bufs[i] = static_cast<char*>(scratch) + total;
      total += (sizes[i] + 255) & ~size_t(255);
    }
    if (total > scratch_cap)
      return set_error(LF_ERR_INVALID, "tri_mult_noalloc: N=" + std::to_string(N) + ", c_hidden=" +
                                           std::to_string(H) + " needs " + std::to_string(total) +
                                           " bytes of scratch; the static scratch holds " +
                                           std::to_string(scratch_cap));
  } else {
    LF_TRY(workspace(ctx, sizes, bufs, nbufs));
  }
  pp.stats = static_cast<float2*>(bufs[3]);
  pp.out[0] = static_cast<_Float16*>(bufs[0]);
  pp.out[1] = static_cast<_Float16*>(bufs[1]);
  _Float16* X = static_cast<_Float16*>(bufs[2]);
  WSrc ex[6];
  // the 128-wide project kernel takes its gate weights pre-multiplied by -log2(e)
  const bool v2 = C == 128 && H == 128 && N >= 16;
  // incoming: the 128-wide project kernel stores a and b transposed per channel
  pp.kmajor_out = v2 && a.direction != LF_OUTGOING;
  const float gate = v2 ? TRI_NLOG2E : 1.f;
  for (int i = 0; i < 6; ++i) ex[i] = wsrc(views[i], i % 2 ? gate : 1.f);
  pp.wp[0] = ex[0];
  pp.wg[0] = ex[1];
  pp.wp[1] = ex[2];
  pp.wg[1] = ex[3];
  op.wz = ex[4];
  op.wg = ex[5];

  const int kz = kpad_of(C), kh = kpad_of(H);
  const bool resident = C <= 128 && H <= 128 && N >= 16;
  if (a.dialect == LF_AF3 && resident) {
    // the resident kernels stage each interleaved tensor whole and split its columns in LDS
    WView full[2];
    LF_TRY(make_view(w.ap, C, 2 * C, "projection", &full[0]));
    LF_TRY(make_view(w.ag, C, 2 * C, "gate", &full[1]));
    pp.split = 1;
    pp.wp[0] = wsrc(full[0]);
    pp.wg[0] = wsrc(full[1], gate);
  }
  {
    LaunchScope ls(ctx, a.direction == LF_OUTGOING ? "tri_out.project" : "tri_in.project");
    if (a.act_dtype == LF_F32) launch_project<DT_F32>(ctx, pp, resident, kz);
    else if (a.act_dtype == LF_F16) launch_project<DT_F16>(ctx, pp, resident, kz);
    else launch_project<DT_BF16>(ctx, pp, resident, kz);
  }
  LF_TRY(check_hip(hipGetLastError(), "tri_project launch"));

  // s = 2^-ceil(log2(N)/2) keeps |X| ~ sqrt(N)*|a||b| well inside f16's range.
  const int sexp = (int)std::ceil(std::log2((double)std::max(N, 2)) / 2.0);
  const float scale = std::ldexp(1.0f, -sexp);
  TriContractParams cp{};
  cp.N = N;
  cp.scale = scale;
  cp.X = X;
  const bool outgoing = a.direction == LF_OUTGOING;
  cp.L = outgoing ? pp.out[0] : pp.out[1];
  cp.R = outgoing ? pp.out[1] : pp.out[0];
  {
    LaunchScope ls(ctx, outgoing ? "tri_out.contract" : "tri_in.contract");
    launch_contract<128, 64, 3>(ctx, cp, H, !(outgoing || pp.kmajor_out));
  }
  LF_TRY(check_hip(hipGetLastError(), "tri_contract launch"));

  // X_math = X_stored * c with c = (rf3 ? 1/N : 1) / s; LN(X_math) = LN_{eps/c^2}(X_stored).
  const double c = (a.dialect == LF_AF3 && a.divide_by_length ? 1.0 / N : 1.0) / scale;
  op.X = X;
  op.z = a.z;
  op.out = a.out;
  op.accumulate = a.accumulate;
  op.ln_in_s = w.ln_in_scale;
  op.ln_in_o = w.ln_in_offset;
  op.ln_out_s = w.ln_out_scale;
  op.ln_out_o = w.ln_out_offset;
  op.eps = a.epsilon;
  op.eps_x = (float)(a.epsilon / (c * c));
  op.fast_var = pp.fast_var;
  op.P = P;
  op.C = C;
  op.H = H;
  op.bz = a.dialect == LF_AF2 ? w.wz_bias : nullptr;
  op.bg = a.dialect == LF_AF2 ? w.wg_bias : nullptr;
  op.stats = pp.stats;
  {
    LaunchScope ls(ctx, outgoing ? "tri_out.output" : "tri_in.output");
    if (a.act_dtype == LF_F32) launch_output<DT_F32>(ctx, op, resident, kz, kh);
    else if (a.act_dtype == LF_F16) launch_output<DT_F16>(ctx, op, resident, kz, kh);
    else launch_output<DT_BF16>(ctx, op, resident, kz, kh);
  }
  return check_hip(hipGetLastError(), "tri_output launch");
}

int tri_mult(lf_context* ctx, const lf_tri_mult_args& a) { return tri_mult_impl(ctx, a, nullptr, 0); }

// ---- the allocation-free entry point ---------------------------------------------------
// A file-scope device array serves as the scratch of lf_tri_mult_noalloc.  Each device holds
// its own copy at its own address, looked up once per device (with that device current) by
// tri_noalloc_init, which lf_context_create calls; host code only ever passes that address,
// never the array's name, which on the host is a stand-in and not a device address.
static __device__ __align__(256) unsigned char scratch[LF_TRI_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int tri_noalloc_init(int device) {
  if (device < 0 || device >= kMaxDevices) return set_error(LF_ERR_INVALID, "tri_noalloc_init: device out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return LF_OK;
  void* p = nullptr;
  LF_TRY(check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
  if (!p) return set_error(LF_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned NULL");
  g_scratch_ptr[device] = p;
  return LF_OK;
}

int tri_mult_noalloc(lf_context* ctx, const lf_tri_mult_args& a) {
  LF_TRY(tri_noalloc_init(ctx->device));   // a lookup only on the first call on this device
  void* p;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[ctx->device];
  }
  return tri_mult_impl(ctx, a, p, LF_TRI_NOALLOC_SCRATCH_BYTES);
}

}  // namespace lf
