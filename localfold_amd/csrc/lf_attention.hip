// Gated self-attention with an optional pair bias: AF2 MSA row / column attention and
// triangle attention (starting / ending node), AF3 grid and single attention.
//
// Semantics (webgpu/kernels/attention.js): x = LN(row) with logical row (b, q) read at storage
// row (q, b) when transposed (:163-168); q = x Wq / sqrt(d) (+ q bias), k = x Wk, v = x Wv,
// g = sigmoid(x Wg + bg) (:482-507); logit = q.k + 1e9 (m_k - 1) + bias[h][q][k], clamped to
// +-1e8 (:917-921); o = softmax(logit) v * g; update = o Wo + bo, stored back transposed.
// Pair bias (:695-783): bias[h][i][j] = LN(z_ij) . W[:, h], from a separate pair tensor or
// from the normalised attention input itself.
//
// Kernels:
//   lnproj  LN + the q/k/v/g (+ bias) projections in one pass over the rows
//           (q, k: [b][h][n][32] f16; v: [b][h][32][n] f16 (transposed for P.V); g: [h][rows][d], head-major)
//   keybias kb[b][k] = 1e9 (mask - 1)
//   flash   per (b, h, 128 queries): S^T = K Q^T on MFMA, online softmax with each lane
//           owning one query (statistics: two cross-lane shuffles), O^T += V^T P^T on MFMA;
//           the N^2 x heads logits never leave registers
//   rowgemm o Wo + bo, + residual, stored through the row map
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <cmath>

#include "lf_rowgemm.h"

namespace lf {

constexpr int FA_DP = 32;       // padded head dim (d <= 32); 16 for d <= 16 (the kernel's DP)
constexpr int FA_QPB = 128;     // queries per block (8 / QT waves of QT 16-query tiles)
// 16-query tiles per wave, with and without a pair bias: one (two measured 60% slower for
// triangle attention at N = 512: 155 VGPRs, half the waves)
constexpr int FA_QT_BIAS = 1, FA_QT_PLAIN = 1;
constexpr int FA_KC = 64;       // keys per chunk
constexpr int FA_VLD = FA_KC + 8, FA_BLD = FA_KC + 8;


struct FlashParams {
  const _Float16 *q, *k, *vt, *g;
  _Float16* o;
  const float* kb;        // [B][Qp] at a row stride of kb_stride (0: one row shared by every b)
  long long kb_stride;
  const _Float16* bias;   // [H][Q][Q] or null
  int B, H, Q, d, HD;
  int dq;                 // head dims q and k hold (d; 0 when every logit is the bias alone)
  int fix;                // dq < DP or Q not a whole number of chunks: the kernel (the FIX
                          // instantiation) zeroes the unwritten parts of q, k and v^T as it
                          // reads them
  int nqb;                // query blocks per (b, h)
  long long nblocks;
};

// The softmax runs in base 2: q, the pair bias and the key-mask bias are stored pre-multiplied
// by log2(e), so p = exp2(x - max) with x = log2(e) * logit, and the +-1e8 clamp becomes
// +-1e8 * log2(e).  Mathematically identical to exp(logit - max).
constexpr float LOG2E = 1.4426950408889634f;
constexpr float FA_CLAMP = 1e8f * LOG2E;
// The running max is raised only when a chunk's scores exceed it by more than this (log2
// units): until then p = exp2(x - m) <= 2^FA_RESCALE, well inside f16 range, and the
// O rescale is skipped.
constexpr float FA_RESCALE = 8.f;

// kb[b][k] for k < Qp (keys padded to whole chunks): 1e9 log2(e) (mask - 1), and -1e30 past Q
__global__ __launch_bounds__(256) void keybias_kernel(const float* mask, float* kb, int B, int Q, int Qp,
                                                      int transpose) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)B * Qp) return;
  const int b = (int)(i / Qp), k = (int)(i % Qp);
  if (k >= Q) {
    kb[i] = -1e30f;
    return;
  }
  const float m = mask[transpose ? (long long)k * B + b : (long long)b * Q + k];
  kb[i] = (1e9f * LOG2E) * (m - 1.0f);
}

// One key-bias row shared by every batch row, from the mask's maximum over the batch
// (AF3 pair-weighted averaging: a token any sequence covers is a key for every sequence).
// A block covers 64 keys with 16 rows of 64 lanes; each lane strides the batch by 16.
__global__ __launch_bounds__(1024) void keymax_kernel(const float* mask, float* kb, int B, int Q, int Qp) {
  __shared__ float part[16][64];
  const int lane = threadIdx.x & 63, r = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + lane;
  float m = 0.f;
  if (k < Q) {
#pragma unroll 8
    for (int b = r; b < B; b += 16) m = fmaxf(m, mask[(long long)b * Q + k]);
  }
  part[r][lane] = m;
  __syncthreads();
  if (r == 0 && k < Qp) {
#pragma unroll
    for (int i = 1; i < 16; ++i) m = fmaxf(m, part[i][lane]);
    kb[k] = k < Q ? (1e9f * LOG2E) * (m - 1.0f) : -1e30f;
  }
}

// Pair-weighted averaging, step 1: P[h][i][j] = softmax_j(bias[h][i][j] + kb[j]) in base 2,
// written as f16 over the bias rows (row stride Qp), keys past Q zero.  One wave per row.
// Every key masked: the 1e9 term swamps the logits in f32 and the row is uniform over the
// Q keys, as in the reference's f32 softmax.
__global__ __launch_bounds__(256) void pwa_softmax_kernel(_Float16* bias, const float* kb, int rows, int Q, int Qp) {
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  _Float16* r = bias + row * Qp;
  float m = -3.0e38f;
  for (int j = lane; j < Q; j += 64) m = fmaxf(m, (float)r[j] + kb[j]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  float t = 0.f;
  for (int j = lane; j < Q; j += 64) t += exp2f((float)r[j] + kb[j] - m);
  t = wave_sum(t);
  const float inv = 1.f / t;
  for (int j = lane; j < Qp; j += 64) r[j] = (_Float16)(j < Q ? exp2f((float)r[j] + kb[j] - m) * inv : 0.f);
}

// Pair-weighted averaging, step 2, per head h an NT GEMM on the matrix cores:
//   O^T[n][i] = sum_j Vt[n][j] P[i][j],  n = (s, e) over sequences s and head dims e < d,
// gated and stored as o[(s Q + i)][h d + e] = O * g.  Vt rows: vt + ((s H + h) d + e) Qp; the
// gate is head-major, g[h][s][i][e], so a block's gate reads are whole lines.
// Block: 4 waves in 2 x 2, a 128 (n) x 128 (i) tile; a wave holds 4 x 4 16x16 accumulators and
// reads its fragments straight from L2 (P of one head is shared by every block of that head).
// A lane's 4 accumulator rows are 4 consecutive n, i.e. 4 consecutive head dims of one
// sequence (d % 4 == 0), stored as one 8-byte word.
constexpr int PWA_T = 128;
struct PwaParams {
  const _Float16 *vt, *p, *g;
  _Float16* o;
  int S, H, Q, Qp, d, HD;
  int ntn, nti;             // tiles along n and i per head
  long long nblocks;
};

constexpr int PWA_KC = 64, PWA_LD = 72;   // k chunk; LDS row pitch in halves (144 B: 16-byte aligned, spread banks)

__global__ __launch_bounds__(256) void pwa_average_kernel(PwaParams p) {
  __shared__ __attribute__((aligned(16))) _Float16 As[2][PWA_T * PWA_LD];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][PWA_T * PWA_LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  // XCD-aware order: each XCD walks a contiguous range, i tiles fastest, so the blocks that
  // share one n tile of V (and one head of P) run on one L2
  long long lb = blockIdx.x;
  const long long per = p.nblocks / 8;
  if (lb < per * 8) lb = (lb % 8) * per + lb / 8;
  const int ti = (int)(lb % p.nti);
  const int tn = (int)((lb / p.nti) % p.ntn);
  const int h = (int)(lb / ((long long)p.nti * p.ntn));
  const int N = p.S * p.d;
  const int nb0 = tn * PWA_T, ib0 = ti * PWA_T;
  const int wn = (wave & 1) * 64, wi = (wave >> 1) * 64;
  const int n0 = nb0 + wn, i0 = ib0 + wi;

  // staging: thread t copies 32 halves (four 16-byte loads) of row t / 2 of each operand tile
  const int srow = tid >> 1, shalf = (tid & 1) * 32;
  const _Float16* ga;
  const _Float16* gb;
  {
    const int n = min(nb0 + srow, N - 1);
    const int s = n / p.d, e = n - s * p.d;
    ga = p.vt + ((long long)(s * p.H + h) * p.d + e) * p.Qp + shalf;
    const int i = min(ib0 + srow, p.Q - 1);
    gb = p.p + ((long long)h * p.Q + i) * p.Qp + shalf;
  }
  f4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
  h8 ra[4], rb[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    ra[u] = *(const h8*)(ga + 8 * u);
    rb[u] = *(const h8*)(gb + 8 * u);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    *(h8*)&As[0][srow * PWA_LD + shalf + 8 * u] = ra[u];
    *(h8*)&Bs[0][srow * PWA_LD + shalf + 8 * u] = rb[u];
  }
  __syncthreads();
  const int nkc = p.Qp / PWA_KC;
  for (int kc = 0; kc < nkc; ++kc) {
    const int buf = kc & 1;
    const bool more = kc + 1 < nkc;
    if (more) {
      const int k1 = (kc + 1) * PWA_KC;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        ra[u] = *(const h8*)(ga + k1 + 8 * u);
        rb[u] = *(const h8*)(gb + k1 + 8 * u);
      }
    }
#pragma unroll
    for (int kk = 0; kk < PWA_KC; kk += 32) {
      h8 fa[4], fb[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        fa[t] = *(const h8*)&As[buf][(wn + t * 16 + r16) * PWA_LD + kk + g4 * 8];
        fb[t] = *(const h8*)&Bs[buf][(wi + t * 16 + r16) * PWA_LD + kk + g4 * 8];
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma16(fa[a], fb[b], acc[a][b]);
    }
    if (more) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        *(h8*)&As[buf ^ 1][srow * PWA_LD + shalf + 8 * u] = ra[u];
        *(h8*)&Bs[buf ^ 1][srow * PWA_LD + shalf + 8 * u] = rb[u];
      }
    }
    __syncthreads();
  }
  // epilogue: gate values first (loads ahead of every store), then the gated stores
  h4 gv[4][4];
  long long oi[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int n = min(n0 + a * 16 + g4 * 4, N - 4);
    const int s = n / p.d, e = n - s * p.d;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int i = min(i0 + b * 16 + r16, p.Q - 1);
      oi[a][b] = ((long long)s * p.Q + i) * p.HD + h * p.d + e;
      gv[a][b] = *(const h4*)(p.g + (((long long)h * p.S + s) * p.Q + i) * p.d + e);
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const bool nok = n0 + a * 16 + g4 * 4 < N;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (!nok || i0 + b * 16 + r16 >= p.Q) continue;
      h4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = (_Float16)(acc[a][b][j] * (float)gv[a][b][j]);
      *(h4*)(p.o + oi[a][b]) = v;
    }
  }
}

// S^T tile += K Q^T over the padded head dims: 16x16x32 for 8 dims a lane, 16x16x16 for 4
__device__ __forceinline__ f4 qk_mfma(h8 k, h8 q, f4 c) { return mfma16(k, q, c); }
__device__ __forceinline__ f4 qk_mfma(h4 k, h4 q, f4 c) { return mfma16k16(k, q, c); }

// (float)v[i] + c in one instruction (i is a constant once the caller's loop is unrolled)
__device__ __forceinline__ float bias_add(const h4& v, int i, float c) {
  const uint2 u = __builtin_bit_cast(uint2, v);
  const uint32_t w = i < 2 ? u.x : u.y;
  return (i & 1) ? f16_add<1>(w, c) : f16_add<0>(w, c);
}

// (With one query tile per wave the kernel stages the block's bias tile through LDS instead;
// this per-lane fetch serves QT > 1.)  Pair-bias values of one lane for one key chunk: the 16 keys k0 + 16*g4 .. +15 of each of the
// lane's queries (rows brow[qt], already offset by 16*g4), as two aligned 16-byte loads;
// bv[qt][kt][i] is key k0 + 16*g4 + 4*kt + i.  Bias rows are padded to whole chunks; values
// past Q are never used.
template <int QT>
__device__ __forceinline__ void bias_fetch(const _Float16* const (&brow)[QT], int k0, h4 (&bv)[QT][4]) {
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const h8 lo = *reinterpret_cast<const h8*>(brow[qt] + k0);
    const h8 hi = *reinterpret_cast<const h8*>(brow[qt] + k0 + 8);
    bv[qt][0] = h4{lo[0], lo[1], lo[2], lo[3]};
    bv[qt][1] = h4{lo[4], lo[5], lo[6], lo[7]};
    bv[qt][2] = h4{hi[0], hi[1], hi[2], hi[3]};
    bv[qt][3] = h4{hi[4], hi[5], hi[6], hi[7]};
  }
}

// One block: 128 queries of one (batch row, head); each wave owns QT 16-query tiles.  Key
// chunks of 64 are staged in double-buffered LDS two chunks ahead (K rows, V^T rows, key
// bias); the pair-bias values a lane needs come straight from global memory, also ahead.
//
// Online softmax with a lazy running max: the S accumulators start at bias - m (m = the
// query's running max, 0 before the first chunk), so the MFMA yields x - m directly; when no
// query's maximum rose by more than FA_RESCALE (a wave-uniform vote; in the first chunk, or
// lies more than FA_RESCALE below 0) p = exp2(x - m) needs no subtraction and O no rescale:
// the standard update with a stale max m, which only scales numerator and denominator alike.
// Otherwise m moves to the new maximum (O rescaled).  Chunks holding masked or past-the-end
// keys take the general update (explicit key bias, clamp, max).  The row sums come from the
// PV MFMAs themselves, through an all-ones operand (third d tile).
//
// Key order within a chunk: row 4*g + i of S^T tile kt is key 16*g + 4*kt + i (K rows are
// stored to LDS in that order), so the 16 scores a lane holds per query are the contiguous
// keys 16*(lane/16) .. +15: its bias, key bias and V^T pieces are single vector loads.
template <bool BIAS, int QT, bool BL = BIAS && QT == 1, int DP = FA_DP, bool FIX = false>
__global__ __launch_bounds__(64 * (8 / QT)) void flash_kernel(FlashParams p) {
  static_assert(!BL || (BIAS && QT == 1), "the LDS-staged bias is for one query tile per wave");
  static_assert(DP == 16 || DP == 32, "padded head dim 16 or 32");
  // DP = 16 (d <= 16): QK^T on 16x16x16 MFMAs (4 head dims a lane), one O tile; DP = 32: QK^T
  // on 16x16x32 MFMAs (8 a lane), two O tiles.  o[NDT] holds the row sums.
  constexpr int KLD = DP + 8, NDT = DP / 16, SEGS = DP / 8;
  using QF = typename std::conditional<DP == 32, h8, h4>::type;
  // (BL, the default with a bias: MSA row attention at 512 x 384 0.30 -> 0.276 ms and triangle
  // attention at N = 384 0.106 -> 0.098 ms per launch, N = 512 -1%, N = 1024 unchanged)
  // per buffer: K rows [64][KLD], then V^T rows [DP][FA_VLD]
  __shared__ __attribute__((aligned(16))) _Float16 KV[2][FA_KC * KLD + DP * FA_VLD];
  // BL: the block's pair-bias tile of each chunk, [128 queries][64 keys] at pitch FA_BLD
  __shared__ __attribute__((aligned(16))) _Float16 Bl[BL ? 2 : 1][BL ? FA_QPB * FA_BLD : 8];
  __shared__ __attribute__((aligned(16))) float Kb[2][FA_KC];
  __shared__ int Kmasked[2];   // chunk has a masked key or a key past Q
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4, kq = g4 * 8;

  // XCD-aware order: the hardware deals consecutive blocks to the 8 XCDs round-robin; remap
  // so each XCD walks a contiguous range of (query block, batch row) for one head, keeping
  // that head's pair bias and each row's K/V in its own L2.
  long long lb = blockIdx.x;
  const long long per = p.nblocks / 8;
  if (lb < per * 8) lb = (lb % 8) * per + lb / 8;
  const int qb = (int)(lb % p.nqb);
  const int b = (int)((lb / p.nqb) % p.B);
  const int h = (int)(lb / ((long long)p.nqb * p.B));

  const int nkc = (p.Q + FA_KC - 1) / FA_KC;
  const int Qp = nkc * FA_KC;   // keys padded to whole chunks in q, k, v^T, the key bias and bias rows
  const size_t bh = (size_t)b * p.H + h;
  const _Float16* qh = p.q + bh * Qp * DP;
  const _Float16* kh = p.k + bh * Qp * DP;
  const _Float16* vh = p.vt + bh * DP * Qp;
  const float* kbb = p.kb + b * p.kb_stride;
  const _Float16* bias = BIAS ? p.bias + (size_t)h * p.Q * Qp : nullptr;

  // Q fragments (B operand of S^T = K Q^T): query r16 of tile qt, dims qd .. +8 (DP 32) or
  // +4 (DP 16); dims past dq are zeroed here (the buffer's padding is never written)
  const int qd = DP == 32 ? kq : 4 * g4;
  int qidx[QT], qc[QT];
  QF qf[QT];
  const _Float16* brow[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    qidx[qt] = qb * FA_QPB + (wave * QT + qt) * 16 + r16;
    qc[qt] = qidx[qt] < p.Q ? qidx[qt] : p.Q - 1;
    qf[qt] = *reinterpret_cast<const QF*>(qh + (size_t)qc[qt] * DP + qd);
    if (FIX) {
#pragma unroll
      for (int e = 0; e < (int)(sizeof(QF) / 2); ++e)
        if (qd + e >= p.dq) qf[qt][e] = (_Float16)0.f;
    }
    brow[qt] = BIAS ? bias + (size_t)qc[qt] * Qp + 16 * g4 : nullptr;
  }
  // the epilogue's gate (head-major [h][row][d]) is read now, so the block's last step does
  // not wait a memory round trip for it (QT == 1, d a multiple of 4)
  const bool gpre = QT == 1 && (p.d & 3) == 0;
  h4 gp0 = h4{0, 0, 0, 0}, gp1 = h4{0, 0, 0, 0};
  if (gpre) {
    const size_t grow = ((size_t)h * p.B * p.Q + (size_t)b * p.Q + qc[0]) * p.d;
    if (4 * g4 < p.d) gp0 = *reinterpret_cast<const h4*>(p.g + grow + 4 * g4);
    if (DP == 32 && 16 + 4 * g4 < p.d) gp1 = *reinterpret_cast<const h4*>(p.g + grow + 16 + 4 * g4);
  }
  const h8 ones = h8{1, 1, 1, 1, 1, 1, 1, 1};
  // identity A operand of a 16x16x16 MFMA: lane supplies I[r16][4*g4 + j]
  const h4 ident = h4{(_Float16)(r16 == 4 * g4), (_Float16)(r16 == 4 * g4 + 1), (_Float16)(r16 == 4 * g4 + 2),
                      (_Float16)(r16 == 4 * g4 + 3)};

  // Staging: a chunk is 16 DP 16-byte pieces: piece t < 8 DP is K row t / SEGS (dims
  // 8 (t % SEGS) .. +8), piece t >= 8 DP V^T row (t - 8 DP) / 8 (keys 8 ((t - 8 DP) % 8) .. +8).
  // Each thread stages NP pieces (DP 16 with 512 threads: threads t and t + 256 load and store
  // the same piece, so every load and store stays unconditional) and lane l of every wave
  // loads key bias l (wave 0 stores it).  With whole padded chunks every load is
  // unconditional, so no branch separates a load from its use and the prefetched chunks stay
  // in flight until they are needed.
  constexpr int NT = 64 * (8 / QT), NPC = 16 * DP, NP = NPC > NT ? NPC / NT : 1;
  const _Float16* gsrc[NP];
  int gstep[NP], loff[NP];   // source advance per chunk and LDS offset (elements)
  // FIX: the piece's first key within a chunk and, for K, how many of its 8 dims are < dq
  // (V^T dims past d only reach output dims that are never stored)
  int pkey[NP], pdims[NP];
  bool pisk[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int t = (tid + j * NT) % NPC, tv = t - 8 * DP;
    const bool isk = t < 8 * DP;   // wave-uniform
    const int key = t / SEGS, seg = t % SEGS;
    gsrc[j] = isk ? kh + (size_t)key * DP + seg * 8 : vh + (size_t)(tv >> 3) * Qp + (tv & 7) * 8;
    gstep[j] = isk ? FA_KC * DP : FA_KC;
    const int krow = 16 * ((key >> 2) & 3) + 4 * (key >> 4) + (key & 3);
    loff[j] = isk ? krow * KLD + seg * 8 : FA_KC * KLD + (tv >> 3) * FA_VLD + (tv & 7) * 8;
    pisk[j] = isk;
    pkey[j] = isk ? key : (tv & 7) * 8;
    pdims[j] = isk ? min(max(p.dq - seg * 8, 0), 8) : 8;
  }
  // BL: thread t stages bias rows t/8 and t/8 + 64 of the block's 128, keys 8 (t % 8) .. +8,
  // so eight consecutive threads read one row's 128 bytes (coalesced, unlike the per-lane
  // fetch, where one wave instruction touched 64 rows)
  const _Float16* bsrc[2];
  int boff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = (tid >> 3) + 64 * j, q = qb * FA_QPB + r;
    bsrc[j] = BL ? bias + (size_t)(q < p.Q ? q : p.Q - 1) * Qp + (tid & 7) * 8 : nullptr;
    boff[j] = r * FA_BLD + (tid & 7) * 8;
  }
  // (the bias tile of chunk c + 1 is loaded at the top of chunk c, before chunk c + 2's K/V, and
  // stored with chunk c + 1's K/V at its end: one chunk of latency, L2 hits)
  // (two named registers, not an array: an array passed by reference here was promoted to LDS)
  uint4 bsn0, bsn1;
  auto bias_load = [&](int c) __attribute__((always_inline)) {
    bsn0 = *reinterpret_cast<const uint4*>(bsrc[0] + c * FA_KC);
    bsn1 = *reinterpret_cast<const uint4*>(bsrc[1] + c * FA_KC);
  };
  auto bias_store = [&](int buf) __attribute__((always_inline)) {
    *reinterpret_cast<uint4*>(&Bl[buf][boff[0]]) = bsn0;
    *reinterpret_cast<uint4*>(&Bl[buf][boff[1]]) = bsn1;
  };
  auto kv_load = [&](int c, uint4 (&r)[NP], float& kbr) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NP; ++j) r[j] = *reinterpret_cast<const uint4*>(gsrc[j] + (size_t)c * gstep[j]);
    kbr = kbb[c * FA_KC + lane];
  };
  // zeroes what q, k and v^T leave unwritten (head dims past dq in K, keys past Q in K and V^T)
  // in the registers of chunk c before they are stored: no padding of those buffers is ever
  // cleared in memory
  auto kv_fix = [&](int c, uint4 (&r)[NP]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int key0 = c * FA_KC + pkey[j];
      const int n = pisk[j] ? (key0 < p.Q ? pdims[j] : 0) : min(max(p.Q - key0, 0), 8);
      uint32_t m[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) m[w] = (2 * w < n ? 0xffffu : 0u) | (2 * w + 1 < n ? 0xffff0000u : 0u);
      r[j].x &= m[0];
      r[j].y &= m[1];
      r[j].z &= m[2];
      r[j].w &= m[3];
    }
  };
  auto kv_store = [&](int buf, uint4 (&r)[NP], float kbr, int c) __attribute__((always_inline)) {
    if constexpr (FIX) kv_fix(c, r);
#pragma unroll
    for (int j = 0; j < NP; ++j) *reinterpret_cast<uint4*>(&KV[buf][loff[j]]) = r[j];
    if (wave == 0) {
      Kb[buf][lane] = kbr;
      const bool any = __any(kbr != 0.f);
      if (lane == 0) Kmasked[buf] = any ? 1 : 0;
    }
  };

  // loads run two chunks ahead (register set c % 2; past the last chunk the last one is
  // loaded again and never stored); chunk c + 1 is written to LDS at the end of chunk c, into
  // the buffer chunk c - 1 used (every wave passed that chunk's barrier)
  uint4 st0[NP], st1[NP];
  float kb0, kb1;
  h4 bq0[QT][4], bq1[QT][4];   // bias of chunk c in set c % 2; chunk c + 2's is fetched once c's is used
  const int c1 = nkc > 1 ? 1 : 0;
  if (BL) bias_load(0);
  kv_load(0, st0, kb0);
  kv_load(c1, st1, kb1);
  if (BIAS && !BL) {
    bias_fetch<QT>(brow, 0, bq0);
    bias_fetch<QT>(brow, c1 * FA_KC, bq1);
  }
  kv_store(0, st0, kb0, 0);
  if (BL) bias_store(0);
  __syncthreads();

  float m_run[QT];
  f4 o[NDT + 1][QT];   // [dt][qt]: O^T[dt*16 + 4*g4 + i][query]; dt = NDT: the row sums
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -1e30f;
#pragma unroll
    for (int dt = 0; dt <= NDT; ++dt) o[dt][qt] = f4{0.f, 0.f, 0.f, 0.f};
  }

  // one chunk; RS = c % 2 is a compile-time constant so every register-set index is static
  auto chunk = [&](int c, auto rs_tag) __attribute__((always_inline)) {
      constexpr int rs = decltype(rs_tag)::value;
      const int buf = rs;
      h4 (&bq)[QT][4] = rs == 0 ? bq0 : bq1;
      if (BL) {   // this chunk's bias from the block's LDS tile: the lane's query, keys 16 g4 .. +15
        const _Float16* br = &Bl[buf][(wave * 16 + r16) * FA_BLD + 16 * g4];
        const h8 lo = *reinterpret_cast<const h8*>(br);
        const h8 hi = *reinterpret_cast<const h8*>(br + 8);
        bq[0][0] = h4{lo[0], lo[1], lo[2], lo[3]};
        bq[0][1] = h4{lo[4], lo[5], lo[6], lo[7]};
        bq[0][2] = h4{hi[0], hi[1], hi[2], hi[3]};
        bq[0][3] = h4{hi[4], hi[5], hi[6], hi[7]};
      }
      const int cn = c + 2 < nkc ? c + 2 : nkc - 1;
      if (BL) {
        bias_load(c + 1 < nkc ? c + 1 : nkc - 1);
        __builtin_amdgcn_sched_barrier(0);   // keep the loads here, a chunk ahead of their store
      }
      if constexpr (rs == 0) kv_load(cn, st0, kb0);
      else kv_load(cn, st1, kb1);
      const bool general = Kmasked[buf] != 0;   // wave-uniform
      _Float16 pv[QT][4][4];
      if (general) {
        f4 s[QT][4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const QF kf = *reinterpret_cast<const QF*>(&KV[buf][(kt * 16 + r16) * KLD + qd]);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) s[qt][kt] = qk_mfma(kf, qf[qt], f4{0.f, 0.f, 0.f, 0.f});
        }
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          float mx = -1e30f;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) {
            const float4 kb4 = *reinterpret_cast<const float4*>(&Kb[buf][16 * g4 + 4 * kt]);
            const float kbv[4] = {kb4.x, kb4.y, kb4.z, kb4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float x = s[qt][kt][i] + kbv[i];
              if (BIAS) x = bias_add(bq[qt][kt], i, x);
              // clamp (keys past Q carry -1e30 and stay below every real logit); one v_med3
              // for the finite logits here, where fminf(fmaxf()) added a canonicalising move
              // (flash at N = 1024: -1.4%)
              x = kbv[i] < -1e29f ? -1e30f : __builtin_amdgcn_fmed3f(x, -FA_CLAMP, FA_CLAMP);
              s[qt][kt][i] = x;
              mx = fmaxf(mx, x);
            }
          }
          mx = lanes4_max(mx);
          const float m_new = fmaxf(m_run[qt], mx);
          const float corr = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) pv[qt][kt][i] = (_Float16)__builtin_amdgcn_exp2f(s[qt][kt][i] - m_new);
          m_run[qt] = m_new;
#pragma unroll
          for (int dt = 0; dt <= NDT; ++dt) o[dt][qt] = o[dt][qt] * corr;
        }
      } else {
        // S accumulators start at bias - m, so the MFMA yields x - m; the bias lands through an
        // identity MFMA (D = I B + C, B = the lane's bias h4 in the accumulator layout)
        // (a first chunk measures against m = 0 and re-bases on its own maximum below unless
        // that lies within FA_RESCALE of 0)
        f4 s[QT][4];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          if (c == 0) m_run[qt] = 0.f;
          const f4 negm = f4{-m_run[qt], -m_run[qt], -m_run[qt], -m_run[qt]};
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) s[qt][kt] = BIAS ? mfma16k16(ident, bq[qt][kt], negm) : negm;
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const QF kf = *reinterpret_cast<const QF*>(&KV[buf][(kt * 16 + r16) * KLD + qd]);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) s[qt][kt] = qk_mfma(kf, qf[qt], s[qt][kt]);
        }
        float mx[QT];
        bool rose = false;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          float v = -1e30f;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) v = fmaxf(v, s[qt][kt][i]);
          mx[qt] = v;
          rose |= v > FA_RESCALE || (c == 0 && v < -FA_RESCALE);
        }
        if (!__any(rose)) {
#pragma unroll
          for (int qt = 0; qt < QT; ++qt)
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
              for (int i = 0; i < 4; ++i) pv[qt][kt][i] = (_Float16)__builtin_amdgcn_exp2f(s[qt][kt][i]);
        } else {
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            // rise of this query's max (in a first chunk the offset from 0 either way, with
            // nothing accumulated to rescale)
            const float d = c == 0 ? lanes4_max(mx[qt]) : fmaxf(lanes4_max(mx[qt]), 0.f);
            const float corr = c == 0 ? 1.f : __builtin_amdgcn_exp2f(-d);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
              for (int i = 0; i < 4; ++i) pv[qt][kt][i] = (_Float16)__builtin_amdgcn_exp2f(s[qt][kt][i] - d);
            m_run[qt] += d;
#pragma unroll
            for (int dt = 0; dt <= NDT; ++dt) o[dt][qt] = o[dt][qt] * corr;
          }
        }
      }
      // this chunk's bias values are consumed: fetch chunk c + 2's into the slot
      if (BIAS && !BL) bias_fetch<QT>(brow, cn * FA_KC, bq);
      // O^T += V^T P^T over two 32-key halves; the ones operand accumulates the row sums
#pragma unroll
      for (int kh2 = 0; kh2 < 2; ++kh2) {
        // MFMA k index 8*g4 + j is key 16*g4 + 8*kh2 + j: one 16-byte piece of the V^T row
        h8 vf[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
          vf[dt] = *reinterpret_cast<const h8*>(&KV[buf][FA_KC * KLD + (dt * 16 + r16) * FA_VLD + 16 * g4 + 8 * kh2]);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const h8 pf = h8{pv[qt][2 * kh2][0], pv[qt][2 * kh2][1], pv[qt][2 * kh2][2], pv[qt][2 * kh2][3],
                           pv[qt][2 * kh2 + 1][0], pv[qt][2 * kh2 + 1][1], pv[qt][2 * kh2 + 1][2],
                           pv[qt][2 * kh2 + 1][3]};
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) o[dt][qt] = mfma16(vf[dt], pf, o[dt][qt]);
          o[NDT][qt] = mfma16(ones, pf, o[NDT][qt]);
        }
      }
      // unconditional (after the last chunk it stores a repeat that nothing reads): with no
      // branch around the store the compiler's waits on the loads stay exact
      if constexpr (rs == 0) kv_store(buf ^ 1, st1, kb1, c + 1 < nkc ? c + 1 : nkc - 1);
      else kv_store(buf ^ 1, st0, kb0, c + 1 < nkc ? c + 1 : nkc - 1);
      if (BL) {
        __builtin_amdgcn_sched_barrier(0);
        bias_store(buf ^ 1);
      }
      __syncthreads();
  };
  int c0 = 0;
  for (; c0 + 2 <= nkc; c0 += 2) {
    chunk(c0, std::integral_constant<int, 0>{});
    chunk(c0 + 1, std::integral_constant<int, 1>{});
  }
  if (c0 < nkc) chunk(c0, std::integral_constant<int, 0>{});
  // o[query][h*d + dd] = O / l * g
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    if (qidx[qt] >= p.Q) continue;
    const float inv = 1.0f / o[NDT][qt][0];
    const size_t row = (size_t)b * p.Q + qidx[qt];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d0 = dt * 16 + 4 * g4;
      if (d0 >= p.d) continue;
      const size_t base = row * p.HD + (size_t)h * p.d + d0;
      const size_t gbase = ((size_t)h * p.B * p.Q + row) * p.d + d0;   // gate head-major [h][row][d]
      if (d0 + 4 <= p.d && (p.d & 3) == 0) {
        const h4 gv = gpre ? (dt == 0 ? gp0 : gp1) : *reinterpret_cast<const h4*>(p.g + gbase);
        h4 ov;
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[i] = (_Float16)(o[dt][qt][i] * inv * (float)gv[i]);
        *reinterpret_cast<h4*>(p.o + base) = ov;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (d0 + i < p.d) p.o[base + i] = (_Float16)(o[dt][qt][i] * inv * (float)p.g[gbase + i]);
      }
    }
  }
}

int attention(lf_context* ctx, const lf_attention_args& a, bool no_qk, bool shared_key_mask) {
  LF_REQUIRE(a.w != nullptr, "attention: weights are NULL");
  LF_REQUIRE(a.batch > 0 && a.queries > 0 && a.channels > 0 && a.heads > 0,
             "attention dimensions must be positive");
  LF_REQUIRE(act_dtype_ok(a.act_dtype), "attention: act_dtype must be f32, f16 or bf16");
  LF_REQUIRE(a.act && a.mask && a.out, "attention: act, mask and out must be device pointers");
  LF_REQUIRE(a.channels <= 384, "attention: channels must be <= 384");
  const int B = a.batch, Q = a.queries, C = a.channels, H = a.heads;
  if (a.head_dim == 0)
    LF_REQUIRE(C % H == 0, "attention: channels must be a multiple of heads when head_dim is 0");
  const int d = a.head_dim > 0 ? a.head_dim : C / H;
  LF_REQUIRE(d >= 1 && d <= 32, "attention: head dimension must be 1..32");
  const int HD = H * d;
  LF_REQUIRE(HD <= 512, "attention: heads * head_dim must be <= 512");
  LF_REQUIRE(a.bias_mode >= LF_BIAS_NONE && a.bias_mode <= LF_BIAS_LOGITS, "attention: bad bias_mode");
  if (a.bias_mode == LF_BIAS_NORMALIZED_INPUT)
    LF_REQUIRE(B == Q, "attention: a bias from the normalised input needs batch == queries (triangle attention)");
  if (a.bias_mode == LF_BIAS_SEPARATE) {
    LF_REQUIRE(a.pair && act_dtype_ok(a.pair_dtype) && a.pair_channels > 0 && a.pair_channels <= 384,
               "attention: separate pair bias needs pair activations (<= 384 channels)");
  }
  if (a.bias_mode == LF_BIAS_LOGITS) LF_REQUIRE(a.bias_logits, "attention: bias_logits is NULL");
  LF_REQUIRE(a.epsilon > 0.f && std::isfinite(a.epsilon), "attention: epsilon must be finite and positive");
  const lf_attention_weights& w = *a.w;
  const long long rows = (long long)B * Q;
  LF_REQUIRE(rows < (1LL << 31), "attention: too many rows");

  WView views[6];
  int nv = 2;
  if (!no_qk) {
    LF_TRY(make_view(w.wq, C, HD, "queryWeight", &views[0]));
    LF_TRY(make_view(w.wk, C, HD, "keyWeight", &views[1]));
  }
  LF_TRY(make_view(w.wv, C, HD, "valueWeight", &views[nv++]));
  LF_TRY(make_view(w.wg, C, HD, "gatingWeight", &views[nv++]));
  LF_TRY(make_view(w.wo, HD, C, "outputWeight", &views[nv++]));
  const bool want_bias = a.bias_mode == LF_BIAS_SEPARATE || a.bias_mode == LF_BIAS_NORMALIZED_INPUT;
  if (want_bias)
    LF_TRY(make_view(w.wb, a.bias_mode == LF_BIAS_SEPARATE ? a.pair_channels : C, H, "pair projectionWeight",
                     &views[nv++]));

  // keys padded to whole 64-key chunks (the flash kernel loads whole chunks)
  const int Qp = (Q + FA_KC - 1) / FA_KC * FA_KC;
  // q, k and V^T padded to DP head dims: 16 when d <= 16 (the extra-MSA and MSA-module heads
  // of 8), else 32
  const int DP = d <= 16 ? 16 : FA_DP;
  const size_t qkv = (size_t)B * H * Qp * DP * sizeof(_Float16);
  const size_t hd = (size_t)rows * HD * sizeof(_Float16);
  const size_t biash = (a.bias_mode == LF_BIAS_NONE) ? 0 : (size_t)H * Q * Qp * sizeof(_Float16);
  // buffers: q, k, v, g, o, key bias, f16 pair bias, output weights, packed lnproj weights x 2
  void* bufs[10];

  // 1. pair bias from a separate pair tensor: bias[h][i][j] = LN(pair_ij) . W[:, h]
  LnProjParams pb{};
  if (a.bias_mode == LF_BIAS_SEPARATE) {
    pb.x = a.pair;
    pb.rows = Q * Q;
    pb.C = a.pair_channels;
    pb.rmQ = 1;
    pb.rmB = 0;
    pb.ln_s = w.pair_norm_scale;
    pb.ln_o = w.pair_norm_offset;
    pb.eps = a.epsilon;
    pb.fast_var = a.fast_variance;
    pb.ngroups = 1;
    Group& g = pb.g[0];
    g.w0 = views[5];
    g.ncols = H;
    g.op = OP_STORE;
    g.scale = LOG2E;
  }
  // 2. LN + q/k/v/g (+ bias from the normalised input)
  LnProjParams pp{};
  pp.x = a.act;
  pp.rows = (int)rows;
  pp.C = C;
  pp.rmQ = Q;
  pp.rmB = a.transpose ? B : 0;
  pp.ln_s = w.norm_scale;
  pp.ln_o = w.norm_offset;
  pp.eps = a.epsilon;
  pp.fast_var = a.fast_variance;
  // group slots: q, k (absent when no_qk: every logit is the bias alone), v, g, bias
  int gq = -1, gk = -1, gv, gg, gbias = -1;
  pp.ngroups = 0;
  if (!no_qk) {
    gq = pp.ngroups++;
    pp.g[gq] = Group{views[0], WView{}, HD, OP_STORE, LOG2E / std::sqrt((float)d), w.q_bias, nullptr, Dst{}};
    gk = pp.ngroups++;
    pp.g[gk] = Group{views[1], WView{}, HD, OP_STORE, 1.f, nullptr, nullptr, Dst{}};
  }
  gv = pp.ngroups++;
  pp.g[gv] = Group{views[2], WView{}, HD, OP_STORE, 1.f, nullptr, nullptr, Dst{}};
  gg = pp.ngroups++;
  pp.g[gg] = Group{views[3], WView{}, HD, OP_SIGMOID, 1.f, w.g_bias, nullptr, Dst{}};
  if (a.bias_mode == LF_BIAS_NORMALIZED_INPUT) {
    gbias = pp.ngroups++;
    pp.g[gbias] = Group{views[5], WView{}, H, OP_STORE, LOG2E, nullptr, nullptr, Dst{}};
  }

  // pair-weighted averaging with d % 4 == 0: one softmax per (h, i) and an NT GEMM over the
  // sequences instead of flash attention per sequence; V^T compact, [b][h][d][Qp]
  const bool pwa = no_qk && shared_key_mask && d % 4 == 0 && !a.transpose && a.bias_mode != LF_BIAS_NONE;
  const size_t vsize = pwa ? (size_t)B * HD * Qp * sizeof(_Float16) : qkv;
  const size_t qksize = pwa ? 256 : qkv;
  size_t sizes[10] = {qksize, qksize, vsize, hd, hd, (size_t)(shared_key_mask ? 1 : B) * Qp * sizeof(float), biash, expanded_bytes(views[4]),
                     lnproj_packed_bytes(pp), a.bias_mode == LF_BIAS_SEPARATE ? lnproj_packed_bytes(pb) : (size_t)0};
  LF_TRY(workspace(ctx, sizes, bufs, 10));
  _Float16 *qb = (_Float16*)bufs[0], *kb = (_Float16*)bufs[1], *vb = (_Float16*)bufs[2];
  _Float16 *gb = (_Float16*)bufs[3], *ob = (_Float16*)bufs[4];
  float* keyb = (float*)bufs[5];
  _Float16* bias16 = (_Float16*)bufs[6];
  // every weight of the op (output projection, pair-bias and q/k/v/g projections) decoded
  // in one launch
  ExpandList xl;
  WExp wo{};
  // the output projection decodes its stored weights itself when it runs weight-resident
  const Dst out_dst = a.transpose ? Dst{a.out, a.act_dtype, Q, C, (long long)B * C, C, 0, 1}
                                  : dst_rowmajor(a.out, a.act_dtype, (int)rows, C);
  const bool wo_inkernel = rowgemm_resident(ctx, (int)rows, HD, C, out_dst);
  if (!wo_inkernel) LF_TRY(expand_add_plain(ctx, xl, views[4], bufs[7], &wo, 1.f, "attention.expand"));
  // V^T keys past Q must be zero (their weight is an exact 0, which must not meet a
  // non-finite value): the averaging GEMM reads them as stored; the flash kernel zeroes them,
  // and the head dims past d of q and k, as it reads them (FlashParams::fix)
  if (pwa && Qp != Q) LF_TRY(check_hip(hipMemsetAsync(bufs[2], 0, vsize, ctx->stream), "attention memset"));
  // f16 bias [h][i][j] (row stride Qp) from row (i, j); swapped: [h][j][i]
  const Dst bias_dst = a.swap_bias ? Dst{bias16, DT_F16, Q, 1, Qp, 1, (long long)Q * Qp, 0}
                                   : Dst{bias16, DT_F16, Q, Qp, 1, 1, (long long)Q * Qp, 0};
  if (a.bias_mode == LF_BIAS_SEPARATE) {
    pb.g[0].dst = bias_dst;
    LF_TRY(lnproj_prepare(ctx, pb, bufs[9], &xl, "attention.pair_bias"));
  }
  {
    const long long hq = (long long)Qp * DP;
    if (gq >= 0) pp.g[gq].dst = Dst{qb, DT_F16, Q, (long long)H * hq, DP, d, hq, 1};
    if (gk >= 0) pp.g[gk].dst = Dst{kb, DT_F16, Q, (long long)H * hq, DP, d, hq, 1};
    pp.g[gv].dst = pwa ? Dst{vb, DT_F16, Q, (long long)HD * Qp, 1, d, (long long)d * Qp, Qp}
                       : Dst{vb, DT_F16, Q, (long long)H * hq, 1, d, hq, Qp};
    // the gate head-major, g[h][b][q][d]: the consumers read one head's slice of many rows,
    // which is then whole lines
    pp.g[gg].dst = Dst{gb, DT_F16, Q, (long long)Q * d, d, d, (long long)B * Q * d, 1};
    if (gbias >= 0) pp.g[gbias].dst = bias_dst;
    LF_TRY(lnproj_prepare(ctx, pp, bufs[8], &xl, "attention.project"));
  }
  LF_TRY(expand_flush(ctx, xl, "attention.expand"));
  if (a.bias_mode == LF_BIAS_SEPARATE) LF_TRY(lnproj_run(ctx, pb, a.pair_dtype, "attention.pair_bias"));
  LF_TRY(lnproj_run(ctx, pp, a.act_dtype, "attention.project"));

  // 3. key-mask bias (inside a stack call, computed by the first block and reused), f16 copy
  // of the pair bias
  {
    void* cached;
    bool filled;
    LF_TRY(mask_table(ctx, a.mask, shared_key_mask ? 1 : 2 + (a.transpose ? 1 : 0), B, Q, 0.f, sizes[5], &cached,
                      &filled));
    if (cached) keyb = static_cast<float*>(cached);
    if (!filled) {
      {
        LaunchScope ls(ctx, "attention.keybias");
        if (shared_key_mask)
          hipLaunchKernelGGL(keymax_kernel, dim3((unsigned)(Qp / 64)), dim3(1024), 0, ctx->stream, a.mask, keyb, B,
                             Q, Qp);
        else
          hipLaunchKernelGGL(keybias_kernel, dim3((unsigned)(((long long)B * Qp + 255) / 256)), dim3(256), 0,
                             ctx->stream, a.mask, keyb, B, Q, Qp, a.transpose);
      }
      LF_TRY(check_hip(hipGetLastError(), "keybias launch"));
    }
  }
  // caller-supplied f32 logits are converted (and transposed per head when swapped); the
  // projected biases were written as f16 by lnproj
  if (a.bias_mode == LF_BIAS_LOGITS)
    LF_TRY(f32_to_f16(ctx, a.bias_logits, bias16, (long long)H * Q * Q, a.swap_bias ? Q : 0, LOG2E, Q, Qp));

  // 4. flash attention, or the pair-weighted averaging's softmax + GEMM
  if (pwa) {
    {
      LaunchScope ls(ctx, "attention.pwa_softmax");
      hipLaunchKernelGGL(pwa_softmax_kernel, dim3((unsigned)(((long long)H * Q + 3) / 4)), dim3(256), 0, ctx->stream,
                         bias16, keyb, H * Q, Q, Qp);
    }
    LF_TRY(check_hip(hipGetLastError(), "pwa softmax launch"));
    PwaParams wp{};
    wp.vt = vb;
    wp.p = bias16;
    wp.g = gb;
    wp.o = ob;
    wp.S = B;
    wp.H = H;
    wp.Q = Q;
    wp.Qp = Qp;
    wp.d = d;
    wp.HD = HD;
    wp.ntn = (int)(((long long)B * d + PWA_T - 1) / PWA_T);
    wp.nti = (Q + PWA_T - 1) / PWA_T;
    wp.nblocks = (long long)wp.ntn * wp.nti * H;
    LF_REQUIRE((long long)B * d < (1LL << 31) && wp.nblocks < (1LL << 31), "attention: too many sequences");
    {
      LaunchScope ls(ctx, "attention.pwa_average");
      hipLaunchKernelGGL(pwa_average_kernel, dim3((unsigned)wp.nblocks), dim3(256), 0, ctx->stream, wp);
    }
    LF_TRY(check_hip(hipGetLastError(), "pwa average launch"));
  } else {
    FlashParams fp{};
    fp.q = qb;
    fp.k = kb;
    fp.vt = vb;
    fp.g = gb;
    fp.o = ob;
    fp.kb = keyb;
    fp.kb_stride = shared_key_mask ? 0 : Qp;
    fp.bias = a.bias_mode == LF_BIAS_NONE ? nullptr : bias16;
    fp.B = B;
    fp.H = H;
    fp.Q = Q;
    fp.d = d;
    fp.HD = HD;
    fp.dq = no_qk ? 0 : d;
    fp.fix = fp.dq < DP || Q != Qp;
    fp.nqb = (Q + FA_QPB - 1) / FA_QPB;
    fp.nblocks = (long long)fp.nqb * B * H;
    LaunchScope ls(ctx, "attention.flash");
    const dim3 grid((unsigned)fp.nblocks), bb(512 / FA_QT_BIAS), bp(512 / FA_QT_PLAIN);
    constexpr bool BLD = FA_QT_BIAS == 1;
    // d <= 16 always zeroes (dq < 16 or Q ragged, or both: d = 16 with whole chunks is the
    // exception, and rare); the 32-wide kernel has a variant without the zeroing for the
    // usual d = 32 with whole chunks
    if (fp.bias && DP == 16)
      hipLaunchKernelGGL((flash_kernel<true, FA_QT_BIAS, BLD, 16, true>), grid, bb, 0, ctx->stream, fp);
    else if (fp.bias && fp.fix)
      hipLaunchKernelGGL((flash_kernel<true, FA_QT_BIAS, BLD, 32, true>), grid, bb, 0, ctx->stream, fp);
    else if (fp.bias)
      hipLaunchKernelGGL((flash_kernel<true, FA_QT_BIAS, BLD, 32, false>), grid, bb, 0, ctx->stream, fp);
    else if (DP == 16)
      hipLaunchKernelGGL((flash_kernel<false, FA_QT_PLAIN, false, 16, true>), grid, bp, 0, ctx->stream, fp);
    else if (fp.fix)
      hipLaunchKernelGGL((flash_kernel<false, FA_QT_PLAIN, false, 32, true>), grid, bp, 0, ctx->stream, fp);
    else
      hipLaunchKernelGGL((flash_kernel<false, FA_QT_PLAIN, false, 32, false>), grid, bp, 0, ctx->stream, fp);
  }
  LF_TRY(check_hip(hipGetLastError(), "flash launch"));

  // 5. output projection + residual, stored through the row map
  {
    RowGemmParams rp{};
    rp.A = ob;
    rp.rows = (int)rows;
    rp.K = HD;
    rp.N = C;
    rp.w = wo;
    rp.wv = views[4];
    rp.wview = wo_inkernel ? 1 : 0;
    rp.bias = w.o_bias;
    rp.op = OP_STORE;
    rp.resid = a.accumulate ? a.act : nullptr;
    rp.dst = out_dst;
    LF_TRY(launch_rowgemm(ctx, rp, "attention.output"));
  }
  return LF_OK;
}

}  // namespace lf
