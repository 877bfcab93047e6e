// Shared MFMA tile machinery: weight staging (in-kernel dequant into LDS) and the
// 16-row x (16*NT)-column wave tile over an LDS-resident A block.
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

// Ws[n][k] = E[n_base + n][k] for n < ncols, k < e.kp (zero past the valid columns).
__device__ __forceinline__ void stage_expanded(_Float16* Ws, int ldw, const WExp& e, int ncols, int n_base, int tid,
                                               int nthreads) {
  const int segs = e.kp >> 3;
  const int total = ncols * segs;
  for (int i = tid; i < total; i += nthreads) {
    const int n = i / segs, seg = i - n * segs;
    h8 v = h8{0, 0, 0, 0, 0, 0, 0, 0};
    if (n_base + n < e.N) v = *reinterpret_cast<const h8*>(e.p + (size_t)(n_base + n) * e.kp + seg * 8);
    *reinterpret_cast<h8*>(Ws + n * ldw + seg * 8) = v;
  }
}

// Ws[n][k] = W[k][n_base + n] for n < ncols, k < kpad (zero outside the view).
__device__ __forceinline__ void stage_weights(_Float16* Ws, int ldw, const WView& w, int ncols, int n_base,
                                              int kpad, int tid, int nthreads) {
  const int total = ncols * kpad;
  if (w.ld_k == 1) {
    for (int e = tid; e < total; e += nthreads) {
      const int n = e / kpad, k = e - n * kpad;
      Ws[n * ldw + k] = (_Float16)wdecode(w, k, n_base + n);
    }
  } else {
    for (int e = tid; e < total; e += nthreads) {
      const int k = e / ncols, n = e - k * ncols;
      Ws[n * ldw + k] = (_Float16)wdecode(w, k, n_base + n);
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
