// Generic row GEMMs on MFMA, shared by the attention, transition and outer-product-mean ops.
//
//  lnproj   y = epilogue(LN(x) W) for LayerNorm'd activation rows (K <= 384): each wave
//           normalises 16 rows straight into MFMA A fragments, then the block streams the
//           weights in 64-column chunks through double-buffered LDS.  Columns are organised
//           in up to 6 GROUPS (e.g. q, k, v, gate, pair bias), each with its own weight
//           matrix, epilogue op and destination layout.
//  rowgemm  y = epilogue(A W) for f16 rows A [rows][K] (any K, streamed in 128-deep slices),
//           with bias, ReLU, a per-row denominator and a residual accumulate through a row map.
//
// Destinations are strided layouts: element (row, col) of a group lands at
//   (row / Q) * sB + (row % Q) * sN + (col / D) * sH + (col % D) * sD
// which covers row-major, channel-major, head-split [b][h][n][d] and transposed [b][h][d][n].
#pragma once
#include "lf_gemm.h"
#include "lf_ops.h"

namespace lf {

struct Dst {
  void* ptr;
  int dtype;       // DT_F32 / DT_F16 / DT_BF16
  int Q;
  long long sB, sN;
  int D;
  long long sH, sD;
};

enum GroupOp { OP_STORE = 0, OP_SIGMOID = 1, OP_RELU = 2, OP_SWIGLU = 3, OP_ROWMASK = 4 };

// One output group of an lnproj launch.  Paired ops (OP_SWIGLU) take 32 columns of w0 (gate)
// and the same 32 columns of w1 (value) per 64-row weight chunk; the others 64 columns of w0.
// The launcher decodes every group's weights into one packed [chunk][64][KP] f16 buffer in
// the order the kernel consumes them.
struct Group {
  WView w0, w1;
  int ncols;          // logical output columns of the group
  int op;
  float scale;        // multiplies the (biased) GEMM result before the op
  const float* bias0; // per output column (nullable)
  const float* bias1;
  Dst dst;
  int tr;             // set by launch_lnproj: the epilogue runs on the transposed tile (a lane
                      // holds 4 consecutive rows of one column) for destinations whose rows,
                      // not columns, are contiguous
  int vec;            // set by launch_lnproj: every 4-element run a lane stores (4 columns, or
                      // 4 rows when tr) is contiguous and 8-byte aligned
};

constexpr int MAX_GROUPS = 6;
constexpr int MAX_CHUNKS = 128;   // 64-column weight chunks per lnproj launch

struct LnProjParams {
  const void* x;
  int rows, C;        // logical rows, channels (LN width == K)
  int rmQ, rmB;       // row map: logical row r = b*rmQ + q reads storage row q*rmB + b (rmB > 0) or r
  const float *ln_s, *ln_o;
  float eps;
  int fast_var;
  const float* rowmask;   // OP_ROWMASK multiplier, indexed by storage row
  Group g[MAX_GROUPS];
  int ngroups;
  const _Float16* wpk;    // packed weights (set by launch_lnproj)
  int nchunks;            // set by launch_lnproj: chunk ci covers group chunk_group[ci]'s
  int chunk_group[MAX_CHUNKS];   // logical columns from chunk_c0[ci] (ints: kernel-argument
  int chunk_c0[MAX_CHUNKS];      // loads of them are scalar, so no vector-memory wait)
  int chunk_fast[MAX_CHUNKS];    // the chunk's columns all exist and its group is vec
};

struct RowGemmParams {
  const _Float16* A;  // [rows][K] f16 (logical rows)
  int rows, K, N;
  WExp w;             // [N][kp]; or, with wview set, the stored weights
  WView wv;           // decoded inside the kernel (weight-resident form only: rowgemm_resident)
  int wview;
  const float* bias;  // [N] nullable
  int op;             // OP_STORE or OP_RELU
  const float* rowden;  // divide row r by rowden[r] (nullable; OPM's norm_eps + sum_s m_si m_sj)
  const void* resid;  // residual added when non-null (same layout and dtype as dst)
  Dst dst;
};

// Host launchers (defined in lf_rowgemm.hip).  `act` is the dtype of x.  `packed` is
// workspace of lnproj_packed_bytes(p) bytes for the decoded weights; repeated launches with
// the same weights (row chunks) pass decode = false after the first.
size_t lnproj_packed_bytes(const LnProjParams& p);
// Whether launch_rowgemm takes the weight-resident form for this shape: then the caller may
// pass the stored weights (RowGemmParams::wv, wview = 1) instead of an f16 expansion, and each
// block decodes them into LDS once.
bool rowgemm_resident(const lf_context* ctx, int rows, int K, int N, const Dst& dst);
int launch_lnproj(lf_context* ctx, LnProjParams p, int act, void* packed, const char* label, bool decode = true);
// launch_lnproj in two steps, so that an op decodes all its weights in one launch: prepare
// validates p, fills its chunk tables and queues the decode of its weights into `packed` on
// xl (null: the caller decoded them before); run launches the kernel once they are decoded.
int lnproj_prepare(lf_context* ctx, LnProjParams& p, void* packed, ExpandList* xl, const char* label);
int lnproj_run(lf_context* ctx, const LnProjParams& p, int act, const char* label);
int launch_rowgemm(lf_context* ctx, const RowGemmParams& p, const char* label);

inline Dst dst_rowmajor(void* ptr, int dtype, int rows, int cols) {
  return Dst{ptr, dtype, rows > 0 ? rows : 1, 0, cols, cols, 0, 1};
}

}  // namespace lf
