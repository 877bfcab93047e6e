// Host-side helpers shared by the op launchers: weight-record validation and the
// conversion of an lf_weight into the kernels' logical K x N view.
#pragma once
#include <string>

#include <algorithm>

#include "lf_gemm.h"
#include "lf_context.h"

namespace lf {

// Validates `w` as a logical [K x N] matrix (K inputs, N outputs) and builds its view.
// `col_off`/`col_stride` select a strided subset of the stored output columns (AF3's
// interleaved a/b split); the stored output count must cover them.
// `subset` allows the view to cover only part of the stored outputs (e.g. one half of a fused
// projection); otherwise a unit-stride view must match the stored output count exactly.
int make_view(const lf_weight& w, int K, int N, const char* name, WView* out, int col_off = 0,
              int col_stride = 1, bool subset = false);

// Decodes `count` weight views into f16 E[n][k] tiles at dst[i] (expanded_bytes(views[i]) each).
// scales (nullable): per-matrix factor applied to the decoded values before the f16 rounding
int expand_weights(lf_context* ctx, const WView* views, int count, void* const* dst, WExp* out, const char* label,
                   const float* scales = nullptr);
size_t expanded_bytes(const WView& v);
// Decodes views[m] into the chunk layout of a packed buffer: column n -> row
// row0[m] + (n / W[m]) * 64 + off[m] + n % W[m], pitch kp, padding columns zeroed.
int expand_packed(lf_context* ctx, const WView* views, const int* W, const int* off, const long long* row0,
                  int count, _Float16* dst, int kp, const char* label);
// Expansions collected for one launch: an op queues every matrix it decodes (plain views
// and packed chunk layouts alike), then flushes once -- one expand launch per op instead of
// one per weight group.  A full batch (8 matrices) launches as it fills.
struct ExpandList {
  ExpandBatch b{};
  long most = 0;
};
int expand_add_plain(lf_context* ctx, ExpandList& l, const WView& v, void* dst, WExp* out, float scale,
                     const char* label);
int expand_add_packed(lf_context* ctx, ExpandList& l, const WView* views, const int* W, const int* off,
                      const long long* row0, int count, _Float16* dst, int kp, const char* label);
int expand_flush(lf_context* ctx, ExpandList& l, const char* label);
// dst = scale * src as f16; tq > 0 transposes each tq x tq plane; ld > 0 writes rows of rowlen
// values at a row stride of ld
int f32_to_f16(lf_context* ctx, const float* src, _Float16* dst, long long n, int tq, float scale = 1.f,
               int rowlen = 0, int ld = 0);

inline bool act_dtype_ok(int dt) { return dt == LF_F32 || dt == LF_F16 || dt == LF_BF16; }
inline size_t act_bytes(int dt) { return dt == LF_F32 ? 4 : 2; }

int tri_mult(lf_context* ctx, const lf_tri_mult_args& a);
// lf_tri_mult on the library's static per-device scratch (no allocation); tri_noalloc_init
// looks up that scratch's address on `device`, which must be current
int tri_mult_noalloc(lf_context* ctx, const lf_tri_mult_args& a);
int tri_noalloc_init(int device);
// no_qk: every logit is the bias alone (AF3 pair-weighted averaging; wq/wk are not read);
// shared_key_mask: one key mask for every batch row, the maximum of a.mask over the batch
int attention(lf_context* ctx, const lf_attention_args& a, bool no_qk = false, bool shared_key_mask = false);
int transition(lf_context* ctx, const lf_transition_args& a);
// fused transition (lf_mlp.hip): c = 128 (ReLU or SwiGLU) or 256 (ReLU), hidden % 32 == 0;
// views: W1 (gate half), [W1 value half,] W2; packed: mlp_packed_bytes of workspace
bool mlp_supported(int C, int H, bool swiglu);
size_t mlp_packed_bytes(int C, int H, bool swiglu);
int transition_fused(lf_context* ctx, const lf_transition_args& a, const WView* views, void* packed);
int outer_product_mean(lf_context* ctx, const lf_opm_args& a);
int global_attention(lf_context* ctx, const lf_global_attention_args& a);
int input_embedder(lf_context* ctx, const lf_input_embedder_args& a);

}  // namespace lf
