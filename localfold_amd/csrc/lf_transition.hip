// Transition: x += ReLU(LN(x) W1 + b1) W2 + b2 (AF2, webgpu/kernels/transition.js:745-766,
// 1080-1085) or x += (swish(h[:H]) * h[H:]) W2 with h = LN(x) W1 (AF3 SwiGLU, blocked split,
// cpu/af3/trunk/pairformer.js:180-201).
//
// c = 128 / 256 (every AF2/AF3 pair and MSA width) runs fused in one kernel (lf_mlp.hip).
// Otherwise two kernels per row chunk: lnproj (LN + W1 + activation -> f16 hidden) and rowgemm
// (hidden W2 + b2 + residual).  Rows are chunked so the hidden buffer stays within `chunk_bytes`
// (transitionChunkRows, webgpu/kernels/transition.js:411-442, without WebGPU's binding-offset
// alignment, which HIP does not have).
#include <algorithm>
#include <cmath>
#include <string>

#include "lf_rowgemm.h"

namespace lf {

int transition(lf_context* ctx, const lf_transition_args& a) {
  LF_REQUIRE(a.w != nullptr, "transition: weights are NULL");
  LF_REQUIRE(a.rows > 0 && a.channels > 0 && a.hidden > 0, "transition dimensions must be positive safe integers");
  LF_REQUIRE(a.channels <= 384, "transition: channels must be <= 384");
  LF_REQUIRE(a.kind == LF_TRANSITION_RELU || a.kind == LF_TRANSITION_SWIGLU, "transition: unknown kind");
  LF_REQUIRE(act_dtype_ok(a.act_dtype), "transition: act_dtype must be f32, f16 or bf16");
  LF_REQUIRE(a.act && a.out, "transition: act and out must be device pointers");
  LF_REQUIRE(a.epsilon > 0.f && std::isfinite(a.epsilon), "transition: epsilon must be finite and positive");
  const lf_transition_weights& w = *a.w;
  const int C = a.channels, Hd = a.hidden;
  WView views[3];
  int nv = 0;
  if (a.kind == LF_TRANSITION_RELU) {
    LF_TRY(make_view(w.w1, C, Hd, "firstWeight", &views[nv++]));
  } else {
    LF_TRY(make_view(w.w1, C, Hd, "transition1(gate half)", &views[nv++], 0, 1, true));
    LF_TRY(make_view(w.w1, C, Hd, "transition1(value half)", &views[nv++], Hd, 1, true));
    const int outs = w.w1.layout == LF_IN_OUT ? w.w1.cols : w.w1.rows;
    LF_REQUIRE(outs == 2 * Hd, "transition1 must have 2 * hidden outputs (gate half, then value half)");
  }
  LF_TRY(make_view(w.w2, Hd, C, "secondWeight", &views[nv++]));

  // fused path: one kernel, no hidden buffer (vector loads need 16-byte aligned rows and biases)
  const bool swiglu = a.kind == LF_TRANSITION_SWIGLU;
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  if (mlp_supported(C, Hd, swiglu) && al16(a.act) && al16(a.out) && al16(w.b1) && al16(w.b2)) {
    size_t sz = mlp_packed_bytes(C, Hd, swiglu);
    void* packed;
    LF_TRY(workspace(ctx, &sz, &packed, 1));
    return transition_fused(ctx, a, views, packed);
  }

  // rows per chunk: all when the f16 hidden buffer fits the budget, else a multiple of 128
  const long long budget = a.chunk_bytes > 0 ? a.chunk_bytes : 32LL * 1024 * 1024;
  const long long row_bytes = (long long)Hd * (long long)sizeof(_Float16);
  long long chunk = a.rows;
  if ((long long)a.rows * row_bytes > budget) {
    chunk = (budget / row_bytes) / 128 * 128;
    LF_REQUIRE(chunk >= 128, "transition: chunk budget cannot hold one 128-row tile of the hidden activation");
  }
  LnProjParams pp{};
  pp.C = C;
  pp.rmQ = 1;
  pp.rmB = 0;
  pp.ln_s = w.norm_scale;
  pp.ln_o = w.norm_offset;
  pp.eps = a.epsilon;
  pp.fast_var = a.fast_variance;
  pp.ngroups = 1;
  if (a.kind == LF_TRANSITION_RELU)
    pp.g[0] = Group{views[0], WView{}, Hd, OP_RELU, 1.f, w.b1, nullptr, Dst{}};
  else
    pp.g[0] = Group{views[0], views[1], Hd, OP_SWIGLU, 1.f, w.b1, w.b1 ? w.b1 + Hd : nullptr, Dst{}};

  size_t sizes[3] = {(size_t)(chunk * row_bytes), expanded_bytes(views[nv - 1]), lnproj_packed_bytes(pp)};
  void* bufs[3];
  LF_TRY(workspace(ctx, sizes, bufs, 3));
  _Float16* hid = static_cast<_Float16*>(bufs[0]);
  WExp w2;
  LF_TRY(expand_weights(ctx, &views[nv - 1], 1, &bufs[1], &w2, "transition.expand"));
  const size_t ab = act_bytes(a.act_dtype);

  for (long long r0 = 0; r0 < a.rows; r0 += chunk) {
    const int n = (int)std::min<long long>(chunk, a.rows - r0);
    pp.x = static_cast<const char*>(a.act) + (size_t)r0 * C * ab;
    pp.rows = n;
    pp.g[0].dst = dst_rowmajor(hid, DT_F16, n, Hd);
    LF_TRY(launch_lnproj(ctx, pp, a.act_dtype, bufs[2], "transition.first", r0 == 0));

    RowGemmParams rp{};
    rp.A = hid;
    rp.rows = n;
    rp.K = Hd;
    rp.N = C;
    rp.w = w2;
    rp.bias = w.b2;
    rp.op = OP_STORE;
    rp.resid = a.accumulate ? static_cast<const char*>(a.act) + (size_t)r0 * C * ab : nullptr;
    rp.dst = dst_rowmajor(static_cast<char*>(a.out) + (size_t)r0 * C * ab, a.act_dtype, n, C);
    LF_TRY(launch_rowgemm(ctx, rp, "transition.second"));
  }
  return LF_OK;
}

}  // namespace lf
