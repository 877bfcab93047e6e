// Global column attention of the AF2 extra-MSA stack: encodeGlobalAttention
// (webgpu/af2/evoformer/block.js:953-1030) and its kernels (block.js:88-400).  Per residue
// column i, over the sequences s, with x = LN(msa):
//   k_si = x_si Wk, v_si = x_si Wv (one head of width d shared by every query head),
//   q_ih = (sum_s m_si x_si / (1e-10 + sum_s m_si)) Wq_h / sqrt(d),
//   a_ih = sum_s softmax_s(q_ih . k_si, -1e9 where m_si = 0) v_si,
//   update_si = (sigmoid(x_si Wg + bg) * a_i) Wo + bo.
//
// Kernels:
//   lnproj   LN(msa) -> qm = m * (x Wq) [N][S][H*d], k, v [N][S][d] (column-contiguous), gate
//            sigmoid(x Wg + bg) [S*N][H*d]; the mean of qm over s is q (the projection is
//            linear, so projecting then averaging equals the reference's average then project)
//   column   one block per column: the mask count, q, an online softmax over the sequences
//            (each thread a stride of sequences, merged over lanes and waves), then the gate
//            rows of the column multiplied in place by a_i
//   rowgemm  gate Wo + bo, + residual
#include <algorithm>
#include <cmath>

#include "lf_rowgemm.h"

namespace lf {

constexpr int GA_MAXHD = 64;   // heads * head_dim supported by the column kernel
constexpr int GA_NT = 256;

struct GlobalColumnParams {
  const _Float16 *qm, *k, *v;   // [N][S][Hd], [N][S][d], [N][S][d]
  _Float16* gate;               // [S*N][Hd], multiplied in place by the column's attended values
  const float* mask;            // [S][N]
  int S, N, H, d;
  float scale;                  // 1/sqrt(d)
};

// Merges an online-softmax state (m, l, acc) with another one (exp of -1e30-scale gaps is 0,
// so an empty state merges away).
template <int D>
__device__ __forceinline__ void sm_merge(float& m, float& l, float (&acc)[D], float m2, float l2, const float (&acc2)[D]) {
  const float mx = fmaxf(m, m2);
  const float a = __expf(m - mx), b = __expf(m2 - mx);
  l = l * a + l2 * b;
#pragma unroll
  for (int e = 0; e < D; ++e) acc[e] = acc[e] * a + acc2[e] * b;
  m = mx;
}

template <int D>
__global__ __launch_bounds__(GA_NT) void global_column_kernel(GlobalColumnParams p) {
  constexpr int HMAX = GA_MAXHD / D;            // heads this head width allows
  __shared__ float part[32][GA_MAXHD];          // query partial sums: 32 row groups
  __shared__ float qs[GA_MAXHD];
  __shared__ float wstate[4][GA_MAXHD + 2 * HMAX];   // per wave: acc [H*D], max [H], sum [H]
  __shared__ float att[GA_MAXHD];
  __shared__ float cnt[4];
  const int i = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int S = p.S, N = p.N, H = p.H, Hd = H * D, pr = Hd / 8;   // 16-byte pieces per row

  // the column's mask count
  float c = 0.f;
  for (int s = tid; s < S; s += GA_NT) c += p.mask[(size_t)s * N + i];
  c = wave_sum(c);
  if (lane == 0) cnt[wave] = c;
  // q: sum over the sequences of qm (16-byte pieces: thread -> piece tid % pr of rows tid / pr + k*rg)
  {
    const int rg = min(32, GA_NT / pr), piece = tid % pr, r0 = tid / pr;   // row groups (<= 32 stored)
    float t[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (r0 < rg)
      for (int s = r0; s < S; s += rg) {
        const h8 v = *reinterpret_cast<const h8*>(p.qm + ((size_t)i * S + s) * Hd + piece * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] += (float)v[e];
      }
    if (r0 < 32) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[r0][piece * 8 + e] = r0 < rg ? t[e] : 0.f;
    }
  }
  __syncthreads();
  const float den = 1e-10f + cnt[0] + cnt[1] + cnt[2] + cnt[3];
  const int rg = min(32, GA_NT / pr);
  for (int hd = tid; hd < Hd; hd += GA_NT) {
    float t = 0.f;
    for (int r = 0; r < rg; ++r) t += part[r][hd];
    qs[hd] = t / den * p.scale;
  }
  __syncthreads();

  // online softmax over this thread's sequences, every head at once (k, v loaded once a sequence)
  float m[HMAX], l[HMAX], acc[HMAX][D];
#pragma unroll
  for (int h = 0; h < HMAX; ++h) {
    m[h] = -1e30f;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < D; ++e) acc[h][e] = 0.f;
  }
  for (int s = tid; s < S; s += GA_NT) {
    float kv[D], vv[D];
#pragma unroll
    for (int e8 = 0; e8 < D; e8 += 8) {
      const h8 kk = *reinterpret_cast<const h8*>(p.k + ((size_t)i * S + s) * D + e8);
      const h8 vx = *reinterpret_cast<const h8*>(p.v + ((size_t)i * S + s) * D + e8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kv[e8 + e] = (float)kk[e];
        vv[e8 + e] = (float)vx[e];
      }
    }
    const bool masked = p.mask[(size_t)s * N + i] == 0.f;
#pragma unroll
    for (int h = 0; h < HMAX; ++h) {
      if (h >= H) break;
      float logit = 0.f;
#pragma unroll
      for (int e = 0; e < D; ++e) logit += qs[h * D + e] * kv[e];
      if (masked) logit = -1e9f;
      const float mx = fmaxf(m[h], logit);
      const float a = __expf(m[h] - mx), w = __expf(logit - mx);
      l[h] = l[h] * a + w;
#pragma unroll
      for (int e = 0; e < D; ++e) acc[h][e] = acc[h][e] * a + w * vv[e];
      m[h] = mx;
    }
  }
  // merge over the wave's lanes, then the four waves through LDS
#pragma unroll
  for (int h = 0; h < HMAX; ++h) {
    if (h >= H) break;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float acc2[D];
#pragma unroll
      for (int e = 0; e < D; ++e) acc2[e] = __shfl_xor(acc[h][e], o, WAVE);
      sm_merge<D>(m[h], l[h], acc[h], __shfl_xor(m[h], o, WAVE), __shfl_xor(l[h], o, WAVE), acc2);
    }
    if (lane == 0) {
#pragma unroll
      for (int e = 0; e < D; ++e) wstate[wave][h * D + e] = acc[h][e];
      wstate[wave][Hd + h] = m[h];
      wstate[wave][Hd + HMAX + h] = l[h];
    }
  }
  __syncthreads();
  for (int hd = tid; hd < Hd; hd += GA_NT) {
    const int h = hd / D;
    float mm = wstate[0][Hd + h], ll = wstate[0][Hd + HMAX + h], a = wstate[0][hd];
    for (int w2 = 1; w2 < 4; ++w2) {
      const float m2 = wstate[w2][Hd + h], l2 = wstate[w2][Hd + HMAX + h], a2 = wstate[w2][hd];
      const float mx = fmaxf(mm, m2), x1 = __expf(mm - mx), x2 = __expf(m2 - mx);
      ll = ll * x1 + l2 * x2;
      a = a * x1 + a2 * x2;
      mm = mx;
    }
    att[hd] = a / ll;
  }
  __syncthreads();
  // gate rows of this column times the attended values, in place, 16 bytes at a time
  for (int e = tid; e < S * pr; e += GA_NT) {
    const int s = e / pr, piece = e - s * pr;
    h8* g = reinterpret_cast<h8*>(p.gate + ((size_t)s * N + i) * Hd + piece * 8);
    h8 v = *g;
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = (_Float16)((float)v[u] * att[piece * 8 + u]);
    *g = v;
  }
}

int global_attention(lf_context* ctx, const lf_global_attention_args& a) {
  LF_REQUIRE(a.w != nullptr, "global column attention: weights are NULL");
  LF_REQUIRE(a.sequences > 0 && a.length > 0 && a.channels > 0 && a.heads > 0,
             "global column attention dimensions must be positive");
  LF_REQUIRE(act_dtype_ok(a.act_dtype), "global column attention: act_dtype must be f32, f16 or bf16");
  LF_REQUIRE(a.act && a.mask && a.out, "global column attention: act, mask and out must be device pointers");
  LF_REQUIRE(a.channels <= 384 && a.channels % 4 == 0, "global column attention: channels must be a multiple of 4, <= 384");
  if (a.head_dim == 0)
    LF_REQUIRE(a.channels % a.heads == 0, "global column attention: channels must be a multiple of heads when head_dim is 0");
  const int S = a.sequences, N = a.length, C = a.channels, H = a.heads;
  const int d = a.head_dim > 0 ? a.head_dim : C / H, Hd = H * d;
  LF_REQUIRE(d == 8 || d == 16 || d == 32, "global column attention: head dimension must be 8, 16 or 32");
  LF_REQUIRE(Hd <= GA_MAXHD && H <= 8, "global column attention: heads * head_dim must be <= 64 and heads <= 8");
  LF_REQUIRE(a.epsilon > 0.f && std::isfinite(a.epsilon), "global column attention: epsilon must be finite and positive");
  const long long rows = (long long)S * N;
  LF_REQUIRE(rows * std::max(Hd, C) < (1LL << 31), "global column attention: too many rows");
  const lf_global_attention_weights& w = *a.w;

  WView views[5];
  LF_TRY(make_view(w.wq, C, Hd, "queryWeight", &views[0]));
  LF_TRY(make_view(w.wk, C, d, "keyWeight", &views[1]));
  LF_TRY(make_view(w.wv, C, d, "valueWeight", &views[2]));
  LF_TRY(make_view(w.wg, C, Hd, "gatingWeight", &views[3]));
  LF_TRY(make_view(w.wo, Hd, C, "outputWeight", &views[4]));

  LnProjParams pp{};
  pp.x = a.act;
  pp.rows = (int)rows;
  pp.C = C;
  pp.ln_s = w.norm_scale;
  pp.ln_o = w.norm_offset;
  pp.eps = a.epsilon;
  pp.rowmask = a.mask;   // storage row s*N + i is mask[s][i]
  pp.g[0] = Group{views[0], WView{}, Hd, OP_ROWMASK, 1.f, nullptr, nullptr, Dst{}};
  pp.g[1] = Group{views[1], WView{}, d, OP_STORE, 1.f, nullptr, nullptr, Dst{}};
  pp.g[2] = Group{views[2], WView{}, d, OP_STORE, 1.f, nullptr, nullptr, Dst{}};
  pp.g[3] = Group{views[3], WView{}, Hd, OP_SIGMOID, 1.f, w.g_bias, nullptr, Dst{}};
  pp.ngroups = 4;

  const size_t qb = (size_t)rows * Hd * sizeof(_Float16), kb = (size_t)rows * d * sizeof(_Float16);
  size_t sizes[6] = {qb, kb, kb, qb, expanded_bytes(views[4]), lnproj_packed_bytes(pp)};
  void* bufs[6];
  LF_TRY(workspace(ctx, sizes, bufs, 6));
  _Float16 *QM = (_Float16*)bufs[0], *K = (_Float16*)bufs[1], *V = (_Float16*)bufs[2], *G = (_Float16*)bufs[3];
  // logical row r = s*N + i (the storage row); column-contiguous [i][s][.] for qm, k, v
  pp.g[0].dst = Dst{QM, DT_F16, N, (long long)Hd, (long long)S * Hd, Hd, 0, 1};
  pp.g[1].dst = Dst{K, DT_F16, N, (long long)d, (long long)S * d, d, 0, 1};
  pp.g[2].dst = Dst{V, DT_F16, N, (long long)d, (long long)S * d, d, 0, 1};
  pp.g[3].dst = dst_rowmajor(G, DT_F16, (int)rows, Hd);
  // the projections and the output weights decoded in one launch
  ExpandList xl;
  WExp wo{};
  const Dst out_dst = dst_rowmajor(a.out, a.act_dtype, (int)rows, C);
  const bool wo_inkernel = rowgemm_resident(ctx, (int)rows, Hd, C, out_dst);
  if (!wo_inkernel) LF_TRY(expand_add_plain(ctx, xl, views[4], bufs[4], &wo, 1.f, "global.expand"));
  LF_TRY(lnproj_prepare(ctx, pp, bufs[5], &xl, "global.project"));
  LF_TRY(expand_flush(ctx, xl, "global.expand"));
  LF_TRY(lnproj_run(ctx, pp, a.act_dtype, "global.project"));

  GlobalColumnParams gp{QM, K, V, G, a.mask, S, N, H, d, 1.f / std::sqrt((float)d)};
  {
    LaunchScope ls(ctx, "global.column");
    if (d == 8) hipLaunchKernelGGL(global_column_kernel<8>, dim3(N), dim3(GA_NT), 0, ctx->stream, gp);
    else if (d == 16) hipLaunchKernelGGL(global_column_kernel<16>, dim3(N), dim3(GA_NT), 0, ctx->stream, gp);
    else hipLaunchKernelGGL(global_column_kernel<32>, dim3(N), dim3(GA_NT), 0, ctx->stream, gp);
  }
  LF_TRY(check_hip(hipGetLastError(), "global column launch"));

  RowGemmParams rp{};
  rp.A = G;
  rp.rows = (int)rows;
  rp.K = Hd;
  rp.N = C;
  rp.w = wo;
  rp.wv = views[4];
  rp.wview = wo_inkernel ? 1 : 0;
  rp.bias = w.o_bias;
  rp.op = OP_STORE;
  rp.resid = a.accumulate ? a.act : nullptr;
  rp.dst = out_dst;
  return launch_rowgemm(ctx, rp, "global.output");
}

}  // namespace lf
