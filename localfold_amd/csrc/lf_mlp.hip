// Fused transition for c in {128, 256}: out = [x +] act(LN(x) W1 + b1) W2 + b2 in one kernel;
// the hidden activation never leaves registers, so no hidden buffer (and no row chunking) is
// needed.  Semantics as the two-kernel path in lf_transition.hip: ReLU (AF2,
// webgpu/kernels/transition.js:745-766, 1080-1085) or swish(h_gate) * h_value (AF3 SwiGLU,
// cpu/af3/trunk/pairformer.js:180-201).
//
// A block of 8 waves owns 256 rows, a wave 32 (two 16-row tiles).  A wave LayerNorms its rows
// into f16 MFMA fragments (lane: row lane%16, channels 32j + 8*(lane/16) .. +7) that stay in
// registers.  The hidden dimension streams through double-buffered LDS in chunks of 32 units:
// W1^T rows [32 (64 for SwiGLU: gate, then value)][C] and W2^T rows [C][32].
//   GEMM1, weights as the A operand: the lane gets H[row][16t + 4g + i] (g = lane/16, i < 4) of
//          the chunk's two 16-unit tiles t, starting from b1; then ReLU or swish-gating.
//   GEMM2: those 8 values are the lane's B fragment as they stand: MFMA k index 8g + e stands
//          for hidden unit 4g + e (e < 4) or 16 + 4g + e - 4 (e >= 4) of the chunk, and the
//          packed W2^T rows hold the hidden units in that order, so A fragments are plain
//          16-byte LDS reads.
//   Output: the lane holds out[row][16ct + 4g + i], started at b2; the residual is added and
//          four channels stored as one vector at the end.
// The next chunk's weights are loaded into registers during the current chunk's MFMAs and
// written to the other LDS buffer before the chunk's barrier.
#include <algorithm>
#include <cmath>

#include "lf_gemm.h"
#include "lf_ops.h"

namespace lf {

constexpr int MLP_WAVES = 8, MLP_ROWS = 32 * MLP_WAVES, MLP_HC = 32;

template <int C, int NG>
struct MlpShape {
  static constexpr int KS = C / 32, CT = C / 16;
  static constexpr int W1P = C + 8, W2P = MLP_HC + 8;          // LDS row pitches (halves)
  static constexpr int W1E = NG * MLP_HC * W1P;                // W1^T section of a buffer
  static constexpr int BUF = W1E + C * W2P;                    // halves per LDS buffer
  static constexpr int CE = (NG * MLP_HC + MLP_HC) * C;        // packed halves per chunk
  // 16-byte pieces of a packed chunk per thread: P1 of the W1^T rows, then P2 of the W2^T rows
  static constexpr int NT = 64 * MLP_WAVES;
  static constexpr int P1 = NG * MLP_HC * C / 8 / NT, P2 = MLP_HC * C / 8 / NT;
  static_assert(P1 * NT * 8 == NG * MLP_HC * C && P2 * NT * 8 == MLP_HC * C, "pieces must divide over the block");
};

struct MlpParams {
  const void* x;
  void* out;
  int accumulate, rows, H, fast_var;
  float eps;
  const _Float16* w;   // packed chunks (mlp_pack_kernel)
  const float *ln_s, *ln_o, *b1g, *b1v, *b2;
};

// GEMM2's k order within a chunk: position q = 8g + e holds hidden unit 4g + e (e < 4) or
// 16 + 4g + e - 4 (e >= 4); q_of is the inverse, the position of hidden unit hl (its 4-aligned
// groups stay together: q_of(4a + i) = q_of(4a) + i).
__host__ __device__ constexpr int mlp_q_of(int hl) {
  return hl < 16 ? 8 * (hl >> 2) + (hl & 3) : 8 * ((hl - 16) >> 2) + 4 + (hl & 3);
}

// Packed weights, chunk s of 32 hidden units: NG x 32 rows of W1^T (row r of group grp =
// hidden unit 32s + r of the gate (grp 0) or value (grp 1) half, over the C inputs), then C
// rows of W2^T, each holding the chunk's 32 hidden units in GEMM2's k order.  Decoding from
// f32/f16/bf16/int8/int5 happens here, on the device, one thread per run of 8 stored weights
// (wrun_fetch / wrun_decode): W1 runs are 8 inputs of one hidden unit (a 16-byte store) or 8
// hidden units of one input (8 rows); W2 runs 8 hidden units of one output (two 4-wide pieces
// of the k order) or 8 outputs of one hidden unit (8 rows).
__global__ __launch_bounds__(256) void mlp_pack_kernel(WView w1g, WView w1v, WView w2, int C, int H, int NG,
                                                       _Float16* dst) {
  const long long ce = (long long)(NG * MLP_HC + MLP_HC) * C, w1e = (long long)NG * MLP_HC * C;
  const bool k1 = w1g.run != WRUN_N, k2 = w2.run != WRUN_N;
  const long long r1 = (long long)NG * H * C / 8, total = r1 + (long long)H * C / 8;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    if (i < r1) {   // W1: (hidden unit u of group grp, input c)
      const int grp = (int)(i / ((long long)H * C / 8)), j = (int)(i - (long long)grp * H * C / 8);
      const int u = k1 ? j / (C / 8) : 8 * (j / C), c = k1 ? 8 * (j % (C / 8)) : j % C;
      const WView& w = grp ? w1v : w1g;
      const h8 h = wrun_decode(w, wrun_fetch(w, c, u, 1.f), c, u, 1.f);
      _Float16* base = dst + (long long)(u / MLP_HC) * ce + (long long)grp * MLP_HC * C + c;
      if (k1) {
        *reinterpret_cast<h8*>(base + (long long)(u % MLP_HC) * C) = h;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) base[(long long)((u + e) % MLP_HC) * C] = h[e];
      }
    } else {        // W2: (hidden unit u, output c)
      const int j = (int)(i - r1);
      const int c = k2 ? j / (H / 8) : 8 * (j % (C / 8)), u = k2 ? 8 * (j % (H / 8)) : j / (C / 8);
      const h8 h = wrun_decode(w2, wrun_fetch(w2, u, c, 1.f), u, c, 1.f);
      _Float16* base = dst + (long long)(u / MLP_HC) * ce + w1e;
      const int q = mlp_q_of(u % MLP_HC);
      if (k2) {   // hidden units u..u+3 and u+4..u+7 sit 8 apart in the k order
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          base[(long long)c * MLP_HC + q + e] = h[e];
          base[(long long)c * MLP_HC + q + 8 + e] = h[4 + e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) base[(long long)(c + e) * MLP_HC + q] = h[e];
      }
    }
  }
}

template <int ACT, int C, int NG>
__global__ __launch_bounds__(64 * MLP_WAVES) void mlp_kernel(MlpParams p) {
  using S = MlpShape<C, NG>;
  constexpr int KS = S::KS, CT = S::CT, P1 = S::P1, P2 = S::P2, NT = S::NT;
  // two buffers of two chunks each: one block barrier per pair of chunks
  __shared__ __attribute__((aligned(16))) _Float16 Wb[2][2 * S::BUF];
  __shared__ __attribute__((aligned(16))) float Gs[2 * C];   // LN scale, offset
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int nch = p.H / MLP_HC;
  const long long row_base = (long long)blockIdx.x * MLP_ROWS + wave * 32;

  // this thread's pieces of a chunk: W1^T piece k is packed element 8 * (tid + k * NT), LDS
  // row tid / (C/8) + k * NT / (C/8); W2^T piece k the same past the W1^T part, LDS row
  // tid / 4 + k * NT / 4 of the W2^T section (offsets: one base register plus constants)
  const int lw1 = (tid / (C / 8)) * S::W1P + (tid % (C / 8)) * 8;
  const int lw2 = S::W1E + (tid >> 2) * S::W2P + (tid & 3) * 8;
  auto load_w1 = [&](const _Float16* src, h8 (&r)[P1]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < P1; ++k) r[k] = *reinterpret_cast<const h8*>(src + 8 * (tid + k * NT));
  };
  auto load_w2 = [&](const _Float16* src, h8 (&r)[P2]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < P2; ++k) r[k] = *reinterpret_cast<const h8*>(src + NG * MLP_HC * C + 8 * (tid + k * NT));
  };
  auto put_w1 = [&](_Float16* dst, const h8 (&r)[P1]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < P1; ++k) *reinterpret_cast<h8*>(dst + lw1 + k * (NT / (C / 8)) * S::W1P) = r[k];
  };
  auto put_w2 = [&](_Float16* dst, const h8 (&r)[P2]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < P2; ++k) *reinterpret_cast<h8*>(dst + lw2 + k * (NT / 4) * S::W2P) = r[k];
  };
  stage_vec(Gs, p.ln_s, C, 1.f, C, tid, NT);
  stage_vec(Gs + C, p.ln_o, C, 0.f, C, tid, NT);
#pragma unroll
  for (int c = 0; c < 2; ++c) {   // chunks 0 and 1 (clamped) into buffer 0
    h8 a1[P1], a2[P2];   // (native vector types: a struct array would be copied through scratch)
    const _Float16* src = p.w + (size_t)(c < nch ? c : nch - 1) * S::CE;
    load_w1(src, a1);
    load_w2(src, a2);
    put_w1(&Wb[0][c * S::BUF], a1);
    put_w2(&Wb[0][c * S::BUF], a2);
  }
  FragTile<ACT, KS> xt[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const long long row = std::min(row_base + rt * 16 + r16, (long long)p.rows - 1);
    frag_load_row(xt[rt], p.x, (size_t)row, C, lane);
  }
  __syncthreads();
  h8 xf[2][KS];
  frag_ln_raw2(xt[0], xt[1], xf[0], xf[1], C, Gs, Gs + C, p.eps, p.fast_var, lane);
  __builtin_amdgcn_sched_barrier(0);   // the raw rows die before the accumulators are born

  f4 acc[2][CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const float4 b = p.b2 ? *reinterpret_cast<const float4*>(p.b2 + ct * 16 + 4 * g4) : make_float4(0.f, 0.f, 0.f, 0.f);
    acc[0][ct] = f4{b.x, b.y, b.z, b.w};
    acc[1][ct] = acc[0][ct];
  }

  for (int s = 0; s < nch; ++s) {
    // chunk s in slot s % 2 of buffer (s / 2) % 2; chunk s + 2 goes to the same slot of the
    // other buffer, which every wave left at the previous pair's barrier
    const _Float16* cur = &Wb[(s >> 1) & 1][(s & 1) * S::BUF];
    _Float16* nxt = &Wb[((s >> 1) & 1) ^ 1][(s & 1) * S::BUF];
    // chunk s + 2's W1^T pieces now, its W2^T pieces after GEMM1 (the last pair reloads the
    // last chunk into a buffer nothing reads again: loads stay unconditional)
    const _Float16* src = p.w + (size_t)(s + 2 < nch ? s + 2 : nch - 1) * S::CE;
    h8 n1[P1];
    load_w1(src, n1);

    // GEMM1: hacc[grp][rt][ht] = H^T tile (hidden 32s + 16ht + 4g4 + i, row r16)
    f4 hacc[NG][2][2];
#pragma unroll
    for (int grp = 0; grp < NG; ++grp) {
      const float* b1 = grp == 0 ? p.b1g : p.b1v;
#pragma unroll
      for (int ht = 0; ht < 2; ++ht) {
        const float4 b =
            b1 ? *reinterpret_cast<const float4*>(b1 + s * MLP_HC + ht * 16 + 4 * g4) : make_float4(0.f, 0.f, 0.f, 0.f);
        hacc[grp][0][ht] = f4{b.x, b.y, b.z, b.w};
        hacc[grp][1][ht] = hacc[grp][0][ht];
      }
    }
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      h8 wa[NG][2];
#pragma unroll
      for (int grp = 0; grp < NG; ++grp)
#pragma unroll
        for (int ht = 0; ht < 2; ++ht)
          wa[grp][ht] = *reinterpret_cast<const h8*>(cur + (grp * MLP_HC + ht * 16 + r16) * S::W1P + 32 * j + 8 * g4);
#pragma unroll
      for (int grp = 0; grp < NG; ++grp)
#pragma unroll
        for (int ht = 0; ht < 2; ++ht)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) hacc[grp][rt][ht] = mfma16(wa[grp][ht], xf[rt][j], hacc[grp][rt][ht]);
    }
    // activation -> GEMM2 B fragments (k order: hidden 4g4 + i, then 16 + 4g4 + i)
    h8 hb[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ht = 0; ht < 2; ++ht)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v;
          if constexpr (NG == 1) {
            v = fmaxf(hacc[0][rt][ht][i], 0.f);
          } else {
            const float gt = hacc[0][rt][ht][i];
            v = gt * sigmoidf_(gt) * hacc[1][rt][ht][i];
          }
          hb[rt][4 * ht + i] = (_Float16)v;
        }
    put_w1(nxt, n1);
    h8 n2[P2];
    load_w2(src, n2);
    __builtin_amdgcn_sched_barrier(0);
    // GEMM2, four output tiles at a time
#pragma unroll
    for (int c4 = 0; c4 < CT; c4 += 4) {
      h8 wb[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        wb[t] = *reinterpret_cast<const h8*>(cur + S::W1E + ((c4 + t) * 16 + r16) * S::W2P + 8 * g4);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) acc[rt][c4 + t] = mfma16(wb[t], hb[rt], acc[rt][c4 + t]);
      __builtin_amdgcn_sched_barrier(0);
    }
    put_w2(nxt, n2);
    if (s & 1) __syncthreads();   // block-uniform: the pair's reads done, the next pair's writes visible
  }

  // residual and store: lane -> row r16 of tile rt, channels 16ct + 4g4 .. +3
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const long long row = row_base + rt * 16 + r16;
    if (row >= p.rows) continue;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const size_t idx = (size_t)row * C + ct * 16 + 4 * g4;
      float v[4] = {acc[rt][ct][0], acc[rt][ct][1], acc[rt][ct][2], acc[rt][ct][3]};
      if (p.accumulate) {
        float r[4];
        ld4v<ACT>(p.x, idx, r);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += r[i];
      }
      st4v<ACT>(p.out, idx, v);
      __builtin_amdgcn_sched_barrier(0);   // one tile's residual in flight at a time
    }
  }
}

bool mlp_supported(int C, int H, bool swiglu) {
  return H % MLP_HC == 0 && (C == 128 || (C == 256 && !swiglu));
}

size_t mlp_packed_bytes(int C, int H, bool swiglu) {
  return (size_t)(H / MLP_HC) * (size_t)((swiglu ? 2 : 1) * MLP_HC + MLP_HC) * C * sizeof(_Float16);
}

template <int ACT>
static void launch_mlp(lf_context* ctx, const MlpParams& mp, int C, bool swiglu, dim3 grid) {
  if (C == 256)
    hipLaunchKernelGGL((mlp_kernel<ACT, 256, 1>), grid, dim3(64 * MLP_WAVES), 0, ctx->stream, mp);
  else if (swiglu)
    hipLaunchKernelGGL((mlp_kernel<ACT, 128, 2>), grid, dim3(64 * MLP_WAVES), 0, ctx->stream, mp);
  else
    hipLaunchKernelGGL((mlp_kernel<ACT, 128, 1>), grid, dim3(64 * MLP_WAVES), 0, ctx->stream, mp);
}

int transition_fused(lf_context* ctx, const lf_transition_args& a, const WView* views, void* packed) {
  const int C = a.channels, H = a.hidden;
  const bool swiglu = a.kind == LF_TRANSITION_SWIGLU;
  const int NG = swiglu ? 2 : 1;
  const lf_transition_weights& w = *a.w;
  {
    LaunchScope ls(ctx, "transition.pack");
    const long long runs = (long long)(NG + 1) * H * C / 8;
    const long long blocks = std::min<long long>((runs + 255) / 256, 8192);
    hipLaunchKernelGGL(mlp_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, views[0],
                       swiglu ? views[1] : views[0], views[NG], C, H, NG, static_cast<_Float16*>(packed));
  }
  LF_TRY(check_hip(hipGetLastError(), "transition pack launch"));
  MlpParams mp{};
  mp.x = a.act;
  mp.out = a.out;
  mp.accumulate = a.accumulate;
  mp.rows = a.rows;
  mp.H = H;
  mp.fast_var = a.fast_variance;
  mp.eps = a.epsilon;
  mp.w = static_cast<const _Float16*>(packed);
  mp.ln_s = w.norm_scale;
  mp.ln_o = w.norm_offset;
  mp.b1g = w.b1;
  mp.b1v = swiglu && w.b1 ? w.b1 + H : nullptr;
  mp.b2 = w.b2;
  const dim3 grid((unsigned)((a.rows + MLP_ROWS - 1) / MLP_ROWS));
  {
    LaunchScope ls(ctx, "transition.fused");
    if (a.act_dtype == LF_F32) launch_mlp<DT_F32>(ctx, mp, C, swiglu, grid);
    else if (a.act_dtype == LF_F16) launch_mlp<DT_F16>(ctx, mp, C, swiglu, grid);
    else launch_mlp<DT_BF16>(ctx, mp, C, swiglu, grid);
  }
  return check_hip(hipGetLastError(), "transition fused launch");
}

}  // namespace lf
