// Outer product mean: z_ij += ((sum_s l_si (x) r_sj) W_out + b) / (norm_eps + sum_s m_si m_sj)
// with l = m * (LN(msa) Wl + bl), r likewise (AF2: webgpu/kernels/outer-product-mean.js:395-416,
// 595-610, 702-742; AF3: cpu/af3/trunk/msa.js:72-155, no projection biases, fast variance).
//
// Kernels:
//   lnproj    LN(msa) -> l, r stored [i][a][s] (sequence-contiguous: the contraction's K axis)
//   count     den[i*N + j] = norm_eps + sum_s m_si m_sj
//   outer     O[(i,j)][a*c + b] = sum_s l[i][a][s] r[j][b][s]: one NT GEMM of (N*c) x (N*c) x S on
//             MFMA, 128x128 tiles, written pair-major f16 (the next GEMM's rows)
//   rowgemm   O W_out + b, / den, + pair residual
#include <algorithm>
#include <cmath>

#include "lf_rowgemm.h"

namespace lf {

struct NtGemmParams {
  const _Float16* A;   // [M][K]
  const _Float16* B;   // [N][K]
  int M, N, K;
  float scale;
  Dst dst;             // f16, element (m, n)
};

constexpr int NT_TILE = 128, NT_BK = 64, NT_LD = NT_BK + 8;

template <bool VEC>
__device__ __forceinline__ void nt_load(_Float16* S, const _Float16* src, int rows, int K, int m0, int k0, int tid) {
  if (VEC) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int e = tid + it * 256, m = e >> 3, seg = e & 7;
      const int gm = m0 + m, gk = k0 + seg * 8;
      h8 v = h8{0, 0, 0, 0, 0, 0, 0, 0};
      if (gm < rows && gk < K) v = *reinterpret_cast<const h8*>(src + (size_t)gm * K + gk);
      *reinterpret_cast<h8*>(S + m * NT_LD + seg * 8) = v;
    }
  } else {
    for (int e = tid; e < NT_TILE * NT_BK; e += 256) {
      const int m = e / NT_BK, k = e % NT_BK, gm = m0 + m, gk = k0 + k;
      S[m * NT_LD + k] = (gm < rows && gk < K) ? src[(size_t)gm * K + gk] : (_Float16)0.f;
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(256) void nt_gemm_kernel(NtGemmParams p) {
  __shared__ __attribute__((aligned(16))) _Float16 As[NT_TILE * NT_LD];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[NT_TILE * NT_LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.x * NT_TILE, n0 = blockIdx.y * NT_TILE;
  f4 acc[4][4];
  zero_acc(acc);
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  for (int k0 = 0; k0 < p.K; k0 += NT_BK) {
    __syncthreads();
    nt_load<VEC>(As, p.A, p.M, p.K, m0, k0, tid);
    nt_load<VEC>(Bs, p.B, p.N, p.K, n0, k0, tid);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < NT_BK; kk += 32) {
      h8 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const h8*>(As + (wm * 64 + i * 16 + r16) * NT_LD + kk + kq);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const h8*>(Bs + (wn * 64 + j * 16 + r16) * NT_LD + kk + kq);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(a[i], b[j], acc[i][j]);
    }
  }
  _Float16* out = static_cast<_Float16*>(p.dst.ptr);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gm = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
      if (gm >= p.M) continue;
      const long long rp = (long long)(gm / p.dst.Q) * p.dst.sB + (long long)(gm % p.dst.Q) * p.dst.sN;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int gn = n0 + wn * 64 + j * 16 + r16;
        if (gn >= p.N) continue;
        const long long cp = (long long)(gn / p.dst.D) * p.dst.sH + (long long)(gn % p.dst.D) * p.dst.sD;
        out[rp + cp] = (_Float16)(acc[i][j][r] * p.scale);
      }
    }
}

// den[i*N + j] = eps + sum_s m[s][i] m[s][j]
__global__ __launch_bounds__(256) void opm_count_kernel(const float* mask, float* den, int S, int N, float eps) {
  const int j = blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
  if (j >= N) return;
  float c = 0.f;
  for (int s = 0; s < S; ++s) c += mask[(size_t)s * N + i] * mask[(size_t)s * N + j];
  den[(size_t)i * N + j] = eps + c;
}

int outer_product_mean(lf_context* ctx, const lf_opm_args& a) {
  LF_REQUIRE(a.w != nullptr, "outer product mean: weights are NULL");
  LF_REQUIRE(a.sequences > 0 && a.length > 0 && a.c_m > 0 && a.c_outer > 0 && a.c_z > 0,
             "outer product mean dimensions must be positive safe integers");
  LF_REQUIRE(a.c_m <= 384, "outer product mean: c_m must be <= 384");
  LF_REQUIRE(a.c_outer <= 64, "outer product mean: c_outer must be <= 64");
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
  pp.rmQ = 1;
  pp.rmB = 0;
  pp.ln_s = w.norm_scale;
  pp.ln_o = w.norm_offset;
  pp.eps = a.epsilon;
  pp.fast_var = a.fast_variance;
  pp.rowmask = a.mask;
  pp.g[0] = Group{views[0], WView{}, co, OP_ROWMASK, 1.f, w.bl, nullptr, Dst{}};
  pp.g[1] = Group{views[1], WView{}, co, OP_ROWMASK, 1.f, w.br, nullptr, Dst{}};
  pp.ngroups = 2;

  const size_t lr = (size_t)N * co * S * sizeof(_Float16);
  const size_t ob = (size_t)pairs * co * co * sizeof(_Float16);
  size_t sizes[6] = {lr, lr, ob, (size_t)pairs * sizeof(float), expanded_bytes(views[2]), lnproj_packed_bytes(pp)};
  void* bufs[6];
  LF_TRY(workspace(ctx, sizes, bufs, 6));
  _Float16 *L = (_Float16*)bufs[0], *R = (_Float16*)bufs[1], *O = (_Float16*)bufs[2];
  float* den = (float*)bufs[3];
  WExp wo;
  LF_TRY(expand_weights(ctx, &views[2], 1, &bufs[4], &wo, "opm.expand"));
  // logical row r = s*N + i -> (i*co + a)*S + s
  pp.g[0].dst = Dst{L, DT_F16, N, 1, (long long)co * S, co, 0, S};
  pp.g[1].dst = Dst{R, DT_F16, N, 1, (long long)co * S, co, 0, S};
  LF_TRY(launch_lnproj(ctx, pp, a.msa_dtype, bufs[5], "opm.project"));
  {
    LaunchScope ls(ctx, "opm.count");
    hipLaunchKernelGGL(opm_count_kernel, dim3((N + 255) / 256, N), dim3(256), 0, ctx->stream, a.mask, den, S, N,
                       a.norm_epsilon);
  }
  LF_TRY(check_hip(hipGetLastError(), "opm count launch"));
  {  // O[(i, j)][a*co + b] = sum_s l[i][a][s] r[j][b][s]
    NtGemmParams gp{};
    gp.A = L;
    gp.B = R;
    gp.M = N * co;
    gp.N = N * co;
    gp.K = S;
    gp.scale = 1.f;
    // element (m = i*co + a, n = j*co + b) -> (i*N + j)*co*co + a*co + b
    gp.dst = Dst{O, DT_F16, co, (long long)N * co * co, co, co, (long long)co * co, 1};
    dim3 grid((gp.M + NT_TILE - 1) / NT_TILE, (gp.N + NT_TILE - 1) / NT_TILE);
    LaunchScope ls(ctx, "opm.outer");
    if ((S & 7) == 0) hipLaunchKernelGGL(nt_gemm_kernel<true>, grid, dim3(256), 0, ctx->stream, gp);
    else hipLaunchKernelGGL(nt_gemm_kernel<false>, grid, dim3(256), 0, ctx->stream, gp);
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
