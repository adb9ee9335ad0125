// fp32 MFMA contraction for the CROWN backward pass (gfx950).
//
//   C[M, N] = A'[M, K] x B[K, N]
//
// M = domains x specs (the coefficient rows), K = current-layer neurons,
// N = previous-layer neurons.  A' is either A itself or A after the ReLU
// relaxation of the layer (boundflow/runtime/crown_ibp.py:1211-1298), applied
// while the A tile is staged into LDS; the row reductions the relaxation needs
// (the bias terms sum_k A * beta_sel and sum_k A' * bias_k, and optionally a
// center term sum_k A' * c_k) are produced in the same pass.  The epilogue
// either stores C or reduces |C| (optionally weighted) along each row, which is
// the Linf / box concretization norm (boundflow/runtime/perturbation.py:175-222,
// 327-359) fused so that the final [M, input] coefficient never reaches HBM.
//
// Tiling: 256 threads = 4 wave64s, block tile 128 x 128, K tile 16, each wave
// owns a 64 x 64 sub-tile computed with 2 x 2 v_mfma_f32_32x32x2f32 ops per
// k-pair.  A and B tiles are stored k-major in LDS (pitch +4 floats) and
// double-buffered; global loads of tile k+1 are in flight while tile k feeds
// the matrix cores.

#include "bf_common.h"
#include "bf_gemm_args.h"

namespace bf {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 128;
constexpr int GBN = 128;
constexpr int GBK = 16;
constexpr int GNT = 256;
constexpr int APITCH = GBM + 4;
constexpr int BPITCH = GBN + 4;
constexpr int A_PER_T = GBM * GBK / GNT;  // 8
constexpr int B_PER_T = GBN * GBK / GNT;  // 8

__device__ __forceinline__ float select_scale(float a, const Relax& r, bool lower, float* beta_sel) {
  // upper: A >= 0 -> (alpha_u, beta_u) else (alpha_l, beta_l); lower: mirrored
  const bool nonneg = a >= 0.f;
  float al, be;
  if (lower) {
    al = nonneg ? r.al : r.au;
    be = nonneg ? r.bl : r.bu;
  } else {
    al = nonneg ? r.au : r.al;
    be = nonneg ? r.bu : r.bl;
  }
  *beta_sel = be;
  return al;
}

template <int PRO, int EPI, bool TRANS_B>
__global__ void __launch_bounds__(GNT)
gemm_kernel(GemmArgs p) {
  __shared__ float As[2][GBK][APITCH];
  __shared__ float Bs[2][GBK][BPITCH];
  __shared__ float red[2][GBM];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int z = blockIdx.z;
  const bool lower = p.z_lower_first ? (z == 0) : (z == 1);
  const float* __restrict__ A = p.A[z];
  const int64_t m0 = (int64_t)blockIdx.x * GBM;
  const int64_t n0 = (int64_t)blockIdx.y * GBN;
  const int64_t M = p.M, N = p.N, K = p.K;
  const bool row_reduce = (PRO == PRO_RELAX) && (blockIdx.y == 0);

  // A-tile element ownership: e = t + GNT*j -> row = e / GBK, kk = e % GBK
  const int a_kk = t % GBK;
  const int a_r0 = t / GBK;  // rows a_r0 + 16*j
  int64_t a_dom[A_PER_T];
  float s_beta[A_PER_T], s_bias[A_PER_T], s_cen[A_PER_T];
#pragma unroll
  for (int j = 0; j < A_PER_T; ++j) {
    int64_t m = m0 + a_r0 + 16 * j;
    a_dom[j] = (PRO == PRO_RELAX) ? (m < M ? m / p.S : 0) : 0;
    s_beta[j] = 0.f; s_bias[j] = 0.f; s_cen[j] = 0.f;
  }

  float a_reg[A_PER_T];
  float b_reg[B_PER_T];

  // A row base offsets (rows are d*S + s; see GemmArgs::lda_d)
  int64_t a_base[A_PER_T];
#pragma unroll
  for (int j = 0; j < A_PER_T; ++j) {
    int64_t m = m0 + a_r0 + 16 * j;
    int64_t mm = m < M ? m : 0;
    a_base[j] = (mm / p.S) * p.lda_d + (mm % p.S) * p.lda;
  }

  auto load_tiles = [&](int64_t k0) {
#pragma unroll
    for (int j = 0; j < A_PER_T; ++j) {
      int64_t m = m0 + a_r0 + 16 * j;
      int64_t k = k0 + a_kk;
      a_reg[j] = (m < M && k < K) ? A[a_base[j] + k] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < B_PER_T; ++j) {
      int e = t + GNT * j;
      float v;
      if (TRANS_B) {
        int n = e / GBK, kk = e % GBK;
        int64_t gn = n0 + n, gk = k0 + kk;
        v = (gn < N && gk < K) ? p.B[gn * p.ldb + gk] : 0.f;
      } else {
        int kk = e / GBN, n = e % GBN;
        int64_t gn = n0 + n, gk = k0 + kk;
        v = (gn < N && gk < K) ? p.B[gk * p.ldb + gn] : 0.f;
      }
      b_reg[j] = p.abs_b ? fabsf(v) : v;
    }
  };

  auto store_tiles = [&](int buf, int64_t k0) {
#pragma unroll
    for (int j = 0; j < A_PER_T; ++j) {
      int r = a_r0 + 16 * j;
      float v = a_reg[j];
      if (PRO == PRO_RELAX) {
        int64_t m = m0 + r;
        int64_t k = k0 + a_kk;
        if (m < M && k < K) {
          const int64_t d = a_dom[j];
          float be = 0.f;
          float out = v;
          if (p.pre_lo) {
            const float l = p.pre_lo[d * p.ld_pre + k];
            const float u = p.pre_hi[d * p.ld_pre + k];
            float alpha = 0.f;
            const bool has_alpha = p.alpha != nullptr;
            if (has_alpha) alpha = clamp01(p.alpha[d * p.alpha_ld + k]);
            Relax rx = relu_relax(l, u, has_alpha, alpha);
            float sc = select_scale(v, rx, lower, &be);
            out = v * sc;
            if (lower && p.add_l) out = out + p.add_l[d * p.add_ld + k];
          }
          if (row_reduce) {
            s_beta[j] += v * be;
            if (p.kbias) s_bias[j] += out * p.kbias[k];
            if (p.cvec) s_cen[j] += out * p.cvec[d * p.cvec_ld + k];
          }
          v = out;
        } else {
          v = 0.f;
        }
      }
      As[buf][a_kk][r] = v;
    }
#pragma unroll
    for (int j = 0; j < B_PER_T; ++j) {
      int e = t + GNT * j;
      if (TRANS_B) {
        int n = e / GBK, kk = e % GBK;
        Bs[buf][kk][n] = b_reg[j];
      } else {
        int kk = e / GBN, n = e % GBN;
        Bs[buf][kk][n] = b_reg[j];
      }
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int64_t nk = ceil_div(K, GBK);
  load_tiles(0);
  store_tiles(0, 0);
  __syncthreads();
  int buf = 0;
  const int lrow = lane & 31;
  const int lk = lane >> 5;
  for (int64_t kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) load_tiles((kt + 1) * GBK);
#pragma unroll
    for (int kk = 0; kk < GBK; kk += 2) {
      float af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = As[buf][kk + lk][wm * 64 + i * 32 + lrow];
#pragma unroll
      for (int j = 0; j < 2; ++j) bfr[j] = Bs[buf][kk + lk][wn * 64 + j * 32 + lrow];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tiles(buf ^ 1, (kt + 1) * GBK);
    __syncthreads();
    buf ^= 1;
  }

  // Row reductions of the relaxation prologue: the 16 threads holding one row
  // are 16 consecutive lanes; reduce with xor shuffles in a fixed order.
  if (row_reduce) {
#pragma unroll
    for (int j = 0; j < A_PER_T; ++j) {
      float sb = s_beta[j], sk = s_bias[j], sc = s_cen[j];
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) {
        sb += __shfl_xor(sb, off, 64);
        sk += __shfl_xor(sk, off, 64);
        sc += __shfl_xor(sc, off, 64);
      }
      int64_t m = m0 + a_r0 + 16 * j;
      if (a_kk == 0 && m < M) {
        float b0 = p.b_in[z] ? p.b_in[z][m] : 0.f;
        if (p.b_out[z]) p.b_out[z][m] = (b0 + sb) + sk;
        if (p.c_out[z]) p.c_out[z][m] = sc;
      }
    }
  }

  if (EPI == EPI_STORE) {
    float* __restrict__ C = p.C[z];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = n0 + wn * 64 + j * 32 + lrow;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
          if (row < M && col < N) {
            float v = acc[i][j][r];
            if (p.r1_row) v = v + p.r1_row[row] * p.r1_col[(row / p.S) * p.r1_ld + col];
            C[row * p.ldc + col] = v;
          }
        }
      }
  } else {
    // sum_n |C[m, n]| * w[d, n] over this block's 128 columns, fixed order.
    float rs[2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int64_t col = n0 + wn * 64 + j * 32 + lrow;
          const float a = acc[i][j][r];
          float v = fabsf(a);
          float wgt = 1.f;
          if (p.wvec) {
            int64_t d = (row < M) ? row / p.S : 0;
            wgt = (row < M && col < N) ? p.wvec[d * p.w_ld + col] : 0.f;
            v = v * wgt;
          }
          s += v;
          if (lower && p.h_out && row < M && col < N) {
            const float sg = (a > 0.f) ? 1.f : ((a < 0.f) ? -1.f : 0.f);
            const float hs = p.h_scale[row];
            p.h_out[row * N + col] = p.wvec ? hs * sg * wgt : hs * sg;
          }
        }
        rs[i][r] = s;
      }
    // reduce across the 32 lanes that share a row set (lanes differ in column)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float s = rs[i][r];
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
        rs[i][r] = s;
      }
    if (lrow == 0) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rloc = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
          red[wn][rloc] = rs[i][r];
        }
    }
    __syncthreads();
    if (t < GBM) {
      int64_t row = m0 + t;
      if (row < M) p.partial[z][(int64_t)blockIdx.y * M + row] = red[0][t] + red[1][t];
    }
  }
}

// Fixed-order sum of the per-column-block partial norms, then
//   lb = (center - eps * norm) + b,   ub = (center + eps * norm) + b
// (perturbation.py:175-222; box: eps = 1 and the norm is already radius-weighted).
__global__ void concretize_finalize_kernel(const float* __restrict__ partial_u, const float* __restrict__ partial_l,
                                           int nparts, int64_t M, const float* __restrict__ cen_u,
                                           const float* __restrict__ cen_l, const float* __restrict__ b_u,
                                           const float* __restrict__ b_l, float eps, float* __restrict__ lb,
                                           float* __restrict__ ub) {
  int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  if (ub) {
    float nu = 0.f;
    for (int q = 0; q < nparts; ++q) nu += partial_u[(int64_t)q * M + m];
    ub[m] = (cen_u[m] + eps * nu) + b_u[m];
  }
  if (lb) {
    float nl = 0.f;
    for (int q = 0; q < nparts; ++q) nl += partial_l[(int64_t)q * M + m];
    lb[m] = (cen_l[m] - eps * nl) + b_l[m];
  }
}

template <int PRO, int EPI>
static int launch_gemm(const GemmArgs& a, int nz, hipStream_t stream) {
  dim3 grid((unsigned)ceil_div(a.M, GBM), (unsigned)ceil_div(a.N, GBN), (unsigned)nz);
  BF_REQUIRE(grid.x < (1u << 31) && grid.y <= 65535, "gemm grid too large (M=%lld N=%lld)", (long long)a.M,
             (long long)a.N);
  if (a.trans_b)
    hipLaunchKernelGGL((gemm_kernel<PRO, EPI, true>), grid, dim3(GNT), 0, stream, a);
  else
    hipLaunchKernelGGL((gemm_kernel<PRO, EPI, false>), grid, dim3(GNT), 0, stream, a);
  BF_LAUNCH_CHECK("gemm_kernel");
  return BF_OK;
}

int gemm_dispatch(const GemmArgs& a, int pro, int epi, int nz, hipStream_t stream) {
  if (pro == PRO_PLAIN && epi == EPI_STORE) return launch_gemm<PRO_PLAIN, EPI_STORE>(a, nz, stream);
  if (pro == PRO_RELAX && epi == EPI_STORE) return launch_gemm<PRO_RELAX, EPI_STORE>(a, nz, stream);
  if (pro == PRO_PLAIN && epi == EPI_ABSSUM) return launch_gemm<PRO_PLAIN, EPI_ABSSUM>(a, nz, stream);
  if (pro == PRO_RELAX && epi == EPI_ABSSUM) return launch_gemm<PRO_RELAX, EPI_ABSSUM>(a, nz, stream);
  set_error("gemm_dispatch: bad mode pro=%d epi=%d", pro, epi);
  return BF_EINVAL;
}

int concretize_finalize(const float* pu, const float* pl, int nparts, int64_t M, const float* cu, const float* cl,
                        const float* bu, const float* bl, float eps, float* lb, float* ub, hipStream_t stream) {
  if (M == 0) return BF_OK;
  hipLaunchKernelGGL(concretize_finalize_kernel, dim3((unsigned)ceil_div(M, 256)), dim3(256), 0, stream, pu, pl,
                     nparts, M, cu, cl, bu, bl, eps, lb, ub);
  BF_LAUNCH_CHECK("concretize_finalize_kernel");
  return BF_OK;
}

int gemm_partial_count(int64_t N) { return (int)ceil_div(N, GBN); }

}  // namespace bf
