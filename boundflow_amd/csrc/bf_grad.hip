// Gradient kernels of alpha / alpha-beta CROWN (north-star kernel #5) and the
// optimiser bookkeeping that stays on the device.
//
// The objective is the lower bound; with G = dL/dlb (one value per
// coefficient row m = d*S + s) the reverse pass through one ReLU relaxation
// (boundflow/runtime/crown_ibp.py:1211-1298, lower half) is, per element,
//
//   A' = A * sel(A >= 0, alpha_l, alpha_u) + add;   b += A * sel(A >= 0, beta_l, beta_u)
//   dL/dA      = dL/dA' * sel(A >= 0, alpha_l, alpha_u) + G * sel(A >= 0, beta_l, beta_u)
//   dL/dalpha  = sum_s dL/dA' * A * 1(A >= 0)   on ambiguous neurons, where 0 <= alpha <= 1
//   dL/dbeta   = -s * 1(s != 0) * sum_s dL/dA'   (add = -beta * s * 1(s != 0),
//                boundflow/runtime/alpha_beta_crown.py:615-640)
//
// The selection itself is not differentiated (torch.where), the clamp passes
// the gradient on [0, 1] inclusive, as autograd does.

#include "bf_common.h"

namespace bf {

// One thread per (domain, neuron); the S rows of the domain are walked in
// order, so the reductions over specs are deterministic and reads of row m are
// coalesced across neurons.
__global__ void relu_grad_kernel(const float* __restrict__ g_out, const float* __restrict__ A, int64_t a_dstride,
                                 int64_t D, int64_t S, int64_t N, const float* __restrict__ lo,
                                 const float* __restrict__ hi, const float* __restrict__ alpha, int64_t alpha_ld,
                                 const float* __restrict__ G, const int8_t* __restrict__ split, int64_t split_ld,
                                 float* __restrict__ g_in, float* __restrict__ g_alpha, float* __restrict__ g_beta) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= D * N) return;
  const int64_t d = i / N, n = i % N;
  const float l = lo[d * N + n], u = hi[d * N + n];
  const bool has_alpha = alpha != nullptr;
  const float araw = has_alpha ? alpha[d * alpha_ld + n] : 0.f;
  const Relax r = relu_relax(l, u, has_alpha, clamp01(araw));
  const bool amb = (l < 0.f) && (u > 0.f);
  const bool pass = has_alpha && amb && (araw >= 0.f) && (araw <= 1.f);
  float ga = 0.f, gs = 0.f;
  // rows in groups of four: the loads of a group are issued together (more bytes in
  // flight per thread), the sums still run over s in order
  int64_t s = 0;
  for (; s + 4 <= S; s += 4) {
    float av[4], gv[4], Gv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t m = d * S + s + u;
      av[u] = A[d * a_dstride + (s + u) * N + n];
      gv[u] = g_out[m * N + n];
      Gv[u] = G[m];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t m = d * S + s + u;
      const bool nn = av[u] >= 0.f;
      const float sa = nn ? r.al : r.au;
      const float sb = nn ? r.bl : r.bu;
      g_in[m * N + n] = gv[u] * sa + Gv[u] * sb;
      if (nn) ga += gv[u] * av[u];
      gs += gv[u];
    }
  }
  for (; s < S; ++s) {
    const int64_t m = d * S + s;
    const float a = A[d * a_dstride + s * N + n];
    const float go = g_out[m * N + n];
    const bool nn = a >= 0.f;
    const float sa = nn ? r.al : r.au;
    const float sb = nn ? r.bl : r.bu;
    g_in[m * N + n] = go * sa + G[m] * sb;
    if (nn) ga += go * a;
    gs += go;
  }
  if (g_alpha) g_alpha[d * N + n] = pass ? ga : 0.f;
  if (g_beta) {
    const int8_t sp = split ? split[d * split_ld + n] : 0;
    g_beta[d * N + n] = sp ? -(float)sp * gs : 0.f;
  }
}

// dL/dA of the dense concretization of the lower bound (perturbation.py:175-222, 327-359):
//   lb[m] = A[m, :] . c[d, :] - sum_j w[d, j] |A[m, j]| + b[m],  w = eps (Linf) or the box radius,
//   g[m, j] = G[m] * c[d, j] + (G[m] * -w[d, j]) * sign(A[m, j])   (sign(0) = 0, as autograd's abs).
__global__ void concretize_dense_grad_kernel(const float* __restrict__ A, int64_t M, int64_t S, int64_t I,
                                             const float* __restrict__ cen, const float* __restrict__ rad, float eps,
                                             const float* __restrict__ G, float* __restrict__ g) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * I) return;
  const int64_t m = div_rows(i, I, M * I < (1LL << 31)), j = i - m * I;
  const int64_t e = div_rows(m, S, M < (1LL << 31)) * I + j;
  const float a = A[i];
  const float sg = (a > 0.f) ? 1.f : ((a < 0.f) ? -1.f : 0.f);
  const float w = rad ? rad[e] : eps;
  g[i] = G[m] * cen[e] + (G[m] * -w) * sg;
}

// The gradient of a row's L2 norm or of its max |.| (the dual norms of the L2 and
// L1 balls, perturbation.py:126-133 and 209-214) as autograd forms it, scaled by
// hs: hs * y / ||y||_2 (0 for a zero row, torch's norm backward), or
// hs * sign(y_j) / count on the entries with |y_j| == max |y| (amax's backward
// shares the gradient among ties).  One workgroup of 256 per row; the row is read
// twice (reduce, then write).
constexpr int kSeedThreads = 256;

__device__ __forceinline__ float lp_row_reduce(const float* __restrict__ y, int64_t I, int nk, float* cnt_out) {
  __shared__ float red[kSeedThreads / 64];
  __shared__ float redc[kSeedThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float s = 0.f;
  for (int64_t j = threadIdx.x; j < I; j += kSeedThreads) {
    const float v = y[j];
    s = nk == 1 ? fmaxf(s, fabsf(v)) : s + v * v;
  }
  s = nk == 1 ? wave_max_nonneg(s) : wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  float t = red[0];
  for (int q = 1; q < kSeedThreads / 64; ++q) t = nk == 1 ? fmaxf(t, red[q]) : t + red[q];
  float c = 0.f;
  if (nk == 1) {
    for (int64_t j = threadIdx.x; j < I; j += kSeedThreads) c += fabsf(y[j]) == t ? 1.f : 0.f;
    c = wave_sum(c);
    if (lane == 0) redc[wave] = c;
    __syncthreads();
    c = redc[0];
    for (int q = 1; q < kSeedThreads / 64; ++q) c += redc[q];
  }
  *cnt_out = c;
  return nk == 1 ? t : sqrtf(t);
}

__device__ __forceinline__ float lp_seed_value(float v, float nrm, float cnt, float hs, int nk) {
  if (nk == 2) return nrm > 0.f ? v * (hs / nrm) : 0.f;
  const float sg = (v > 0.f) ? 1.f : ((v < 0.f) ? -1.f : 0.f);
  return fabsf(v) == nrm ? sg * (hs / cnt) : 0.f;
}

// h[m, :] holds y = the input layer's coefficient row; replaced in place by the
// seed hs[m] * d norm(y) / dy.
__global__ void __launch_bounds__(kSeedThreads)
lp_seed_rows_kernel(float* __restrict__ h, int64_t I, const float* __restrict__ h_scale, int nk) {
  const int64_t m = blockIdx.x;
  float* y = h + m * I;
  float cnt;
  const float nrm = lp_row_reduce(y, I, nk, &cnt);
  const float hs = h_scale[m];
  for (int64_t j = threadIdx.x; j < I; j += kSeedThreads) y[j] = lp_seed_value(y[j], nrm, cnt, hs, nk);
}

// dL/dA of the dense concretization of the lower bound over an L2 or L1 ball:
//   g[m, j] = G[m] * c[d, j] + seed with hs = G[m] * -eps.
__global__ void __launch_bounds__(kSeedThreads)
concretize_dense_grad_lp_kernel(const float* __restrict__ A, int64_t S, int64_t I, const float* __restrict__ cen,
                                float eps, const float* __restrict__ G, float* __restrict__ g, int nk) {
  const int64_t m = blockIdx.x;
  const float* a = A + m * I;
  const float* c = cen + (m / S) * I;
  float cnt;
  const float nrm = lp_row_reduce(a, I, nk, &cnt);
  const float gm = G[m];
  const float hs = gm * -eps;
  for (int64_t j = threadIdx.x; j < I; j += kSeedThreads)
    g[m * I + j] = gm * c[j] + lp_seed_value(a[j], nrm, cnt, hs, nk);
}

int lp_seed_rows(float* h, int64_t M, int64_t I, const float* h_scale, int norm_p, hipStream_t stream) {
  if (M == 0) return BF_OK;
  BF_REQUIRE(M < (1LL << 31), "lp_seed_rows: too many rows");
  hipLaunchKernelGGL(lp_seed_rows_kernel, dim3((unsigned)M), dim3(kSeedThreads), 0, stream, h, I, h_scale, norm_p);
  BF_LAUNCH_CHECK("lp_seed_rows_kernel");
  return BF_OK;
}

// out[d, n] = max over the S rows of domain d of max(|A_u[m, n]|, |A_l[m, n]|) (either
// may be NULL): the objective influence of a ReLU, crown_ibp.py:1810-1833.
__global__ void rows_abs_max_kernel(const float* __restrict__ A_u, const float* __restrict__ A_l, int64_t D,
                                    int64_t S, int64_t N, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= D * N) return;
  const int64_t d = i / N, n = i - d * N;
  float v = 0.f;
  for (int64_t s = 0; s < S; ++s) {
    const int64_t e = (d * S + s) * N + n;
    if (A_u) v = fmaxf(v, fabsf(A_u[e]));
    if (A_l) v = fmaxf(v, fabsf(A_l[e]));
  }
  out[i] = v;
}

// out[m, n] = (a[m, n] + b[m, n]) + r_row[m] * vec[(m / S) * v_ld + n], each term optional;
// out may be a or b (elementwise, each element read before it is written).
__global__ void rows_add_kernel(const float* a, const float* b, int64_t M, int64_t N, int64_t S,
                                const float* __restrict__ r_row, const float* __restrict__ vec, int64_t v_ld,
                                float* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * N) return;
  float v = a ? a[i] : 0.f;
  if (b) v = a ? v + b[i] : b[i];
  if (r_row) {
    const int64_t m = i / N, n = i - (i / N) * N;
    v = v + r_row[m] * vec[(m / S) * v_ld + n];
  }
  out[i] = v;
}

// add[d, n] = -beta[d, n] * s[d, n] * 1(s != 0)
__global__ void beta_coeff_kernel(const float* __restrict__ beta, int64_t beta_ld, const int8_t* __restrict__ split,
                                  int64_t split_ld, int64_t D, int64_t N, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= D * N) return;
  const int64_t d = i / N, n = i % N;
  const int8_t s = split[d * split_ld + n];
  const float sf = (float)s;
  out[i] = (-beta[d * beta_ld + n] * sf) * (s != 0 ? 1.f : 0.f);
}

// Per-domain best-of tracking (boundflow/runtime/alpha_beta_crown.py:840-876):
// metric = mean over specs of the lower bound; on the first call or when the
// metric strictly improves, keep the bounds and flag the domain.
__global__ void best_update_kernel(const float* __restrict__ lb, const float* __restrict__ ub, int64_t D, int64_t S,
                                   float* __restrict__ best_metric, float* __restrict__ best_lb,
                                   float* __restrict__ best_ub, int* __restrict__ improved, int first) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= D) return;
  float sum = 0.f;
  for (int64_t s = 0; s < S; ++s) sum += lb[d * S + s];
  const float metric = sum / (float)S;
  const bool take = first || (metric > best_metric[d]);
  improved[d] = take ? 1 : 0;
  if (take) {
    best_metric[d] = metric;
    for (int64_t s = 0; s < S; ++s) best_lb[d * S + s] = lb[d * S + s];
    if (ub)
      for (int64_t s = 0; s < S; ++s) best_ub[d * S + s] = ub[d * S + s];
  }
}

// Spec reductions of the optimisation objective (alpha_beta_crown.py:787-815) over
// the S specs of one domain: mean; min / max (first index on ties, as torch's
// min/max over a dimension); softmin -tau log sum exp(-x / tau) / softmax
// tau log sum exp(x / tau), with the max-shifted log-sum-exp.  ``dir`` -1 is
// the min direction, +1 the max direction; ``w`` receives dR/dx_s.
__device__ float spec_reduce(const float* x, int64_t S, int reduce, int dir, float tau, float* w) {
  if (reduce == 0) {
    // the 1/S of the mean is applied by the caller, after the upstream factor (torch's
    // MeanBackward divides the incoming gradient by S)
    float sum = 0.f;
    for (int64_t s = 0; s < S; ++s) sum += x[s];
    for (int64_t s = 0; s < S; ++s) w[s] = 1.f;
    return sum / (float)S;
  }
  if (reduce == 1) {
    int64_t best = 0;
    for (int64_t s = 1; s < S; ++s)
      if (dir < 0 ? x[s] < x[best] : x[s] > x[best]) best = s;
    for (int64_t s = 0; s < S; ++s) w[s] = (s == best) ? 1.f : 0.f;
    return x[best];
  }
  // softmin / softmax through v = dir * x / tau
  float m = -INFINITY;
  for (int64_t s = 0; s < S; ++s) m = fmaxf(m, (dir < 0 ? -x[s] : x[s]) / tau);
  float se = 0.f;
  for (int64_t s = 0; s < S; ++s) se += expf((dir < 0 ? -x[s] : x[s]) / tau - m);
  const float lse = m + logf(se);
  for (int64_t s = 0; s < S; ++s) w[s] = expf((dir < 0 ? -x[s] : x[s]) / tau - lse);
  return dir < 0 ? -tau * lse : tau * lse;
}

constexpr int kObjMaxSpecs = 64;

// One domain per thread: the objective metric of alpha_beta_crown.py:787-815 from the
// lower bound lb [D, S] of C and nub [D, S], the lower bound of -C (= -ub), the
// per-row loss gradients G_l = dL/dlb and G_nu = dL/dnub for L = g_scale * sum_d
// metric_d (g_scale = -1 per domain, -1/D shared), and the per-domain best-of
// update (first call, or a strictly larger metric) of the metric and both bounds.
// objective 0 lower: R_min(lb); 1 upper: -R_max(ub); 2 gap: -R_max(ub - lb);
// 3 both: w_lb R_min(lb) - w_ub R_max(ub).
__global__ void objective_step_kernel(const float* __restrict__ lb, const float* __restrict__ nub, int64_t D,
                                      int64_t S, int objective, int reduce, float tau, float w_lb, float w_ub,
                                      float g_scale, float* __restrict__ metric_out, float* __restrict__ G_l,
                                      float* __restrict__ G_nu, float* __restrict__ best_metric,
                                      float* __restrict__ best_lb, float* __restrict__ best_ub,
                                      int* __restrict__ improved, int first) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= D) return;
  float x[kObjMaxSpecs], w1[kObjMaxSpecs], w2[kObjMaxSpecs];
  const float* l = lb ? lb + d * S : nullptr;
  const float* nu = nub ? nub + d * S : nullptr;
  float metric = 0.f;
  for (int64_t s = 0; s < S; ++s) {
    w1[s] = 0.f;
    w2[s] = 0.f;
  }
  if (objective == 0) {
    metric = spec_reduce(l, S, reduce, -1, tau, w1);                      // dmetric/dlb = w1
  } else if (objective == 1) {
    for (int64_t s = 0; s < S; ++s) x[s] = -nu[s];
    metric = -spec_reduce(x, S, reduce, +1, tau, w2);
    for (int64_t s = 0; s < S; ++s) w2[s] = -w2[s];                       // dmetric/dub
  } else if (objective == 2) {
    for (int64_t s = 0; s < S; ++s) x[s] = -nu[s] - l[s];
    metric = -spec_reduce(x, S, reduce, +1, tau, w2);
    for (int64_t s = 0; s < S; ++s) {
      w1[s] = w2[s];                                                        // dmetric/dlb
      w2[s] = -w2[s];                                                       // dmetric/dub
    }
  } else {
    const float rl = spec_reduce(l, S, reduce, -1, tau, w1);
    for (int64_t s = 0; s < S; ++s) x[s] = -nu[s];
    const float ru = spec_reduce(x, S, reduce, +1, tau, w2);
    metric = w_lb * rl - w_ub * ru;
    for (int64_t s = 0; s < S; ++s) {
      w1[s] = w_lb * w1[s];
      w2[s] = -(w_ub * w2[s]);
    }
  }
  metric_out[d] = metric;
  const float div = reduce == 0 ? (float)S : 1.f;
  for (int64_t s = 0; s < S; ++s) {
    if (G_l) G_l[d * S + s] = (g_scale * w1[s]) / div;
    if (G_nu) G_nu[d * S + s] = -((g_scale * w2[s]) / div);                // dL/dnub = -dL/dub
  }
  if (best_metric) {
    const bool take = first || (metric > best_metric[d]);
    improved[d] = take ? 1 : 0;
    if (take) {
      best_metric[d] = metric;
      if (l && best_lb)
        for (int64_t s = 0; s < S; ++s) best_lb[d * S + s] = l[s];
      if (nu && best_ub)
        for (int64_t s = 0; s < S; ++s) best_ub[d * S + s] = -nu[s];
    }
  }
}

// x[m, :] *= scale[m] (a concretization gradient seed formed with unit row weights)
__global__ void scale_rows_kernel(float* __restrict__ x, int64_t M, int64_t N, const float* __restrict__ scale) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * N) return;
  x[i] = scale[div_rows(i, N, M * N < (1LL << 31))] * x[i];
}

__global__ void masked_copy_rows_kernel(float* __restrict__ dst, const float* __restrict__ src, int64_t D, int64_t N,
                                        const int* __restrict__ mask) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= D * N) return;
  if (mask[i / N]) dst[i] = src[i];
}

// out[n] = sum_d x[d, n] in domain order (gradient of a parameter shared by all domains)
__global__ void sum_rows_kernel(const float* __restrict__ x, int64_t D, int64_t N, float* __restrict__ out) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float s = 0.f;
  for (int64_t d = 0; d < D; ++d) s += x[d * N + n];
  out[n] = s;
}

// "alpha from CROWN" initialisation
// (boundflow/runtime/native_alpha_beta_optimizer_schedule.py:635-653):
// 1 on stable-active neurons, 1(u > -l) on ambiguous ones, 0 otherwise.
__global__ void alpha_from_crown_kernel(const float* __restrict__ lo, const float* __restrict__ hi, int64_t n,
                                        float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float l = lo[i], u = hi[i];
  const bool pos = l >= 0.f;
  const bool neg = u <= 0.f;
  float a = 0.f;
  if (pos) a = 1.f;
  if (!pos && !neg) a = (u > -l) ? 1.f : 0.f;
  out[i] = a;
}

// The ADAPTIVE lower slope of the native plain-CROWN relaxation
// (boundflow/runtime/bound_ir_interpreter.py:1380-1397): on an ambiguous neuron
// 1 when the upper chord's slope u / max(u - l, eps) exceeds one half, else 0;
// 1 on stable-active, 0 on stable-inactive neurons.
__global__ void alpha_adaptive_kernel(const float* __restrict__ lo, const float* __restrict__ hi, int64_t n,
                                      float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float l = lo[i], u = hi[i];
  const bool pos = l >= 0.f;
  const bool neg = u <= 0.f;
  float a = 0.f;
  if (pos) a = 1.f;
  if (!pos && !neg) a = (u / fmaxf(u - l, kF32Eps) > 0.5f) ? 1.f : 0.f;
  out[i] = a;
}

// Branching rule of the native ReLU-split queue for one ReLU layer
// (native_relu_split_bab_runtime.py:1015-1049): per domain, the widest unsplit
// ambiguous neuron with the width u - l taken in double (the reference compares
// Python floats), the first index on ties; the running best is replaced only
// when strictly wider, so layers processed in sorted-name order win ties in
// that order.  One wave per domain.
__global__ void branch_update_native_kernel(const float* __restrict__ lo, const float* __restrict__ hi,
                                            const int8_t* __restrict__ split, int64_t split_ld, int64_t D, int64_t N,
                                            int layer, double* __restrict__ best_width, int* __restrict__ best_layer,
                                            int* __restrict__ best_idx, float* __restrict__ best_lo,
                                            float* __restrict__ best_hi) {
  const int lane = threadIdx.x & 63;
  const int64_t d = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (d >= D) return;
  double w = -1.0;
  int idx = -1;
  for (int64_t n = lane; n < N; n += 64) {
    const float l = lo[d * N + n], u = hi[d * N + n];
    const int8_t s = split ? split[d * split_ld + n] : (int8_t)0;
    if (s == 0 && l < 0.f && u > 0.f) {
      const double wd = (double)u - (double)l;
      if (wd > w) {
        w = wd;
        idx = (int)n;
      }
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const double ow = __shfl_xor(w, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (oi >= 0 && (idx < 0 || ow > w || (ow == w && oi < idx))) {
      w = ow;
      idx = oi;
    }
  }
  if (lane == 0 && idx >= 0 && w > best_width[d]) {
    best_width[d] = w;
    best_layer[d] = layer;
    best_idx[d] = idx;
    best_lo[d] = lo[d * N + idx];
    best_hi[d] = hi[d * N + idx];
  }
}

// BaB node verdict (boundflow/runtime/bab.py:870-895): a domain is closed when
// min_s lb >= threshold - tol; a domain whose split emptied a box is closed as
// infeasible.  status: 0 = open (to branch), 1 = certified, 2 = infeasible.
__global__ void domain_status_kernel(const float* __restrict__ lb, int64_t D, int64_t S,
                                     const int* __restrict__ infeasible, float threshold, float tol,
                                     int* __restrict__ status) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= D) return;
  if (infeasible && infeasible[d]) {
    status[d] = 2;
    return;
  }
  float mn = lb[d * S];
  for (int64_t s = 1; s < S; ++s) mn = fminf(mn, lb[d * S + s]);
  status[d] = (mn >= threshold - tol) ? 1 : 0;
}

}  // namespace bf

using namespace bf;

extern "C" {

int bf_relu_grad(const float* g_out, const float* A, int64_t a_dstride, int64_t D, int64_t S, int64_t N,
                 const float* pre_lo, const float* pre_hi, const float* alpha, int64_t alpha_ld, const float* G,
                 const int8_t* split, int64_t split_ld, float* g_in, float* g_alpha, float* g_beta,
                 hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0 && N > 0, "bf_relu_grad: bad sizes");
  if (D == 0) return BF_OK;
  BF_REQUIRE(g_out && A && pre_lo && pre_hi && G && g_in, "bf_relu_grad: null pointer");
  hipLaunchKernelGGL(relu_grad_kernel, dim3((unsigned)ceil_div(D * N, 256)), dim3(256), 0, stream, g_out, A,
                     a_dstride, D, S, N, pre_lo, pre_hi, alpha, alpha_ld, G, split, split_ld, g_in, g_alpha, g_beta);
  BF_LAUNCH_CHECK("relu_grad_kernel");
  return BF_OK;
}

int bf_rows_abs_max(const float* A_u, const float* A_l, int64_t D, int64_t S, int64_t N, float* out,
                    hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0 && N > 0, "bf_rows_abs_max: bad sizes");
  if (D == 0) return BF_OK;
  BF_REQUIRE((A_u || A_l) && out, "bf_rows_abs_max: null pointer");
  hipLaunchKernelGGL(rows_abs_max_kernel, dim3((unsigned)ceil_div(D * N, 256)), dim3(256), 0, stream, A_u, A_l, D, S,
                     N, out);
  BF_LAUNCH_CHECK("rows_abs_max_kernel");
  return BF_OK;
}

int bf_concretize_dense_grad(const float* A, int64_t D, int64_t S, int64_t I, const float* center, const float* rad,
                             float eps, int norm_p, const float* G, float* g, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0 && I > 0, "bf_concretize_dense_grad: bad sizes");
  BF_REQUIRE(norm_p >= 0 && norm_p <= 2 && (norm_p == 0 || rad == nullptr),
             "bf_concretize_dense_grad: norm_p is 0, 1 or 2; the box radius goes with 0");
  if (D == 0) return BF_OK;
  BF_REQUIRE(A && center && G && g, "bf_concretize_dense_grad: null pointer");
  if (norm_p != 0) {
    BF_REQUIRE(D * S < (1LL << 31), "bf_concretize_dense_grad: too many rows");
    hipLaunchKernelGGL(concretize_dense_grad_lp_kernel, dim3((unsigned)(D * S)), dim3(kSeedThreads), 0, stream, A, S,
                       I, center, eps, G, g, norm_p);
    BF_LAUNCH_CHECK("concretize_dense_grad_lp_kernel");
    return BF_OK;
  }
  const int64_t n = D * S * I;
  hipLaunchKernelGGL(concretize_dense_grad_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, A, D * S,
                     S, I, center, rad, eps, G, g);
  BF_LAUNCH_CHECK("concretize_dense_grad_kernel");
  return BF_OK;
}

int bf_rows_add(const float* a, const float* b, int64_t M, int64_t N, int64_t S, const float* r_row, const float* vec,
                int64_t v_ld, float* out, hipStream_t stream) {
  BF_REQUIRE(M >= 0 && N > 0 && S > 0 && v_ld >= 0, "bf_rows_add: bad sizes");
  if (M == 0) return BF_OK;
  BF_REQUIRE(out && (a || b || r_row), "bf_rows_add: null pointer");
  BF_REQUIRE(r_row == nullptr || vec != nullptr, "bf_rows_add: rank-1 term without its vector");
  hipLaunchKernelGGL(rows_add_kernel, dim3((unsigned)ceil_div(M * N, 256)), dim3(256), 0, stream, a, b, M, N, S,
                     r_row, vec, v_ld, out);
  BF_LAUNCH_CHECK("rows_add_kernel");
  return BF_OK;
}

int bf_beta_coeff(const float* beta, int64_t beta_ld, const int8_t* split, int64_t split_ld, int64_t D, int64_t N,
                  float* out, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && N >= 0, "bf_beta_coeff: bad sizes");
  if (D * N == 0) return BF_OK;
  BF_REQUIRE(beta && split && out, "bf_beta_coeff: null pointer");
  hipLaunchKernelGGL(beta_coeff_kernel, dim3((unsigned)ceil_div(D * N, 256)), dim3(256), 0, stream, beta, beta_ld,
                     split, split_ld, D, N, out);
  BF_LAUNCH_CHECK("beta_coeff_kernel");
  return BF_OK;
}

int bf_best_update(const float* lb, const float* ub, int64_t D, int64_t S, float* best_metric, float* best_lb,
                   float* best_ub, int* improved, int first, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0, "bf_best_update: bad sizes");
  if (D == 0) return BF_OK;
  BF_REQUIRE(lb && best_metric && best_lb && improved, "bf_best_update: null pointer");
  BF_REQUIRE((ub == nullptr) == (best_ub == nullptr), "bf_best_update: ub and best_ub must both be given or both be null");
  hipLaunchKernelGGL(best_update_kernel, dim3((unsigned)ceil_div(D, 256)), dim3(256), 0, stream, lb, ub, D, S,
                     best_metric, best_lb, best_ub, improved, first);
  BF_LAUNCH_CHECK("best_update_kernel");
  return BF_OK;
}

int bf_objective_step(const float* lb, const float* nub, int64_t D, int64_t S, int objective, int reduce, float tau,
                      float w_lb, float w_ub, float g_scale, float* metric, float* G_l, float* G_nu,
                      float* best_metric, float* best_lb, float* best_ub, int* improved, int first,
                      hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0, "bf_objective_step: bad sizes");
  if (D == 0) return BF_OK;
  if (S > kObjMaxSpecs) {
    set_error("bf_objective_step: %lld specs per domain above %d", (long long)S, kObjMaxSpecs);
    return BF_ERANGE;
  }
  BF_REQUIRE(objective >= 0 && objective <= 3 && reduce >= 0 && reduce <= 2, "bf_objective_step: bad mode");
  BF_REQUIRE(reduce != 2 || tau > 0.f, "bf_objective_step: soft_tau must be >0");
  BF_REQUIRE(metric && (objective == 1 || lb) && (objective == 0 || nub), "bf_objective_step: missing bound");
  BF_REQUIRE(best_metric == nullptr || improved != nullptr, "bf_objective_step: best-of needs the improved flags");
  hipLaunchKernelGGL(objective_step_kernel, dim3((unsigned)ceil_div(D, 64)), dim3(64), 0, stream, lb, nub, D, S,
                     objective, reduce, tau, w_lb, w_ub, g_scale, metric, G_l, G_nu, best_metric, best_lb, best_ub,
                     improved, first);
  BF_LAUNCH_CHECK("objective_step_kernel");
  return BF_OK;
}

int bf_scale_rows(float* x, int64_t M, int64_t N, const float* scale, hipStream_t stream) {
  BF_REQUIRE(M >= 0 && N >= 0, "bf_scale_rows: bad sizes");
  if (M * N == 0) return BF_OK;
  BF_REQUIRE(x && scale, "bf_scale_rows: null pointer");
  hipLaunchKernelGGL(scale_rows_kernel, dim3((unsigned)ceil_div(M * N, 256)), dim3(256), 0, stream, x, M, N, scale);
  BF_LAUNCH_CHECK("scale_rows_kernel");
  return BF_OK;
}

int bf_masked_copy_rows(float* dst, const float* src, int64_t D, int64_t N, const int* mask, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && N >= 0, "bf_masked_copy_rows: bad sizes");
  if (D * N == 0) return BF_OK;
  BF_REQUIRE(dst && src && mask, "bf_masked_copy_rows: null pointer");
  hipLaunchKernelGGL(masked_copy_rows_kernel, dim3((unsigned)ceil_div(D * N, 256)), dim3(256), 0, stream, dst, src,
                     D, N, mask);
  BF_LAUNCH_CHECK("masked_copy_rows_kernel");
  return BF_OK;
}

int bf_sum_rows(const float* x, int64_t D, int64_t N, float* out, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && N >= 0, "bf_sum_rows: bad sizes");
  if (N == 0) return BF_OK;
  BF_REQUIRE(x && out, "bf_sum_rows: null pointer");
  hipLaunchKernelGGL(sum_rows_kernel, dim3((unsigned)ceil_div(N, 256)), dim3(256), 0, stream, x, D, N, out);
  BF_LAUNCH_CHECK("sum_rows_kernel");
  return BF_OK;
}

int bf_domain_status(const float* lb, int64_t D, int64_t S, const int* infeasible, float threshold, float tol,
                     int* status, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0, "bf_domain_status: bad sizes");
  if (D == 0) return BF_OK;
  BF_REQUIRE(lb && status, "bf_domain_status: null pointer");
  hipLaunchKernelGGL(domain_status_kernel, dim3((unsigned)ceil_div(D, 256)), dim3(256), 0, stream, lb, D, S,
                     infeasible, threshold, tol, status);
  BF_LAUNCH_CHECK("domain_status_kernel");
  return BF_OK;
}

int bf_alpha_adaptive(const float* lo, const float* hi, int64_t n, float* out, hipStream_t stream) {
  BF_REQUIRE(n >= 0, "bf_alpha_adaptive: bad size");
  if (n == 0) return BF_OK;
  BF_REQUIRE(lo && hi && out, "bf_alpha_adaptive: null pointer");
  hipLaunchKernelGGL(alpha_adaptive_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, lo, hi, n, out);
  BF_LAUNCH_CHECK("alpha_adaptive_kernel");
  return BF_OK;
}

int bf_branch_update_native(const float* lo, const float* hi, const int8_t* split, int64_t split_ld, int64_t D,
                            int64_t N, int layer, double* best_width, int* best_layer, int* best_idx, float* best_lo,
                            float* best_hi, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && N >= 0 && split_ld >= 0, "bf_branch_update_native: bad sizes");
  if (D == 0 || N == 0) return BF_OK;
  BF_REQUIRE(lo && hi && best_width && best_layer && best_idx && best_lo && best_hi,
             "bf_branch_update_native: null pointer");
  hipLaunchKernelGGL(branch_update_native_kernel, dim3((unsigned)ceil_div(D, 4)), dim3(256), 0, stream, lo, hi,
                     split, split_ld, D, N, layer, best_width, best_layer, best_idx, best_lo, best_hi);
  BF_LAUNCH_CHECK("branch_update_native_kernel");
  return BF_OK;
}

int bf_alpha_from_crown(const float* lo, const float* hi, int64_t n, float* out, hipStream_t stream) {
  BF_REQUIRE(n >= 0, "bf_alpha_from_crown: bad size");
  if (n == 0) return BF_OK;
  BF_REQUIRE(lo && hi && out, "bf_alpha_from_crown: null pointer");
  hipLaunchKernelGGL(alpha_from_crown_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, lo, hi, n, out);
  BF_LAUNCH_CHECK("alpha_from_crown_kernel");
  return BF_OK;
}

}  // extern "C"
