// First-layer split infeasibility certificate of branch-and-bound nodes.
//
// A node's splits on a ReLU whose input is an affine function of the network
// input give halfspaces s_i * (r_i . x + c_i) >= 0 (r_i a row of the layer's
// weight, or of the conv's Jacobian; c_i its bias).  If no x of the input set
// satisfies all of them, some convex combination w of the halfspaces has a
// negative maximum over the set:
//     max_x (sum_i w_i a_i) . x + sum_i w_i c_i  <  -tol     (a_i = s_i r_i, c_i = s_i b_i)
// which closes the node.  The search for w is the reference's: w = softmax(z)
// from z = 0, Adam (lr 0.1, betas 0.9 / 0.999, eps 1e-8) on the maximum,
// 200 steps, stopping at the first step whose maximum is below -tol
// (boundflow/runtime/alpha_beta_crown.py:391-532, halfspaces collected in
// op order then neuron order at :259-389).  The maximum over an Lp ball is
// a . x0 + eps * |a|_q + c with q the dual exponent (|a|_1 for Linf, |a|_2 for
// L2, max |a| for L1), over a box a . mid + |a| . rad + c
// (boundflow/runtime/perturbation.py:175-222, :327-359).
//
// One workgroup per node runs the whole search: the node's nonzero splits are
// compacted into LDS in neuron order, each step forms a = sum_i w_i a_i in LDS
// (every column summed over i in order), reduces the maximum, and takes the
// gradient dmax/dw_i = a_i . (x0 + eps * d|a|_q/da) + c_i (one wave per row),
// the softmax's backward and the Adam step on z.  Rows are read from the
// weight itself (L2-resident across steps); nothing is materialised per node.

#include "bf_common.h"

namespace bf {

constexpr int kCertThreads = 256;
constexpr int kCertMaxHalfspaces = 1024;
constexpr int kCertMaxSteps = 256;

// Adam's per-step scalars, computed on the host in double and rounded as torch does
struct CertAdamTable {
  float neg_step[kCertMaxSteps];   // -(lr / (1 - beta1^t))
  float bc2_sqrt[kCertMaxSteps];   // sqrt(1 - beta2^t)
};

__device__ __forceinline__ float block_sum_cert(float v, float* red) {
  // wave sums in a fixed order, then the four wave totals in order
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const float t = ((red[0] + red[1]) + red[2]) + red[3];
  return t;
}

__device__ __forceinline__ float block_max_cert(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float sign_f(float a) { return a > 0.f ? 1.f : (a < 0.f ? -1.f : 0.f); }

template <bool BOX>
__global__ __launch_bounds__(kCertThreads) void split_certificate_kernel(
    const float* __restrict__ rows, int64_t row_ld, const float* __restrict__ bias,
    const int8_t* __restrict__ split, int64_t split_ld, const float* __restrict__ center, int64_t center_ld,
    const float* __restrict__ rad, int64_t rad_ld, float eps, int nk, int n0, int in_dim, int steps, double tol,
    float w1, float b2, float w2, float adam_eps, CertAdamTable tab, int32_t* __restrict__ out,
    float* __restrict__ max_out) {
  extern __shared__ float a_vec[];                       // [in_dim]: the combined normal a
  __shared__ int h_idx[kCertMaxHalfspaces];              // neuron of each halfspace, in order
  __shared__ float h_sgn[kCertMaxHalfspaces];            // its split sign s_i
  __shared__ float z[kCertMaxHalfspaces], mz[kCertMaxHalfspaces], vz[kCertMaxHalfspaces];
  __shared__ float w[kCertMaxHalfspaces], g[kCertMaxHalfspaces];
  __shared__ float red[4];
  __shared__ int count_s;
  __shared__ int wave_cnt[4];

  const int node = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int8_t* sp = split + (int64_t)node * split_ld;
  const float* x0 = center + (int64_t)node * center_ld;
  const float* rr = BOX ? rad + (int64_t)node * rad_ld : nullptr;

  // 1. compact the nonzero splits in neuron order (chunks of 256, ballot prefix per wave)
  if (tid == 0) count_s = 0;
  __syncthreads();
  for (int base = 0; base < n0; base += kCertThreads) {
    const int i = base + tid;
    const int8_t s = (i < n0) ? sp[i] : (int8_t)0;
    const uint64_t mask = __ballot(s != 0);
    const int before = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[wave] = __popcll(mask);
    __syncthreads();
    int off = count_s;
    for (int k = 0; k < wave; ++k) off += wave_cnt[k];
    if (s != 0) {
      const int pos = off + before;
      if (pos < kCertMaxHalfspaces) {
        h_idx[pos] = i;
        h_sgn[pos] = (float)s;
      }
    }
    __syncthreads();
    if (tid == 0) count_s += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
  }
  const int m = count_s;
  if (m == 0) {                // no first-layer halfspace: nothing to certify
    if (tid == 0) {
      out[node] = 0;
      if (max_out) max_out[node] = 0.f;
    }
    return;
  }
  if (m > kCertMaxHalfspaces) {  // beyond the LDS stage: reported, the host raises
    if (tid == 0) {
      out[node] = -1;
      if (max_out) max_out[node] = 0.f;
    }
    return;
  }
  for (int i = tid; i < m; i += kCertThreads) {
    z[i] = 0.f;
    mz[i] = 0.f;
    vz[i] = 0.f;
  }
  __syncthreads();
  // a single halfspace: w = [1] at every step and its gradient through the
  // softmax is 0, so the first step decides (the reference's m == 1 case)
  const int n_steps = (m == 1) ? 1 : steps;
  int verdict = 0;
  float best = INFINITY;   // the smallest maximum seen (the certificate's value when it closes the node)
  for (int t = 0; t < n_steps; ++t) {
    // 2. w = softmax(z)
    float zmax = -INFINITY;
    for (int i = tid; i < m; i += kCertThreads) zmax = fmaxf(zmax, z[i]);
    zmax = block_max_cert(zmax, red);
    float esum = 0.f;
    for (int i = tid; i < m; i += kCertThreads) {
      const float e = expf(z[i] - zmax);
      w[i] = e;
      esum += e;
    }
    esum = block_sum_cert(esum, red);
    for (int i = tid; i < m; i += kCertThreads) w[i] = w[i] / esum;
    __syncthreads();
    // 3. a = sum_i w_i s_i r_i (each column summed over i in order) and the maximum
    // nk (Lp ball): 0 sum |a| (Linf), 2 the L2 norm, 1 max |a| (L1)
    float ct = 0.f, nrm = 0.f;
    for (int j = tid; j < in_dim; j += kCertThreads) {
      float acc = 0.f;
      for (int i = 0; i < m; ++i) acc += w[i] * (h_sgn[i] * rows[(int64_t)h_idx[i] * row_ld + j]);
      a_vec[j] = acc;
      ct += acc * x0[j];
      if (BOX) nrm += fabsf(acc) * rr[j];
      else nrm = nk == 1 ? fmaxf(nrm, fabsf(acc)) : nrm + (nk == 2 ? acc * acc : fabsf(acc));
    }
    ct = block_sum_cert(ct, red);
    nrm = (!BOX && nk == 1) ? block_max_cert(nrm, red) : block_sum_cert(nrm, red);
    if (!BOX && nk == 2) nrm = sqrtf(nrm);
    float ties = 1.f;   // L1: entries at max |a| share amax's gradient
    if (!BOX && nk == 1) {
      float cnt = 0.f;
      for (int j = tid; j < in_dim; j += kCertThreads) cnt += fabsf(a_vec[j]) == nrm ? 1.f : 0.f;
      ties = block_sum_cert(cnt, red);
    }
    float c = 0.f;
    if (bias != nullptr)
      for (int i = 0; i < m; ++i) c += w[i] * (h_sgn[i] * bias[h_idx[i]]);
    const float ub = BOX ? (ct + nrm) + c : (ct + eps * nrm) + c;
    best = fminf(best, ub);
    // compared in double, as the reference compares the Python float of the fp32 maximum
    if ((double)ub < -tol) {   // uniform over the workgroup
      verdict = 1;
      break;
    }
    if (t + 1 == n_steps) break;
    // 4. dub/dw_i = a_i . (x0 + eps * d|a|_q/da) + c_i, one wave per halfspace; d|a|_q/da is
    //    sign(a) (Linf), a / |a|_2 (L2, 0 at a = 0), sign(a) / ties on the maxima of |a| (L1)
    const float l2s = nrm > 0.f ? eps / nrm : 0.f;
    const float l1s = eps / ties;
    for (int i = wave; i < m; i += kCertThreads / 64) {
      const float* r = rows + (int64_t)h_idx[i] * row_ld;
      float acc = 0.f;
      for (int j = lane; j < in_dim; j += 64) {
        const float aj = a_vec[j];
        float ga;
        if (BOX) ga = x0[j] + sign_f(aj) * rr[j];
        else if (nk == 2) ga = x0[j] + aj * l2s;
        else if (nk == 1) ga = x0[j] + (fabsf(aj) == nrm ? sign_f(aj) * l1s : 0.f);
        else ga = x0[j] + eps * sign_f(aj);
        acc += (h_sgn[i] * r[j]) * ga;
      }
      acc = wave_sum(acc);
      if (lane == 0) g[i] = acc + (bias != nullptr ? h_sgn[i] * bias[h_idx[i]] : 0.f);
    }
    __syncthreads();
    // 5. softmax backward: dz_i = w_i * (g_i - sum_k g_k w_k)
    float gw = 0.f;
    for (int i = tid; i < m; i += kCertThreads) gw += g[i] * w[i];
    gw = block_sum_cert(gw, red);
    // 6. Adam on z (torch's single-tensor update order)
    const float neg_step = tab.neg_step[t], bc2 = tab.bc2_sqrt[t];
    for (int i = tid; i < m; i += kCertThreads) {
      const float gi = w[i] * (g[i] - gw);
      float mi = mz[i];
      mi = (w1 < 0.5f) ? fmaf(w1, gi - mi, mi) : fmaf(w1 - 1.0f, gi - mi, gi);
      float vi = vz[i] * b2;
      vi = vi + w2 * gi * gi;
      mz[i] = mi;
      vz[i] = vi;
      const float denom = sqrtf(vi) / bc2 + adam_eps;
      z[i] = z[i] + neg_step * mi / denom;
    }
    __syncthreads();
  }
  if (tid == 0) {
    out[node] = verdict;
    if (max_out) max_out[node] = best;
  }
}

}  // namespace bf

using namespace bf;

extern "C" int bf_split_certificate(const float* rows, int64_t row_ld, const float* bias, const int8_t* split,
                                    int64_t split_ld, const float* center, int64_t center_ld, const float* rad,
                                    int64_t rad_ld, float eps, int norm_p, int64_t nodes, int64_t n0, int64_t in_dim,
                                    int steps, double lr, double tol, int32_t* out, float* max_out,
                                    hipStream_t stream) {
  BF_REQUIRE(nodes >= 0 && n0 >= 0 && in_dim >= 1, "bf_split_certificate: bad sizes");
  BF_REQUIRE(norm_p >= 0 && norm_p <= 2 && (norm_p == 0 || rad == nullptr),
             "bf_split_certificate: norm_p is 0, 1 or 2; the box radius goes with 0");
  if (nodes == 0) return BF_OK;
  BF_REQUIRE(rows && split && center && out, "bf_split_certificate: null pointer");
  BF_REQUIRE(steps >= 1 && steps <= kCertMaxSteps, "bf_split_certificate: steps must be in [1, %d]", kCertMaxSteps);
  BF_REQUIRE(row_ld >= in_dim && (split_ld >= n0 || split_ld == 0) && (center_ld >= in_dim || center_ld == 0),
             "bf_split_certificate: bad leading dimensions");
  BF_REQUIRE(rad == nullptr || rad_ld >= in_dim || rad_ld == 0, "bf_split_certificate: bad radius stride");
  if (in_dim > 16384) {
    set_error("bf_split_certificate: input dimension %lld above 16384 (the LDS stage of the combined normal)",
              (long long)in_dim);
    return BF_ERANGE;
  }
  if (nodes > (1LL << 31) - 1) {
    set_error("bf_split_certificate: %lld nodes, above 2^31 - 1 (one workgroup per node)", (long long)nodes);
    return BF_ERANGE;
  }
  if (n0 > (1LL << 30)) {
    set_error("bf_split_certificate: %lld first-layer neurons, above 2^30 (32-bit split offsets)", (long long)n0);
    return BF_ERANGE;
  }
  CertAdamTable tab;
  const double beta1 = 0.9, beta2 = 0.999;
  for (int t = 0; t < steps; ++t) {
    // bias corrections in double then rounded, as torch computes them from Python floats
    const double bc1 = 1.0 - __builtin_pow(beta1, (double)(t + 1));
    const double bc2 = 1.0 - __builtin_pow(beta2, (double)(t + 1));
    tab.neg_step[t] = (float)(-(lr / bc1));
    tab.bc2_sqrt[t] = (float)__builtin_sqrt(bc2);
  }
  const float w1 = (float)(1.0 - beta1), w2 = (float)(1.0 - beta2);
  const size_t lds = (size_t)in_dim * sizeof(float);
  if (rad != nullptr)
    hipLaunchKernelGGL(split_certificate_kernel<true>, dim3((unsigned)nodes), dim3(kCertThreads), lds, stream, rows,
                       row_ld, bias, split, split_ld, center, center_ld, rad, rad_ld, 0.f, 0, (int)n0, (int)in_dim,
                       steps, tol, w1, (float)beta2, w2, 1e-8f, tab, out, max_out);
  else
    hipLaunchKernelGGL(split_certificate_kernel<false>, dim3((unsigned)nodes), dim3(kCertThreads), lds, stream, rows,
                       row_ld, bias, split, split_ld, center, center_ld, rad, rad_ld, eps, norm_p, (int)n0,
                       (int)in_dim, steps, tol, w1, (float)beta2, w2, 1e-8f, tab, out, max_out);
  BF_LAUNCH_CHECK("split_certificate_kernel");
  return BF_OK;
}
