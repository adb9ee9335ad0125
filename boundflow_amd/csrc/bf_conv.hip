// Conv2d kernels of the bound-propagation path (NCHW, groups = 1, dilation = 1).
//
// Both kernels work on "rows": one row is one (domain, spec) coefficient map
// or one input sample.  A workgroup owns one row; the row's input map is
// staged once in LDS and every output element of that row is computed from
// LDS, with weights read through the L1/L2 (they are a few KB).
//
// * conv2d_rows:  y[r] = conv2d(x[r / in_div], W or |W|) (+ s[r] * v[r / v_div]).
//   IBP in center/radius form (center with W, radius with |W|), the center
//   projection of the input (x0 conv W), and the gradient of a transposed
//   convolution (d/dA of conv_transpose2d(A, W) is conv2d(G, W)).
// * conv_transpose_rows: y[r] = conv_transpose2d(A[r], W), the CROWN backward
//   through a conv layer (boundflow/runtime/linear_operator.py:1067-1092), with
//   an optional fused concretization epilogue: the weighted |y| row sum (the
//   Linf / box norm) and, for the gradient pass, h = h_scale[r] * sign(y) * w.

#include "bf_common.h"

namespace bf {

constexpr int CT = 256;

__global__ void __launch_bounds__(CT)
conv2d_rows_kernel(const float* __restrict__ x, int64_t in_div, int Ci, int Hi, int Wi,
                   const float* __restrict__ W, int abs_w, int Co, int KH, int KW, int sh, int sw, int ph, int pw,
                   int Ho, int Wo, float* __restrict__ y, const float* __restrict__ rs, const float* __restrict__ v,
                   int64_t v_div, int64_t v_ld) {
  extern __shared__ float xs[];
  const int64_t r = blockIdx.x;
  const int nin = Ci * Hi * Wi;
  const float* __restrict__ xr = x + (r / in_div) * (int64_t)nin;
  for (int i = threadIdx.x; i < nin; i += CT) xs[i] = xr[i];
  __syncthreads();
  const int nout = Co * Ho * Wo;
  float* __restrict__ yr = y + r * (int64_t)nout;
  const float scale = rs ? rs[r] : 0.f;
  const float* __restrict__ vr = v ? v + (r / v_div) * v_ld : nullptr;
  for (int e = threadIdx.x; e < nout; e += CT) {
    const int co = e / (Ho * Wo);
    const int rem = e - co * Ho * Wo;
    const int ho = rem / Wo;
    const int wo = rem - ho * Wo;
    float acc = 0.f;
    for (int ci = 0; ci < Ci; ++ci) {
      const float* __restrict__ wp = W + ((int64_t)co * Ci + ci) * KH * KW;
      const float* __restrict__ xp = xs + ci * Hi * Wi;
      for (int kh = 0; kh < KH; ++kh) {
        const int hi = ho * sh - ph + kh;
        if (hi < 0 || hi >= Hi) continue;
        for (int kw = 0; kw < KW; ++kw) {
          const int wi = wo * sw - pw + kw;
          if (wi < 0 || wi >= Wi) continue;
          float w = wp[kh * KW + kw];
          if (abs_w) w = fabsf(w);
          acc += xp[hi * Wi + wi] * w;
        }
      }
    }
    if (rs) acc = acc + scale * vr[e];
    yr[e] = acc;
  }
}

__global__ void __launch_bounds__(CT)
conv_transpose_rows_kernel(const float* __restrict__ A_u, const float* __restrict__ A_l, int Co, int Ho, int Wo,
                           const float* __restrict__ W, int Ci, int KH, int KW, int sh, int sw, int ph, int pw,
                           int Hi, int Wi, float* __restrict__ y_u, float* __restrict__ y_l, int64_t S,
                           const float* __restrict__ wv, int64_t w_ld, float* __restrict__ norm_u,
                           float* __restrict__ norm_l, const float* __restrict__ h_scale, float* __restrict__ h_out) {
  extern __shared__ float as[];
  __shared__ float red[CT / 64];
  const int z = blockIdx.y;
  const bool lower = (A_u == nullptr) || (z == 1);
  const float* __restrict__ A = lower ? A_l : A_u;
  float* __restrict__ y = lower ? y_l : y_u;
  float* __restrict__ nrm = lower ? norm_l : norm_u;
  const int64_t r = blockIdx.x;
  const int nin = Co * Ho * Wo;
  const float* __restrict__ ar = A + r * (int64_t)nin;
  for (int i = threadIdx.x; i < nin; i += CT) as[i] = ar[i];
  __syncthreads();
  const int nout = Ci * Hi * Wi;
  const int64_t d = r / S;
  float s = 0.f;
  const float hs = (lower && h_out) ? h_scale[r] : 0.f;
  for (int e = threadIdx.x; e < nout; e += CT) {
    const int ci = e / (Hi * Wi);
    const int rem = e - ci * Hi * Wi;
    const int hi = rem / Wi;
    const int wi = rem - hi * Wi;
    float acc = 0.f;
    for (int kh = 0; kh < KH; ++kh) {
      const int th = hi + ph - kh;
      if (th < 0 || th % sh) continue;
      const int ho = th / sh;
      if (ho >= Ho) continue;
      for (int kw = 0; kw < KW; ++kw) {
        const int tw = wi + pw - kw;
        if (tw < 0 || tw % sw) continue;
        const int wo = tw / sw;
        if (wo >= Wo) continue;
        for (int co = 0; co < Co; ++co)
          acc += as[(co * Ho + ho) * Wo + wo] * W[(((int64_t)co * Ci + ci) * KH + kh) * KW + kw];
      }
    }
    if (y) y[r * (int64_t)nout + e] = acc;
    if (nrm) {
      const float wgt = wv ? wv[d * w_ld + e] : 1.f;
      s += wv ? fabsf(acc) * wgt : fabsf(acc);
      if (lower && h_out) {
        const float sg = (acc > 0.f) ? 1.f : ((acc < 0.f) ? -1.f : 0.f);
        h_out[r * (int64_t)nout + e] = wv ? hs * sg * wgt : hs * sg;
      }
    }
  }
  if (nrm) {
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int q = 0; q < CT / 64; ++q) t += red[q];
      nrm[r] = t;
    }
  }
}

int ibp_center_radius(const float* lo, const float* hi, int64_t n, int apply_relu, float* mid, float* rad,
                      hipStream_t stream);
int ibp_finalize(const float* c, const float* r, const float* rownorm, float eps, const float* bias,
                 int64_t bias_div, const int8_t* split, int64_t split_ld, int64_t B, int64_t N, float* lo, float* hi,
                 int* infeasible, hipStream_t stream);
int fill_value(float* p, int64_t n, float v, hipStream_t stream);

static int conv2d_launch(const float* x, int64_t in_div, int64_t R, int Ci, int Hi, int Wi, const float* W, int abs_w,
                         int Co, int KH, int KW, int sh, int sw, int ph, int pw, int Ho, int Wo, float* y,
                         const float* rs, const float* v, int64_t v_div, int64_t v_ld, hipStream_t stream) {
  const size_t lds = sizeof(float) * (size_t)Ci * Hi * Wi;
  BF_REQUIRE(lds <= 64 * 1024, "conv2d: input map of %d x %d x %d exceeds the 64 KB LDS row stage", Ci, Hi, Wi);
  BF_REQUIRE(R < (1LL << 31), "conv2d: too many rows");
  hipLaunchKernelGGL(conv2d_rows_kernel, dim3((unsigned)R), dim3(CT), lds, stream, x, in_div, Ci, Hi, Wi, W, abs_w,
                     Co, KH, KW, sh, sw, ph, pw, Ho, Wo, y, rs, v, v_div, v_ld);
  BF_LAUNCH_CHECK("conv2d_rows_kernel");
  return BF_OK;
}

}  // namespace bf

using namespace bf;

extern "C" {

int bf_conv2d_rows(const float* x, int64_t in_div, int64_t R, int Ci, int Hi, int Wi, const float* W, int abs_w,
                   int Co, int KH, int KW, int sh, int sw, int ph, int pw, int Ho, int Wo, float* y,
                   const float* row_scale, const float* vec, int64_t vec_div, int64_t vec_ld, hipStream_t stream) {
  BF_REQUIRE(R >= 0 && Ci > 0 && Co > 0 && KH > 0 && KW > 0 && sh > 0 && sw > 0 && Ho > 0 && Wo > 0,
             "bf_conv2d_rows: bad sizes");
  if (R == 0) return BF_OK;
  BF_REQUIRE(x && W && y && in_div > 0, "bf_conv2d_rows: null pointer");
  BF_REQUIRE((row_scale == nullptr) == (vec == nullptr) && (vec == nullptr || vec_div > 0),
             "bf_conv2d_rows: rank-1 term needs both row_scale and vec");
  return conv2d_launch(x, in_div, R, Ci, Hi, Wi, W, abs_w, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, y, row_scale, vec,
                       vec ? vec_div : 1, vec_ld, stream);
}

int bf_conv_transpose_rows(const float* A_u, const float* A_l, int64_t R, int Co, int Ho, int Wo, const float* W,
                           int Ci, int KH, int KW, int sh, int sw, int ph, int pw, int Hi, int Wi, float* y_u,
                           float* y_l, int64_t S, const float* wvec, int64_t w_ld, float* norm_u, float* norm_l,
                           const float* h_scale, float* h_out, hipStream_t stream) {
  BF_REQUIRE(R >= 0 && Co > 0 && Ci > 0 && KH > 0 && KW > 0 && sh > 0 && sw > 0 && Hi > 0 && Wi > 0 && S > 0,
             "bf_conv_transpose_rows: bad sizes");
  if (R == 0) return BF_OK;
  BF_REQUIRE(W && (A_u || A_l), "bf_conv_transpose_rows: null pointer");
  BF_REQUIRE((A_u == nullptr) == (y_u == nullptr && norm_u == nullptr) && (A_l == nullptr) == (y_l == nullptr && norm_l == nullptr),
             "bf_conv_transpose_rows: each given coefficient needs an output or a norm");
  BF_REQUIRE((h_out == nullptr) == (h_scale == nullptr) && (h_out == nullptr || norm_l != nullptr),
             "bf_conv_transpose_rows: h_out needs h_scale and the lower norm");
  const size_t lds = sizeof(float) * (size_t)Co * Ho * Wo;
  BF_REQUIRE(lds <= 64 * 1024, "bf_conv_transpose_rows: coefficient map exceeds the 64 KB LDS row stage");
  const unsigned nz = (A_u && A_l) ? 2u : 1u;
  hipLaunchKernelGGL(conv_transpose_rows_kernel, dim3((unsigned)R, nz), dim3(CT), lds, stream, A_u, A_l, Co, Ho, Wo,
                     W, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, y_u, y_l, S, wvec, w_ld, norm_u, norm_l, h_scale, h_out);
  BF_LAUNCH_CHECK("conv_transpose_rows_kernel");
  return BF_OK;
}

int bf_ibp_conv2d(const float* in_lo, const float* in_hi, int64_t B, int Ci, int Hi, int Wi, int input_kind,
                  float eps, int apply_relu, const float* W, const float* bias, int Co, int KH, int KW, int sh,
                  int sw, int ph, int pw, int Ho, int Wo, const int8_t* split, int64_t split_ld, float* workspace,
                  float* out_lo, float* out_hi, float* center_out, int* infeasible, hipStream_t stream) {
  // input_kind 0: interval [in_lo, in_hi] (through ReLU when apply_relu); 1: Linf ball of radius eps around in_lo
  BF_REQUIRE(B >= 0 && Ci > 0 && Co > 0, "bf_ibp_conv2d: bad sizes");
  if (B == 0) return BF_OK;
  BF_REQUIRE(in_lo && W && out_lo && out_hi && workspace, "bf_ibp_conv2d: null pointer");
  const int64_t nin = (int64_t)Ci * Hi * Wi;
  const int64_t nout = (int64_t)Co * Ho * Wo;
  // workspace: mid [B*nin], rad [B*nin], c [B*nout], r [B*nout]
  float* mid = workspace;
  float* rad = mid + B * nin;
  float* c = rad + B * nin;
  float* r = c + B * nout;
  float* cdst = center_out ? center_out : c;
  int rc;
  if (input_kind == 1) {
    // center x0 conv W; the radius map is eps everywhere inside the image (padding has none)
    rc = conv2d_launch(in_lo, 1, B, Ci, Hi, Wi, W, 0, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, cdst, nullptr, nullptr, 1, 0,
                       stream);
    if (rc) return rc;
    rc = fill_value(rad, B * nin, eps, stream);
    if (rc) return rc;
  } else {
    BF_REQUIRE(in_hi, "bf_ibp_conv2d: interval input needs in_hi");
    rc = ibp_center_radius(in_lo, in_hi, B * nin, apply_relu, mid, rad, stream);
    if (rc) return rc;
    rc = conv2d_launch(mid, 1, B, Ci, Hi, Wi, W, 0, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, cdst, nullptr, nullptr, 1, 0,
                       stream);
    if (rc) return rc;
  }
  rc = conv2d_launch(rad, 1, B, Ci, Hi, Wi, W, 1, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, r, nullptr, nullptr, 1, 0,
                     stream);
  if (rc) return rc;
  return ibp_finalize(cdst, r, nullptr, 0.f, bias, (int64_t)Ho * Wo, split, split_ld, B, nout, out_lo, out_hi,
                      infeasible, stream);
}

int64_t bf_ibp_conv2d_workspace(int64_t B, int64_t nin, int64_t nout) { return 2 * B * nin + 2 * B * nout; }

}  // extern "C"
