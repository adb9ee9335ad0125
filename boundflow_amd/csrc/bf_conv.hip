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

#include <cstdlib>
#include <cstring>

#include "bf_common.h"

namespace bf {

constexpr int CT = 256;

// One output v's share of its row's concretization norm, by the input set:
// nk 0 sums |v| (Linf ball), or |v| * wgt when weighted (box radius wgt);
// nk 2 sums v * v (L2 ball: the root is taken by the finalize); nk 1 keeps
// max |v| (L1 ball).  The partial norms of a row combine with norm_join.
__device__ __forceinline__ float norm_step(float s, float v, float wgt, bool weighted, int nk) {
  const float a = fabsf(v);
  if (nk == 1) return fmaxf(s, a);
  if (nk == 2) return s + v * v;
  return s + (weighted ? a * wgt : a);
}

__device__ __forceinline__ float norm_join(float a, float b, int nk) { return nk == 1 ? fmaxf(a, b) : a + b; }

// norm_join over the 64 lanes of a wave by an xor butterfly, the total in every lane
__device__ __forceinline__ float norm_wave_xor(float s, int nk) {
  for (int off = 32; off >= 1; off >>= 1) s = norm_join(s, __shfl_xor(s, off, 64), nk);
  return s;
}

// STAGED: the row's input map is copied to LDS first (maps of at most 64 KB); otherwise
// the taps read it from global memory through the caches, for maps of any size.
template <bool STAGED>
__global__ void __launch_bounds__(CT)
conv2d_rows_kernel(const float* __restrict__ x, int64_t in_div, int Ci, int Hi, int Wi,
                   const float* __restrict__ W, int abs_w, int Co, int KH, int KW, int sh, int sw, int ph, int pw,
                   int Ho, int Wo, float* __restrict__ y, const float* __restrict__ rs, const float* __restrict__ v,
                   int64_t v_div, int64_t v_ld) {
  extern __shared__ float xs_lds[];
  const int64_t r = blockIdx.x;
  const int nin = Ci * Hi * Wi;
  const float* __restrict__ xr = x + (r / in_div) * (int64_t)nin;
  const float* xs = xr;
  if constexpr (STAGED) {
    for (int i = threadIdx.x; i < nin; i += CT) xs_lds[i] = xr[i];
    __syncthreads();
    xs = xs_lds;
  }
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

// STAGED as for conv2d_rows_kernel: the coefficient map in LDS, or read from global memory.
template <bool STAGED>
__global__ void __launch_bounds__(CT)
conv_transpose_rows_kernel(const float* __restrict__ A_u, const float* __restrict__ A_l, int Co, int Ho, int Wo,
                           const float* __restrict__ W, int Ci, int KH, int KW, int sh, int sw, int ph, int pw,
                           int Hi, int Wi, float* __restrict__ y_u, float* __restrict__ y_l, int64_t S,
                           const float* __restrict__ wv, int64_t w_ld, int nk, float* __restrict__ norm_u,
                           float* __restrict__ norm_l, const float* __restrict__ h_scale, float* __restrict__ h_out) {
  extern __shared__ float as_lds[];
  __shared__ float red[CT / 64];
  const int z = blockIdx.y;
  const bool lower = (A_u == nullptr) || (z == 1);
  const float* __restrict__ A = lower ? A_l : A_u;
  float* __restrict__ y = lower ? y_l : y_u;
  float* __restrict__ nrm = lower ? norm_l : norm_u;
  const int64_t r = blockIdx.x;
  const int nin = Co * Ho * Wo;
  const float* __restrict__ ar = A + r * (int64_t)nin;
  const float* as = ar;
  if constexpr (STAGED) {
    for (int i = threadIdx.x; i < nin; i += CT) as_lds[i] = ar[i];
    __syncthreads();
    as = as_lds;
  }
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
      s = norm_step(s, acc, wgt, wv != nullptr, nk);
      if (lower && h_out) {
        const float sg = (acc > 0.f) ? 1.f : ((acc < 0.f) ? -1.f : 0.f);
        h_out[r * (int64_t)nout + e] = wv ? hs * sg * wgt : hs * sg;
      }
    }
  }
  if (nrm) {
    s = norm_wave_xor(s, nk);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int q = 0; q < CT / 64; ++q) t = norm_join(t, red[q], nk);
      nrm[r] = t;
    }
  }
}

// ---------------------------------------------------------------------------
// Convolutions of rows on fp32 MFMA (v_mfma_f32_16x16x4f32) as gather-GEMMs.
//
// One row's input map is staged in LDS with a zero halo, so every operand
// gather is in bounds without checks, and the weights once per workgroup.
// Output pixels are grouped in classes; within a class,
//   out[n, pixel] = sum_k Wc[n, k] * map[koff[k] + poff(pixel)],
// computed as 16 (channel) x 16 (pixel) tiles per wave, D = Wc . gather.
//
// * MODE_T (conv_transpose2d of coefficient rows, KH % sh == 0, KW % sw == 0):
//   sh*sw parity classes (alpha, beta) = ((hi + ph) % sh, (wi + pw) % sw); in a
//   class y[ci, u, v] = sum_{co, a, b} A[co, u - a, v - b] W[co, ci, alpha + sh*a,
//   beta + sw*b], k = (co, a, b).  Epilogue: store, or the concretization norm
//   sum |y| * w and the gradient seed h = h_scale * sign(y) * w.
// * MODE_F (conv2d): one class, k = (ci, kh, kw),
//   y[co, ho, wo] = sum_k W[co, ci, kh, kw] x[ci, ho*sh - ph + kh, wo*sw - pw + kw]
//   (optionally |W|), plus the rank-1 term row_scale[r] * vec[(r / vec_div) * vec_ld + e].
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int GT = 256;
// threads of a gather-GEMM or tap-product workgroup: its waves share one LDS copy of the weights
constexpr int GTM = 512;
constexpr int GMAX_CLASSES = 16;
enum : int { MODE_T = 0, MODE_F = 1 };

// q = n / d for n, d < 2^16 as a multiply-high by m = ceil(2^32 / d): with
// m d = 2^32 + e (0 <= e < d), n m / 2^32 = n / d + n e / (d 2^32) and n e < 2^32,
// so the error never reaches the next integer.  d == 1 is kept apart (m would
// need 33 bits).  Every numerator below indexes an LDS array of at most 64 KB.
struct FastDiv {
  uint32_t m, d;
};
static FastDiv make_fdiv(int d) {
  FastDiv f;
  f.d = (uint32_t)d;
  f.m = d > 1 ? (uint32_t)((0x100000000ull + (uint64_t)d - 1) / (uint64_t)d) : 0u;
  return f;
}
__device__ __forceinline__ int fdivq(int n, FastDiv f) { return f.d == 1 ? n : (int)__umulhi((uint32_t)n, f.m); }

struct GatherClass {
  int np;              // pixels of the class
  int n2;              // pixels per class row: p -> (q1, q2) = (p / n2, p % n2)
  int poff0, s1, s2;   // padded-map offset of a pixel: poff0 + q1*s1 + q2*s2
  int out0, o1, o2;    // output-map offset of a pixel: out0 + q1*o1 + q2*o2
  int tbase;           // first task index of the class
};

struct GatherArgs {
  const float* X[2];   // input rows per blockIdx.y
  float* y[2];
  float* nrm[2];
  const float* W;
  int abs_w;           // MODE_F: bit z set -> operand pair z multiplies by |W|
  const float* wv;     // MODE_T norm weights [D, nout] (w_ld)
  int nkind;           // MODE_T norm: 0 sum |y| (weighted by wv), 2 sum y^2, 1 max |y|
  const float* h_scale;
  float* h_out;
  const float* rs;     // MODE_F rank-1 term
  const float* v;
  int64_t v_div, v_ld;
  int64_t R, S, w_ld, in_div;
  int rows_per_wg, z_lower_first;
  int Cm, Hm, Wm, Hp, Wp, pad_h, pad_w;   // input map and its padded LDS copy
  int Cin, KH, KW, sh, sw;                // W is [Co, Ci, KH, KW]; Cin = Ci
  int nch, HWout;                         // output channels and pixels per channel
  int nA, nB, T;                          // MODE_T taps per class
  int Kc, Kc4, npad, nblk, nclasses, ntasks;
  FastDiv f_kstride, f_npad, f_T, f_nB, f_sw, f_KHKW, f_KW, f_HpWp, f_Wp;   // staging index divisions
  FastDiv f_HWm, f_Wm;                    // channel-last staging: divisions by Hm*Wm and Wm
  FastDiv f_Kc4;                          // MODE_F weight staging in source order: division by Kc4
  const float* wpack;                     // channel-last: weights already in LDS order (or null)
  // MODE_F interval input (IBP): 0 X[z] as given; IVL_BOX X[0] = lo, ivl_hi = hi, operand z = 0
  // the center (l + u) / 2, z = 1 the radius (u - l) / 2 (IVL_RELU: of max(., 0)); IVL_BALL
  // z = 0 X[0], z = 1 ivl_eps inside the map (the padding stays zero)
  int ivl;
  const float* ivl_hi;
  float ivl_eps;
  GatherClass cls[GMAX_CLASSES];
};
constexpr int IVL_BOX = 1, IVL_RELU = 2, IVL_BALL = 4;

static void gather_fdivs(GatherArgs& g) {
  g.f_kstride = make_fdiv(g.Kc4 * g.npad);
  g.f_npad = make_fdiv(g.npad);
  g.f_T = make_fdiv(g.T > 0 ? g.T : 1);
  g.f_nB = make_fdiv(g.nB > 0 ? g.nB : 1);
  g.f_sw = make_fdiv(g.sw);
  g.f_KHKW = make_fdiv(g.KH * g.KW);
  g.f_KW = make_fdiv(g.KW);
  g.f_HpWp = make_fdiv(g.Hp * g.Wp);
  g.f_Wp = make_fdiv(g.Wp);
  g.f_Kc4 = make_fdiv(g.Kc4 > 0 ? g.Kc4 : 1);
}

// LDS layout of the gather-GEMM operands.  The weights of class c, output channel n
// (block cb = n / 16, column col = n % 16) and reduction index k = j + 4 s
// (j = k % 4, the MFMA k lane group; s = 4 sq + e) live at
//   ((((c nblk + cb) 4 + j) (Kc4 / 16) + sq) 16 + col) 4 + e,
// so the four weights of steps 4 sq .. 4 sq + 3 of one lane are one 16-byte chunk and
// the 16 columns of a lane group read consecutive chunks; the map offsets of k are at
// (j (Kc4 / 16) + sq) 4 + e (the same for all 16 columns: a broadcast).  Kc4 is a
// multiple of 16.
__device__ __forceinline__ int ws_index(const GatherArgs& g, int c, int n, int k) {
  const int cb = n >> 4, col = n & 15, j = k & 3, s = k >> 2, sq = s >> 2, e = s & 3;
  return ((((c * g.nblk + cb) * 4 + j) * (g.Kc4 >> 4) + sq) * 16 + col) * 4 + e;
}
__device__ __forceinline__ int koff_index(const GatherArgs& g, int k) {
  const int j = k & 3, s = k >> 2;
  return (j * (g.Kc4 >> 4) + (s >> 2)) * 4 + (s & 3);
}

template <int MODE>
__global__ void __launch_bounds__(GTM)
conv_mfma_kernel(GatherArgs g) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Ws = smem;                                              // [nclasses][Kc4][npad]
  int* koff = reinterpret_cast<int*>(Ws + (size_t)g.nclasses * g.Kc4 * g.npad);   // [Kc4]
  float* As = reinterpret_cast<float*>(koff + g.Kc4);            // [Cm][Hp][Wp]
  __shared__ float red[GTM / 64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: task indices stay scalar
  const int z = blockIdx.y;
  const bool lower = g.z_lower_first ? (z == 0) : (z == 1);
  const float* __restrict__ X = g.X[z];
  float* __restrict__ y = g.y[z];
  float* __restrict__ nrm = g.nrm[z];
  const int kstride = g.Kc4 * g.npad;

  // weights of every class, zero-padded in k (to Kc4) and in channels (to npad);
  // eight loads per thread in flight, from clamped addresses, before the stores.
  // MODE_F (one class) walks them in the source order, k fastest, so a wave's loads
  // are consecutive floats of one output channel's row (W[n * Kc + k]), and scatters
  // them into the LDS order.
  const int wtotal = g.nclasses * kstride;
  auto w_coords = [&](int idx, int& c, int& k, int& n) {
    if (MODE == MODE_F) {
      c = 0;
      n = fdivq(idx, g.f_Kc4);
      k = idx - n * g.Kc4;
    } else {
      c = fdivq(idx, g.f_kstride);
      const int rem = idx - c * kstride;
      k = fdivq(rem, g.f_npad);
      n = rem - k * g.npad;
    }
  };
  for (int base = 0; base < wtotal; base += 8 * GTM) {
    float wv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = base + u * GTM + tid;
      int c, k, n;
      w_coords(idx, c, k, n);
      const bool ok = idx < wtotal && k < g.Kc && n < g.nch;
      int64_t src;
      if (MODE == MODE_T) {
        const int co = fdivq(k, g.f_T), t = k - co * g.T;
        const int a = fdivq(t, g.f_nB), b = t - a * g.nB;
        const int cr = fdivq(c, g.f_sw);
        const int kh = cr + g.sh * a, kw = (c - cr * g.sw) + g.sw * b;
        src = (((int64_t)co * g.Cin + n) * g.KH + kh) * g.KW + kw;
      } else {
        src = (int64_t)n * g.Kc + k;   // k = (ci * KH + kh) * KW + kw
      }
      float w = g.W[ok ? src : 0];
      if (MODE == MODE_F && ((g.abs_w >> z) & 1)) w = fabsf(w);
      wv[u] = ok ? w : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = base + u * GTM + tid;
      if (idx < wtotal) {
        int c, k, n;
        w_coords(idx, c, k, n);
        Ws[ws_index(g, c, n, k)] = wv[u];
      }
    }
  }
  for (int k = tid; k < g.Kc4; k += GTM) {
    int off = 0;
    if (k < g.Kc) {
      if (MODE == MODE_T) {
        const int co = fdivq(k, g.f_T), t = k - co * g.T;
        const int a = fdivq(t, g.f_nB), b = t - a * g.nB;
        off = co * g.Hp * g.Wp - a * g.Wp - b;
      } else {
        const int ci = fdivq(k, g.f_KHKW), t = k - ci * g.KH * g.KW;
        const int kh = fdivq(t, g.f_KW), kw = t - kh * g.KW;
        off = (ci * g.Hp + kh) * g.Wp + kw;
      }
    }
    koff[koff_index(g, k)] = off;
  }

  const int nin = g.Cm * g.Hm * g.Wm;
  const int64_t nout = (int64_t)g.nch * g.HWout;
  const int map = g.Cm * g.Hp * g.Wp;
  const int j = lane >> 4;     // k sub-index of the MFMA operands; output row group
  const int col = lane & 15;   // pixel column (B operand / D column); channel row (A operand)

  for (int i = 0; i < g.rows_per_wg; ++i) {
    const int64_t r = (int64_t)blockIdx.x * g.rows_per_wg + i;
    if (r >= g.R) break;   // uniform
    __syncthreads();       // weights staged / previous row's map and partial sums consumed
    const float* __restrict__ xr = X + (r / g.in_div) * nin;
    // interval input: the operand is made from the bounds as the map is staged (the
    // arithmetic of ibp_center_radius_kernel), uniform over the launch
    const int ivl = MODE == MODE_F ? g.ivl : 0;
    const float* __restrict__ hr_row = (ivl & IVL_BOX) ? g.ivl_hi + (r / g.in_div) * nin : nullptr;
    for (int base = 0; base < map; base += 8 * GTM) {
      float xv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int idx = base + u * GTM + tid;
        const int c = fdivq(idx, g.f_HpWp), rem = idx - c * g.Hp * g.Wp;
        const int hr = fdivq(rem, g.f_Wp);
        const int hm = hr - g.pad_h, wm = (rem - hr * g.Wp) - g.pad_w;
        const bool ok = idx < map && hm >= 0 && hm < g.Hm && wm >= 0 && wm < g.Wm;
        const int src = ok ? (c * g.Hm + hm) * g.Wm + wm : 0;
        float x;
        if (ivl & IVL_BOX) {
          float l = xr[src], h = hr_row[src];
          if (ivl & IVL_RELU) {
            l = fmaxf(l, 0.f);
            h = fmaxf(h, 0.f);
          }
          x = z == 0 ? (l + h) / 2.0f : (h - l) / 2.0f;
        } else if ((ivl & IVL_BALL) && z == 1) {
          x = g.ivl_eps;
        } else {
          x = xr[src];
        }
        xv[u] = ok ? x : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int idx = base + u * GTM + tid;
        if (idx < map) As[idx] = xv[u];
      }
    }
    __syncthreads();
    const int64_t d = r / g.S;
    const float hs = (MODE == MODE_T && lower && g.h_out) ? g.h_scale[r] : 0.f;
    const float rsv = (MODE == MODE_F && g.rs) ? g.rs[r] : 0.f;
    const float* __restrict__ vr = (MODE == MODE_F && g.rs) ? g.v + (r / g.v_div) * g.v_ld : nullptr;
    float s = 0.f;
    for (int task = wave; task < g.ntasks; task += GTM / 64) {
      int c = 0;
      while (c + 1 < g.nclasses && task >= g.cls[c + 1].tbase) ++c;
      const GatherClass& C = g.cls[c];
      const int tl = task - C.tbase;
      const int pt = tl / g.nblk, cb = tl - pt * g.nblk;
      const int p = pt * 16 + col;
      const bool pok = p < C.np;
      const int pc = pok ? p : C.np - 1;
      const int q1 = pc / C.n2, q2 = pc - q1 * C.n2;
      const float* __restrict__ as = As + C.poff0 + q1 * C.s1 + q2 * C.s2;
      // k = j + 4 s, s = 4 sq + e: one 128-bit LDS read gives this lane's weights of four
      // consecutive k steps, one broadcast read their map offsets
      const float* __restrict__ wl = Ws + ws_index(g, c, cb * 16 + col, j);
      const int* __restrict__ kl = koff + koff_index(g, j);
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      const int nq = g.Kc4 / 16;
#pragma unroll 2
      for (int sq = 0; sq < nq; ++sq) {
        const float4 w4 = *reinterpret_cast<const float4*>(wl + sq * 64);
        const int4 o4 = *reinterpret_cast<const int4*>(kl + sq * 4);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.x, as[o4.x], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.y, as[o4.y], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.z, as[o4.z], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.w, as[o4.w], acc, 0, 0, 0);
      }
      const int opix = C.out0 + q1 * C.o1 + q2 * C.o2;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int n = cb * 16 + 4 * j + rr;
        if (n < g.nch && pok) {
          float v = acc[rr];
          const int64_t oidx = (int64_t)n * g.HWout + opix;
          if (MODE == MODE_F && vr) v = v + rsv * vr[oidx];
          if (y) y[r * nout + oidx] = v;
          if (MODE == MODE_T && nrm) {
            const float wgt = g.wv ? g.wv[d * g.w_ld + oidx] : 1.f;
            s = norm_step(s, v, wgt, g.wv != nullptr, g.nkind);
            if (lower && g.h_out) {
              const float sg = (v > 0.f) ? 1.f : ((v < 0.f) ? -1.f : 0.f);
              g.h_out[r * nout + oidx] = g.wv ? hs * sg * wgt : hs * sg;
            }
          }
        }
      }
    }
    if (MODE == MODE_T && nrm) {
      s = norm_wave_xor(s, g.nkind);
      if (lane == 0) red[wave] = s;
      __syncthreads();
      if (tid == 0) {
        float t = 0.f;
        for (int q = 0; q < GTM / 64; ++q) t = norm_join(t, red[q], g.nkind);
        nrm[r] = t;
      }
    }
  }
}

// IBP of a conv layer in one launch: the forward gather-GEMM above with both products of
// the center/radius form taken together -- the row's center map and radius map staged
// side by side from the input set (IVL_BOX [| IVL_RELU] from lo / hi, or IVL_BALL from the
// center and eps, the arithmetic of conv_mfma_kernel<MODE_F>'s staging), each task running
// a center accumulator with W and a radius accumulator with |W| -- and the finalize of
// ibp_finalize_kernel applied to the two accumulators in registers:
//   lo = (c - r) + bias[ch],  hi = (c + r) + bias[ch],  then the consumer's split and the
//   infeasibility flag (crown_ibp.py:70-98); c to c_out when asked (the center projection).
// blockIdx.y halves a row's tasks: with an even number of 16-channel blocks, half y takes
// blocks [y nblk / 2, (y + 1) nblk / 2) and stages only their weights (CB_SPLIT); otherwise
// it takes the pixel tiles of parity y.
struct IbpConvOut {
  const float* bias;    // [nch] or null
  const int8_t* split;  // [R, nout] (split_ld) or null
  int64_t split_ld;
  float* lo;            // [R, nout]
  float* hi;
  float* c_out;         // [R, nout] or null
  int* infeasible;      // [R] or null
};

template <bool CB_SPLIT>
__global__ void __launch_bounds__(GTM)
conv_ibp_kernel(GatherArgs g, IbpConvOut o) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int half = blockIdx.y;
  const int nbl = CB_SPLIT ? g.nblk / 2 : g.nblk;   // channel blocks staged here
  const int cb0 = CB_SPLIT ? half * nbl : 0;
  const int nloc = nbl * 16;
  float* Ws = smem;                                                    // [Kc4][nloc] in ws order (nblk = nbl)
  int* koff = reinterpret_cast<int*>(Ws + (size_t)g.Kc4 * nloc);      // [Kc4]
  const int map = g.Cm * g.Hp * g.Wp;
  float* Mc = reinterpret_cast<float*>(koff + g.Kc4);                 // center map [Cm][Hp][Wp]
  float* Mr = Mc + map;                                                // radius map

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = g.Kc4 >> 4;
  auto ws_at = [&](int n, int k) {   // ws_index with nbl blocks
    const int cb = n >> 4, col = n & 15, j = k & 3, s = k >> 2, sq = s >> 2, e = s & 3;
    return (((cb * 4 + j) * kq + sq) * 16 + col) * 4 + e;
  };
  // weights of this half's channels in the source order (k fastest: consecutive floats of
  // one output channel's row), eight loads per thread in flight, scattered into the LDS order
  const int wtotal = g.Kc4 * nloc;
  for (int base = 0; base < wtotal; base += 8 * GTM) {
    float wv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = base + u * GTM + tid;
      const int n = fdivq(idx, g.f_Kc4), k = idx - n * g.Kc4;
      const int ch = 16 * cb0 + n;
      const bool ok = idx < wtotal && k < g.Kc && ch < g.nch;
      const float w = g.W[ok ? (int64_t)ch * g.Kc + k : 0];
      wv[u] = ok ? w : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = base + u * GTM + tid;
      if (idx < wtotal) {
        const int n = fdivq(idx, g.f_Kc4), k = idx - n * g.Kc4;
        Ws[ws_at(n, k)] = wv[u];
      }
    }
  }
  for (int k = tid; k < g.Kc4; k += GTM) {
    int off = 0;
    if (k < g.Kc) {
      const int ci = fdivq(k, g.f_KHKW), t = k - ci * g.KH * g.KW;
      const int kh = fdivq(t, g.f_KW), kw = t - kh * g.KW;
      off = (ci * g.Hp + kh) * g.Wp + kw;
    }
    koff[koff_index(g, k)] = off;
  }

  const int nin = g.Cm * g.Hm * g.Wm;
  const int64_t nout = (int64_t)g.nch * g.HWout;
  const int j = lane >> 4;
  const int col = lane & 15;
  const GatherClass& C = g.cls[0];
  const int npt = (C.np + 15) / 16;
  // tasks of this half: (pixel tile, local channel block)
  const int ntl = CB_SPLIT ? npt * nbl : ((npt - half + 1) / 2) * g.nblk;
  const bool box = (g.ivl & IVL_BOX) != 0, relu = (g.ivl & IVL_RELU) != 0;

  for (int i = 0; i < g.rows_per_wg; ++i) {
    const int64_t r = (int64_t)blockIdx.x * g.rows_per_wg + i;
    if (r >= g.R) break;   // uniform
    __syncthreads();       // weights staged / the previous row's maps consumed
    const float* __restrict__ xr = g.X[0] + r * nin;
    const float* __restrict__ hr_row = box ? g.ivl_hi + r * nin : nullptr;
    for (int base = 0; base < map; base += 8 * GTM) {
      float cv[8], rv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int idx = base + u * GTM + tid;
        const int c = fdivq(idx, g.f_HpWp), rem = idx - c * g.Hp * g.Wp;
        const int hr = fdivq(rem, g.f_Wp);
        const int hm = hr - g.pad_h, wm = (rem - hr * g.Wp) - g.pad_w;
        const bool ok = idx < map && hm >= 0 && hm < g.Hm && wm >= 0 && wm < g.Wm;
        const int src = ok ? (c * g.Hm + hm) * g.Wm + wm : 0;
        float cx, rx;
        if (box) {
          float l = xr[src], h = hr_row[src];
          if (relu) {
            l = fmaxf(l, 0.f);
            h = fmaxf(h, 0.f);
          }
          cx = (l + h) / 2.0f;
          rx = (h - l) / 2.0f;
        } else {
          cx = xr[src];
          rx = g.ivl_eps;
        }
        cv[u] = ok ? cx : 0.f;
        rv[u] = ok ? rx : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int idx = base + u * GTM + tid;
        if (idx < map) {
          Mc[idx] = cv[u];
          Mr[idx] = rv[u];
        }
      }
    }
    __syncthreads();
    for (int tl = wave; tl < ntl; tl += GTM / 64) {
      int pt, cbl;
      if (CB_SPLIT) {
        pt = tl / nbl;
        cbl = tl - pt * nbl;
      } else {
        const int q = tl / g.nblk;
        cbl = tl - q * g.nblk;
        pt = 2 * q + half;
      }
      const int p = pt * 16 + col;
      const bool pok = p < C.np;
      const int pc = pok ? p : C.np - 1;
      const int q1 = pc / C.n2, q2 = pc - q1 * C.n2;
      const int moff = C.poff0 + q1 * C.s1 + q2 * C.s2;
      const float* __restrict__ mc = Mc + moff;
      const float* __restrict__ mr = Mr + moff;
      const float* __restrict__ wl = Ws + ws_at(cbl * 16 + col, j);
      const int* __restrict__ kl = koff + koff_index(g, j);
      floatx4 acc_c = {0.f, 0.f, 0.f, 0.f};
      floatx4 acc_r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
      for (int sq = 0; sq < kq; ++sq) {
        const float4 w4 = *reinterpret_cast<const float4*>(wl + sq * 64);
        const int4 o4 = *reinterpret_cast<const int4*>(kl + sq * 4);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.x, mc[o4.x], acc_c, 0, 0, 0);
        acc_r = __builtin_amdgcn_mfma_f32_16x16x4f32(fabsf(w4.x), mr[o4.x], acc_r, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.y, mc[o4.y], acc_c, 0, 0, 0);
        acc_r = __builtin_amdgcn_mfma_f32_16x16x4f32(fabsf(w4.y), mr[o4.y], acc_r, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.z, mc[o4.z], acc_c, 0, 0, 0);
        acc_r = __builtin_amdgcn_mfma_f32_16x16x4f32(fabsf(w4.z), mr[o4.z], acc_r, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.w, mc[o4.w], acc_c, 0, 0, 0);
        acc_r = __builtin_amdgcn_mfma_f32_16x16x4f32(fabsf(w4.w), mr[o4.w], acc_r, 0, 0, 0);
      }
      const int opix = C.out0 + q1 * C.o1 + q2 * C.o2;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int n = 16 * (cb0 + cbl) + 4 * j + rr;
        if (n < g.nch && pok) {
          const float cvv = acc_c[rr], dev = acc_r[rr];
          const int64_t oidx = (int64_t)n * g.HWout + opix;
          float l = cvv - dev;
          float u = cvv + dev;
          if (o.bias) {
            l = l + o.bias[n];
            u = u + o.bias[n];
          }
          if (o.split) {
            const int8_t sp = o.split[r * o.split_ld + oidx];
            if (sp > 0) l = fmaxf(l, 0.f);
            if (sp < 0) u = fminf(u, 0.f);
            if (l > u && o.infeasible) o.infeasible[r] = 1;
          }
          o.lo[r * nout + oidx] = l;
          o.hi[r * nout + oidx] = u;
          if (o.c_out) o.c_out[r * nout + oidx] = cvv;
        }
      }
    }
  }
}

// conv_transpose2d of coefficient rows with the map channel-last in LDS (Co % 16 == 0).
//
// The row's map is staged as [Hp][Wp][CP] (channel pitch CP = Co + 4, zero halo
// written once per workgroup), so in parity class c the operand of output pixel
// (u, v) for tap (a, b) and channels co .. co + 3 is ONE float4 at
//   ((u + pad_h - a) Wp + (v + pad_w - b)) CP + co
// -- a lane-constant base plus a per-step uniform offset, with no offset table
// read in front of it.  The reduction index of a step quad q (T taps x Co / 16
// halves) is k = 16 q + 4 e + j for MFMA step e and lane group j, mapped to
// (tap ab = q / (Co / 16), channel co = 16 (q % (Co / 16)) + 4 j + e); the weights
// are staged in the same order (ws_index), one float4 per lane per quad.
//
// RELAX: the ReLU relaxation of the region is applied while the map is staged
// (the sign-split A+ pos + A- neg of runtime/linear_operator.py:722-905 and the
// dense ReLU backward of runtime/crown_ibp.py:1211-1298, slopes computed from the
// pre-activation box as bf_crown_relu_relax_lu does), with the row sums
//   b_out = (b_in + sum A * beta_sel) + sum A' * kbias
// reduced in the same pass; the relaxed rows are written out only when asked.
struct ConvRelax {
  const float* lo;       // pre-activation box [D, nin] of the ReLU (nin = Co*Ho*Wo)
  const float* hi;
  const float* alpha;    // lower-slope override, [D, nin] (alpha_ld nin) or shared (0); null = CROWN slopes
  int64_t alpha_ld;
  const float* add;      // lower bound: split term [D, nin] (add_ld)
  int64_t add_ld;
  const float* kbias;    // [nin] bias map of the conv whose output the ReLU reads
  const float* b_in[2];
  float* b_out[2];
  float* relaxed[2];     // optional A' rows [R, nin]
  const float* cvec;     // input layer only (conv_t_small_kernel): center projection [D, nin]
  float* c_out[2];       //   and its row sums sum A' * cvec
  const float* pl[4];    // conv_t_hwc_kernel: the relaxation as four planes [D, nin] {alpha_u, beta_u, alpha_l,
                         //   beta_l} (the executor's request), in place of the box; pl[0] null = from the box
};

// One element of a coefficient row through the ReLU relaxation (the sign-split
// transform and the dense backward's bias term; slopes from the pre-activation box
// as bf_crown_relu_relax_lu computes them): returns A', adds A * beta_sel to sb.
__device__ __forceinline__ float relax_element(const ConvRelax& rx, bool lower, float v, float lo, float hi, float al,
                                               float ad, float& sb) {
  float4 t = make_float4(1.f, 0.f, 1.f, 0.f);
  if (rx.lo) {
    const bool has_alpha = rx.alpha != nullptr;
    const Relax rr = relu_relax(lo, hi, has_alpha, has_alpha ? clamp01(al) : 0.f);
    t = make_float4(rr.au, rr.bu, rr.al, rr.bl);
  }
  const bool nn = v >= 0.f;
  float o;
  if (lower) {
    o = v * (nn ? t.z : t.x);
    sb += v * (nn ? t.w : t.y);
    if (rx.add) o = o + ad;
  } else {
    o = v * (nn ? t.x : t.z);
    sb += v * (nn ? t.y : t.w);
  }
  return o;
}

// Weights of every class of conv_t_hwc_kernel in the quad order of ws_index, zero-padded in
// k and channels: a float4 copy of the packed layout when the caller keeps one
// (conv_t_hwc_pack_kernel), else gathered from the OIHW tensor.
template <int NT>
__device__ __forceinline__ void hwc_stage_weights(const GatherArgs& g, float* Ws, int tid) {
  const int hq = g.Cm >> 4;
  const int kstride = g.Kc4 * g.npad;
  const int wtotal = g.nclasses * kstride;
  if (g.wpack) {
    for (int i4 = tid; i4 < wtotal / 4; i4 += NT)
      reinterpret_cast<float4*>(Ws)[i4] = reinterpret_cast<const float4*>(g.wpack)[i4];
  }
  for (int base = 0; base < wtotal && !g.wpack; base += 8 * NT) {
    float wv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = base + u * NT + tid;
      const int c = fdivq(idx, g.f_kstride), rem = idx - c * kstride;
      const int k = fdivq(rem, g.f_npad), n = rem - k * g.npad;
      const bool ok = idx < wtotal && k < g.Kc && n < g.nch;
      const int j = k & 3, q = k >> 4, e = (k >> 2) & 3;
      const int ab = q / hq, half = q - ab * hq;
      const int co = 16 * half + 4 * j + e;
      const int a = fdivq(ab, g.f_nB), b = ab - a * g.nB;
      const int cr = fdivq(c, g.f_sw);
      const int kh = cr + g.sh * a, kw = (c - cr * g.sw) + g.sw * b;
      const int64_t src = (((int64_t)co * g.Cin + n) * g.KH + kh) * g.KW + kw;
      const float w = g.W[ok ? src : 0];
      wv[u] = ok ? w : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = base + u * NT + tid;
      if (idx < wtotal) {
        const int c = fdivq(idx, g.f_kstride), rem = idx - c * kstride;
        const int k = fdivq(rem, g.f_npad), n = rem - k * g.npad;
        Ws[ws_index(g, c, n, k)] = wv[u];
      }
    }
  }
}

// The MFMA tasks of one coefficient row against its staged channel-last map Mp (every
// output pixel class, pixel block and output-channel block the wave owns), with the
// store / weighted-norm / gradient-seed epilogue; the norm terms accumulate in s.
__device__ __forceinline__ void hwc_row_tasks(const GatherArgs& g, const float* Ws, const float* Mp, int wave, int lane,
                                              int64_t r, int64_t d, bool lower, float* __restrict__ y,
                                              float* __restrict__ nrm, float hs, float& s) {
  const int CP = g.Cm + 4;
  const int hq = g.Cm >> 4;
  const int64_t nout = (int64_t)g.nch * g.HWout;
  const int j = lane >> 4;     // k lane group of the MFMA operands; output row group
  const int col = lane & 15;   // pixel column (B operand / D column); channel row (A operand)
  for (int task = wave; task < g.ntasks; task += GTM / 64) {
    int c = 0;
    while (c + 1 < g.nclasses && task >= g.cls[c + 1].tbase) ++c;
    const GatherClass& C = g.cls[c];
    const int tl = task - C.tbase;
    const int pt = tl / g.nblk, cb = tl - pt * g.nblk;
    const int p = pt * 16 + col;
    const bool pok = p < C.np;
    const int pc = pok ? p : C.np - 1;
    const int q1 = pc / C.n2, q2 = pc - q1 * C.n2;
    const float* __restrict__ mp = Mp + (C.poff0 + q1 * C.s1 + q2 * C.s2) * CP + 4 * j;
    const float* __restrict__ wl = Ws + ws_index(g, c, cb * 16 + col, j);
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    int q = 0;
    for (int a = 0; a < g.nA; ++a) {
      for (int b = 0; b < g.nB; ++b) {
        const float* __restrict__ tp = mp - (a * g.Wp + b) * CP;
        for (int half = 0; half < hq; ++half, ++q) {
          const float4 w4 = *reinterpret_cast<const float4*>(wl + q * 64);
          const float4 x4 = *reinterpret_cast<const float4*>(tp + 16 * half);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.x, x4.x, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.y, x4.y, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.z, x4.z, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w4.w, x4.w, acc, 0, 0, 0);
        }
      }
    }
    const int opix = C.out0 + q1 * C.o1 + q2 * C.o2;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int n = cb * 16 + 4 * j + rr;
      if (n < g.nch && pok) {
        const float v = acc[rr];
        const int64_t oidx = (int64_t)n * g.HWout + opix;
        if (y) y[r * nout + oidx] = v;
        if (nrm) {
          const float wgt = g.wv ? g.wv[d * g.w_ld + oidx] : 1.f;
          s = norm_step(s, v, wgt, g.wv != nullptr, g.nkind);
          if (lower && g.h_out) {
            const float sg = (v > 0.f) ? 1.f : ((v < 0.f) ? -1.f : 0.f);
            g.h_out[r * nout + oidx] = g.wv ? hs * sg * wgt : hs * sg;
          }
        }
      }
    }
  }
}

// The relaxation entry of element e of domain d for the channel-last staging: the four
// planes, or the slopes from the pre-activation box (and lower-slope override) as
// bf_crown_relu_relax_lu computes them; ad the lower bound's split term.
template <bool RELAX>
__device__ __forceinline__ void hwc_relax_operands(const ConvRelax& rx, bool lower, int nin, int64_t d, int e,
                                                   float4& t, float& ad) {
  t = make_float4(1.f, 0.f, 1.f, 0.f);
  ad = 0.f;
  if constexpr (RELAX) {
    if (rx.pl[0]) {
      const int64_t i = d * nin + e;
      t = make_float4(rx.pl[0][i], rx.pl[1][i], rx.pl[2][i], rx.pl[3][i]);
    } else if (rx.lo) {
      const float lo = rx.lo[d * nin + e], hi = rx.hi[d * nin + e];
      const bool has_alpha = rx.alpha != nullptr;
      const float al = has_alpha ? rx.alpha[d * rx.alpha_ld + e] : 0.f;
      const Relax rr = relu_relax(lo, hi, has_alpha, has_alpha ? clamp01(al) : 0.f);
      t = make_float4(rr.au, rr.bu, rr.al, rr.bl);
    }
    if (rx.add && lower) ad = rx.add[d * rx.add_ld + e];
  }
}

// One element e (CHW order) of coefficient row r relaxed (RELAX; t = {alpha_u, beta_u,
// alpha_l, beta_l}) into the channel-last map Mp, its bias terms added to sb and sk.
template <bool RELAX>
__device__ __forceinline__ void hwc_stage_element(const GatherArgs& g, const ConvRelax& rx, bool lower, int z,
                                                  float* Mp, int CP, int HWm, FastDiv f_hw, FastDiv f_w, int nin,
                                                  int64_t r, int e, float v, float4 t, float ad, float& sb,
                                                  float& sk) {
  const int co = fdivq(e, f_hw), rem = e - co * HWm;
  const int yy = fdivq(rem, f_w), xx = rem - yy * g.Wm;
  if constexpr (RELAX) {
    const bool nn = v >= 0.f;
    float o;
    if (lower) {
      o = v * (nn ? t.z : t.x);
      sb += v * (nn ? t.w : t.y);
      if (rx.add) o = o + ad;
    } else {
      o = v * (nn ? t.x : t.z);
      sb += v * (nn ? t.y : t.w);
    }
    if (rx.kbias) sk += o * rx.kbias[e];
    if (rx.relaxed[z]) rx.relaxed[z][r * nin + e] = o;
    v = o;
  }
  Mp[((yy + g.pad_h) * g.Wp + xx + g.pad_w) * CP + co] = v;
}

template <bool RELAX>
__global__ void __launch_bounds__(GTM)
conv_t_hwc_kernel(GatherArgs g, ConvRelax rx) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Ws = smem;                                                  // [nclasses][Kc4][npad] (ws_index order)
  float* Mp = Ws + (size_t)g.nclasses * g.Kc4 * g.npad;              // [Hp][Wp][CP]
  __shared__ float red[GTM / 64][2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: task indices stay scalar
  const int z = blockIdx.y;
  const bool lower = g.z_lower_first ? (z == 0) : (z == 1);
  const float* __restrict__ X = g.X[z];
  float* __restrict__ y = g.y[z];
  float* __restrict__ nrm = g.nrm[z];
  const int CP = g.Cm + 4;

  hwc_stage_weights<GTM>(g, Ws, tid);
  // zero halo (and channel padding): interior positions are rewritten per row, the rest stays zero
  const int mtotal = g.Hp * g.Wp * CP;
  for (int i = tid; i < mtotal; i += GTM) Mp[i] = 0.f;

  const int HWm = g.Hm * g.Wm;
  const int nin = g.Cm * HWm;
  const FastDiv f_hw = g.f_HWm;
  const FastDiv f_w = g.f_Wm;

  auto stage = [&](int64_t r, int64_t d, int e, float v, float4 t, float ad, float& sb, float& sk) {
    hwc_stage_element<RELAX>(g, rx, lower, z, Mp, CP, HWm, f_hw, f_w, nin, r, e, v, t, ad, sb, sk);
  };
  // The coefficients of rows of at most PF * GTM elements are fetched one row ahead,
  // into registers, so that their loads overlap the MFMAs of the row before (the
  // relaxation operands are per domain: the rows of a domain find them in cache).
  constexpr int PF = 4;
  const bool pf = nin <= PF * GTM;   // uniform
  float pa[PF];
  auto fetch = [&](int64_t r) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int e = tid + u * GTM;
      pa[u] = e < nin ? X[r * nin + e] : 0.f;
    }
  };
  auto relax_operands = [&](int64_t d, int e, float4& t, float& ad) {
    hwc_relax_operands<RELAX>(rx, lower, nin, d, e, t, ad);
  };
  const int64_t r_first = (int64_t)blockIdx.x * g.rows_per_wg;
  if (pf && r_first < g.R) fetch(r_first);

  for (int i = 0; i < g.rows_per_wg; ++i) {
    const int64_t r = (int64_t)blockIdx.x * g.rows_per_wg + i;
    if (r >= g.R) break;   // uniform
    __syncthreads();       // weights / halo staged; previous row's map and partial sums consumed
    const int64_t d = r / g.S;
    float sb = 0.f, sk = 0.f;
    if (pf) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int e = tid + u * GTM;
        if (e < nin) {
          float4 t;
          float ad;
          relax_operands(d, e, t, ad);
          stage(r, d, e, pa[u], t, ad, sb, sk);
        }
      }
    } else {
      for (int e = tid; e < nin; e += GTM) {
        float4 t;
        float ad;
        relax_operands(d, e, t, ad);
        stage(r, d, e, X[r * nin + e], t, ad, sb, sk);
      }
    }
    if constexpr (RELAX) {
      sb = wave_sum(sb);
      sk = wave_sum(sk);
      if (lane == 0) {
        red[wave][0] = sb;
        red[wave][1] = sk;
      }
    }
    __syncthreads();
    if constexpr (RELAX) {
      if (tid == 0 && rx.b_out[z]) {
        float tb = 0.f, tk = 0.f;
        for (int q = 0; q < GTM / 64; ++q) {
          tb += red[q][0];
          tk += red[q][1];
        }
        rx.b_out[z][r] = ((rx.b_in[z] ? rx.b_in[z][r] : 0.f) + tb) + tk;
      }
    }
    if (pf && i + 1 < g.rows_per_wg && r + 1 < g.R) fetch(r + 1);   // lands during this row's MFMAs
    const float hs = (lower && g.h_out) ? g.h_scale[r] : 0.f;
    float s = 0.f;
    hwc_row_tasks(g, Ws, Mp, wave, lane, r, d, lower, y, nrm, hs, s);
    if (nrm) {
      s = g.nkind == 1 ? wave_max_nonneg(s) : wave_sum(s);
      __syncthreads();   // red of the row sums above is read; reuse it
      if (lane == 0) red[wave][0] = s;
      __syncthreads();
      if (tid == 0) {
        float t = 0.f;
        for (int q2 = 0; q2 < GTM / 64; ++q2) t = norm_join(t, red[q2][0], g.nkind);
        nrm[r] = t;
      }
    }
  }
}


// The weights of conv_t_hwc_kernel in its LDS order (ws_index over classes, output
// channels and the quad-ordered reduction index), zero-padded: what each workgroup
// would otherwise gather from the OIHW tensor, computed once per weight.
__global__ void conv_t_hwc_pack_kernel(GatherArgs g, float* __restrict__ out) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const int kstride = g.Kc4 * g.npad;
  if (idx >= g.nclasses * kstride) return;
  const int hq = g.Cm >> 4;
  const int c = idx / kstride, rem = idx - c * kstride;
  const int k = rem / g.npad, n = rem - k * g.npad;
  float w = 0.f;
  if (k < g.Kc && n < g.nch) {
    const int j = k & 3, q = k >> 4, e = (k >> 2) & 3;
    const int ab = q / hq, half = q - ab * hq;
    const int co = 16 * half + 4 * j + e;
    const int a = ab / g.nB, b = ab - a * g.nB;
    const int cr = c / g.sw;
    const int kh = cr + g.sh * a, kw = (c - cr * g.sw) + g.sw * b;
    w = g.W[(((int64_t)co * g.Cin + n) * g.KH + kh) * g.KW + kw];
  }
  out[ws_index(g, c, n, k)] = w;
}

// conv_transpose2d of rows with few output channels (Ci <= 4, KH * KW <= 16),
// where the gather-GEMM above leaves most of its 16 MFMA channel rows idle.
// Per row and per output channel n, the taps are computed as one dense product
//   Z_n[(kh, kw), p] = sum_co W[co, n, kh, kw] * X[co, p]      (p: pixel of the Ho x Wo map)
// on v_mfma_f32_16x16x4f32 (16 tap rows, 16 pixels, 4 channels per step), kept
// in LDS, and each output pixel then gathers its taps (col2im):
//   y[n, oh, ow] = sum over (kh, kw) with ih = (oh + ph - kh) / sh, iw = (ow + pw - kw) / sw
//   integral and inside the map of Z_n[(kh, kw), (ih, iw)],
// followed by the store / weighted-norm / gradient-seed epilogue of conv_mfma_kernel.
struct SmallTArgs {
  const float* X[2];
  float* y[2];
  float* nrm[2];
  const float* W;          // [Co, Ci, KH, KW]
  const float* wv;         // norm weights [D, Ci*Hi*Wi] (w_ld) or NULL
  int nkind;               // norm: 0 sum |y| (weighted by wv), 2 sum y^2, 1 max |y|
  const float* h_scale;
  float* h_out;
  int64_t R, S, w_ld;
  int rows_per_wg, z_lower_first;
  int Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi;
  int Co4, npix, nblk;     // channels padded to 4, pixels Ho*Wo, 16-pixel blocks
  int vec;                 // rows copied as float4 (npix % 16 == 0 and 16-byte aligned row starts)
  FastDiv f_Wi, f_sh, f_sw, f_pitch;   // index divisions of the col2im and the map copy
  int pitchz, zsz;         // conv_t_small_fast_kernel: tap-row pitch of Z, floats per channel block
  float* bnd[2];           // conv_t_small_fast_kernel<relaxation>: the row's bound (c -/+ eps * norm) + b, or null
  float eps;
};

// RELAX: the input layer's ReLU relaxation applied while each row is staged, with
// the row sums b_out = (b_in + sum A * beta_sel) + sum A' * kbias and
// c_out = sum A' * cvec[d] reduced in the same pass (a wave sum per wave, then the
// waves in order) and the relaxed rows written only when asked.
template <bool RELAX>
__global__ void __launch_bounds__(GTM, 6)   // 6 waves per SIMD: three workgroups per CU
conv_t_small_kernel(SmallTArgs g, ConvRelax rx) {
  extern __shared__ float smem[];
  float* Wsm = smem;                                   // [Ci][Co4][16]: tap-fastest MFMA A operand
  float* Xs = Wsm + (size_t)g.Ci * g.Co4 * 16;          // [Co4][nblk * 16]
  float* Zs = Xs + (size_t)g.Co4 * g.nblk * 16;         // [16][nblk * 16]
  __shared__ float red[GTM / 64];
  __shared__ float rred[GTM / 64][3];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: task indices stay scalar
  const int z = blockIdx.y;
  const bool lower = g.z_lower_first ? (z == 0) : (z == 1);
  const float* __restrict__ X = g.X[z];
  float* __restrict__ y = g.y[z];
  float* __restrict__ nrm = g.nrm[z];
  const int taps = g.KH * g.KW;
  const int pitch = g.nblk * 16;
  const int nin = g.Co * g.npix;
  const int64_t nout = (int64_t)g.Ci * g.Hi * g.Wi;

  for (int idx = tid; idx < g.Ci * g.Co4 * 16; idx += GTM) {
    const int n = idx / (g.Co4 * 16), rem = idx - n * g.Co4 * 16;
    const int co = rem / 16, t = rem - co * 16;
    float w = 0.f;
    if (co < g.Co && t < taps) w = g.W[((int64_t)co * g.Ci + n) * taps + t];   // t = kh * KW + kw
    Wsm[idx] = w;
  }

  const int k4 = lane >> 4;    // k sub-index of the operands; row group of the result
  const int col = lane & 15;
  for (int i = 0; i < g.rows_per_wg; ++i) {
    const int64_t r = (int64_t)blockIdx.x * g.rows_per_wg + i;
    if (r >= g.R) break;   // uniform
    __syncthreads();       // weights staged / the previous row's maps consumed
    const float* __restrict__ xr = X + r * nin;
    const int64_t d = r / g.S;
    float sb = 0.f, sk = 0.f, sc = 0.f;
    // the row's (uniform) bases of the relaxation operands
    const float* __restrict__ lo_d = RELAX && rx.lo ? rx.lo + d * nin : nullptr;
    const float* __restrict__ hi_d = RELAX && rx.lo ? rx.hi + d * nin : nullptr;
    const float* __restrict__ al_d = RELAX && rx.alpha ? rx.alpha + d * rx.alpha_ld : nullptr;
    const float* __restrict__ ad_d = RELAX && rx.add ? rx.add + d * rx.add_ld : nullptr;
    const float* __restrict__ cv_d = RELAX && rx.cvec ? rx.cvec + d * nin : nullptr;
    float* __restrict__ rel_r = RELAX && rx.relaxed[z] ? rx.relaxed[z] + r * nin : nullptr;
    // element e of the row through the relaxation (RELAX), summed in each thread's order
    auto relax_at = [&](int e, float v) -> float {
      if constexpr (RELAX) {
        const float lo = rx.lo ? rx.lo[d * nin + e] : 0.f, hi = rx.lo ? rx.hi[d * nin + e] : 0.f;
        const float al = rx.alpha ? rx.alpha[d * rx.alpha_ld + e] : 0.f;
        const float ad = (rx.add && lower) ? rx.add[d * rx.add_ld + e] : 0.f;
        const float o = relax_element(rx, lower, v, lo, hi, al, ad, sb);
        if (rx.kbias) sk += o * rx.kbias[e];
        if (rx.cvec) sc += o * rx.cvec[d * nin + e];
        if (rx.relaxed[z]) rx.relaxed[z][r * nin + e] = o;
        return o;
      } else {
        return v;
      }
    };
    if (g.vec) {
      // unpadded map (npix % 16 == 0, 16-byte aligned rows): a float4 copy, then the zero channels
      const float4* __restrict__ x4 = reinterpret_cast<const float4*>(xr);
      float4* xs4 = reinterpret_cast<float4*>(Xs);
#pragma unroll 1
      for (int q = tid; q < nin / 4; q += GTM) {
        float4 v = x4[q];
        if constexpr (RELAX) {
          // the four elements' operands as float4 loads (16-byte aligned, checked by the host)
          const int e = 4 * q;
          const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
          auto ld4 = [](const float* p) { return *reinterpret_cast<const float4*>(p); };
          const float4 lo4 = rx.lo ? ld4(lo_d + e) : zero;
          const float4 hi4 = rx.lo ? ld4(hi_d + e) : zero;
          const float4 al4 = rx.alpha ? ld4(al_d + e) : zero;
          const float4 ad4 = (rx.add && lower) ? ld4(ad_d + e) : zero;
          const float vv[4] = {v.x, v.y, v.z, v.w}, lo[4] = {lo4.x, lo4.y, lo4.z, lo4.w},
                      hi[4] = {hi4.x, hi4.y, hi4.z, hi4.w}, al[4] = {al4.x, al4.y, al4.z, al4.w},
                      ad[4] = {ad4.x, ad4.y, ad4.z, ad4.w};
          float o[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) o[u] = relax_element(rx, lower, vv[u], lo[u], hi[u], al[u], ad[u], sb);
          // the bias and center operands after the relaxation (fewer registers live at once)
          __builtin_amdgcn_sched_barrier(0);
          const float4 kb4 = rx.kbias ? ld4(rx.kbias + e) : zero;
          const float4 cv4 = rx.cvec ? ld4(cv_d + e) : zero;
          const float kb[4] = {kb4.x, kb4.y, kb4.z, kb4.w}, cv[4] = {cv4.x, cv4.y, cv4.z, cv4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (rx.kbias) sk += o[u] * kb[u];
            if (rx.cvec) sc += o[u] * cv[u];
          }
          v = make_float4(o[0], o[1], o[2], o[3]);
          if (rx.relaxed[z]) *reinterpret_cast<float4*>(rel_r + e) = v;
        }
        xs4[q] = v;
      }
      for (int idx = nin + tid; idx < g.Co4 * pitch; idx += GTM) Xs[idx] = 0.f;
    } else {
      for (int idx = tid; idx < g.Co4 * pitch; idx += GTM) {
        const int co = fdivq(idx, g.f_pitch), p = idx - co * pitch;
        Xs[idx] = (co < g.Co && p < g.npix) ? relax_at(co * g.npix + p, xr[co * g.npix + p]) : 0.f;
      }
    }
    if constexpr (RELAX) {
      sb = wave_sum(sb);
      sk = wave_sum(sk);
      sc = wave_sum(sc);
      if (lane == 0) {
        rred[wave][0] = sb;
        rred[wave][1] = sk;
        rred[wave][2] = sc;
      }
      __syncthreads();
      if (tid == 0) {
        float tb = 0.f, tk = 0.f, tc = 0.f;
        for (int q = 0; q < GTM / 64; ++q) {
          tb += rred[q][0];
          tk += rred[q][1];
          tc += rred[q][2];
        }
        if (rx.b_out[z]) rx.b_out[z][r] = ((rx.b_in[z] ? rx.b_in[z][r] : 0.f) + tb) + tk;
        if (rx.c_out[z]) rx.c_out[z][r] = tc;
      }
    }
    const float hs = (lower && g.h_out) ? g.h_scale[r] : 0.f;
    float s = 0.f;
    for (int n = 0; n < g.Ci; ++n) {
      __syncthreads();   // Xs staged / the previous channel's taps consumed
      const float* __restrict__ wn = Wsm + (size_t)n * g.Co4 * 16;
      for (int jb = wave; jb < g.nblk; jb += GTM / 64) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int k = k4; k < g.Co4; k += 4)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wn[k * 16 + col], Xs[k * pitch + jb * 16 + col], acc, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) Zs[(4 * k4 + q) * pitch + jb * 16 + col] = acc[q];
      }
      __syncthreads();
      for (int o = tid; o < g.Hi * g.Wi; o += GTM) {
        const int oh = fdivq(o, g.f_Wi), ow = o - oh * g.Wi;
        // taps kh = kh0 + sh*a reach map row ih0 - a (kh0 = (oh + ph) mod sh), likewise for columns
        const int qh = fdivq(oh + g.ph, g.f_sh), qw = fdivq(ow + g.pw, g.f_sw);
        const int kh0 = oh + g.ph - qh * g.sh, kw0 = ow + g.pw - qw * g.sw;
        float v = 0.f;
        for (int kh = kh0, ih = qh; kh < g.KH; kh += g.sh, --ih) {
          if (ih < 0 || ih >= g.Ho) continue;
          for (int kw = kw0, iw = qw; kw < g.KW; kw += g.sw, --iw) {
            if (iw < 0 || iw >= g.Wo) continue;
            v += Zs[(kh * g.KW + kw) * pitch + ih * g.Wo + iw];
          }
        }
        const int64_t oidx = (int64_t)n * g.Hi * g.Wi + o;
        if (y) y[r * nout + oidx] = v;
        if (nrm) {
          const float wgt = g.wv ? g.wv[d * g.w_ld + oidx] : 1.f;
          s = norm_step(s, v, wgt, g.wv != nullptr, g.nkind);
          if (lower && g.h_out) {
            const float sg = (v > 0.f) ? 1.f : ((v < 0.f) ? -1.f : 0.f);
            g.h_out[r * nout + oidx] = g.wv ? hs * sg * wgt : hs * sg;
          }
        }
      }
    }
    if (nrm) {
      s = norm_wave_xor(s, g.nkind);
      if (lane == 0) red[wave] = s;
      __syncthreads();
      if (tid == 0) {
        float tsum = 0.f;
        for (int q = 0; q < GTM / 64; ++q) tsum = norm_join(tsum, red[q], g.nkind);
        nrm[r] = tsum;
      }
    }
  }
}

// Register form of conv_t_small_kernel for the usual input layers: at most 16 map
// channels, at most 256 map pixels, at most 3 output channels of at most 2 GTM pixels,
// at most 2 x 2 taps per output pixel (the 1 -> 16 and 3 -> 16, 4 x 4 stride-2
// convolutions of 28 x 28 and 32 x 32 images, say).
//   * Workgroups of 16 waves, one per CU.  Wave jb owns the 16-pixel block jb of the
//     map: lane (k4, col) loads the row's elements (co = k4 + 4 kk, pixel 16 jb + col)
//     straight into registers -- exactly its B operands of MFMA step kk -- and applies the
//     relaxation there, so the map never passes through LDS.  The relaxation's slopes
//     and intercepts, the split term and the center projection stay in registers while
//     consecutive rows share a domain, the bias map for the whole launch, the weights
//     (A operands) in LDS.
//   * A lane slot past the map's channels or pixels reads element 0 of the row and
//     carries zero slopes, zero weights and zero operands, so it adds exact zeros
//     (the coefficient rows are finite).
//   * Z of every output channel is written to LDS at a fixed layout; the col2im reads
//     each output pixel's taps at offsets computed once per workgroup (an absent tap
//     reads a zero cell: adding +0 to a sum that starts at +0 leaves it unchanged).
//   * Two barriers per row; the next row's elements load during the gather.
// The tap products, the col2im order and the norm order are those of
// conv_t_small_kernel, so y, the norms and the gradient seeds are identical; the row
// sums b_out and c_out add the same terms in another order.
// SRC: 0 the rows as given (no relaxation); 1 the relaxation from the pre-activation
// box (lo, hi, optional alpha); 2 from the four planes {alpha_u, beta_u, alpha_l, beta_l}.
constexpr int SF_NT = 1024;   // threads per workgroup
constexpr int SF_NW = SF_NT / 64;
constexpr int SF_UB = 1;      // 16-pixel blocks per wave: map pixels <= 16 * SF_NW * SF_UB
constexpr int SF_KS = 4;      // MFMA k steps: map channels <= 4 * SF_KS
constexpr int SF_CI = 3;      // output channels
constexpr int SF_PPT = 1;     // output pixels per thread: Hi * Wi <= SF_PPT * SF_NT
constexpr int SF_PITCHZ = 16 * SF_NW * SF_UB + 4;   // tap-row pitch of Z: 4 banks between tap rows
constexpr int SF_ZSZ = 16 * SF_PITCHZ + 4;               // floats per output channel: Z, then the zero cell
constexpr int SF_WS = SF_CI * SF_KS * 64;                // the A operands

template <int SRC>
__global__ void __launch_bounds__(SF_NT, 4)   // 4 waves per SIMD: one workgroup per CU
conv_t_small_fast_kernel(SmallTArgs g, ConvRelax rx) {
  constexpr bool RELAX = SRC != 0;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Ws = smem;           // [SF_CI][SF_KS][64 lanes]
  float* Zs = smem + SF_WS;   // [SF_CI][SF_ZSZ]
  __shared__ float red[SF_NW];
  __shared__ float rred[SF_NW][3];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: block indices stay scalar
  const int z = blockIdx.y;
  const bool lower = g.z_lower_first ? (z == 0) : (z == 1);
  const float* __restrict__ X = g.X[z];
  float* __restrict__ y = g.y[z];
  float* __restrict__ nrm = g.nrm[z];
  float* __restrict__ relaxed = RELAX ? rx.relaxed[z] : nullptr;
  const int taps = g.KH * g.KW;
  const int npix = g.npix, HW = g.Hi * g.Wi;
  const uint32_t nin = (uint32_t)(g.Co * npix);
  const int64_t nout = (int64_t)g.Ci * HW;
  const int k4 = lane >> 4, col = lane & 15;
  constexpr int zero_cell = 16 * SF_PITCHZ;
  const int ksteps = g.Co4 >> 2;   // uniform

  if (tid < SF_CI) Zs[tid * SF_ZSZ + zero_cell] = 0.f;
  // A operands: Ws[n][kk][lane (k4, col)] = W[co = k4 + 4 kk, n, tap = col]
  for (int i = tid; i < SF_WS; i += SF_NT) {
    const int l = i & 63, nk = i >> 6, n = nk / SF_KS, kk = nk - n * SF_KS;
    const int co = (l >> 4) + 4 * kk, t = l & 15;
    Ws[i] = (n < g.Ci && co < g.Co && t < taps) ? g.W[((int64_t)co * g.Ci + n) * taps + t] : 0.f;
  }
  // this lane's row element of block u, step kk: xo[u][kk] (0 for a slot past the map)
  uint32_t xo[SF_UB][SF_KS];
  uint32_t pmask = 0;   // bit u SF_KS + kk: the slot holds an element of the map
#pragma unroll
  for (int u = 0; u < SF_UB; ++u)
#pragma unroll
    for (int kk = 0; kk < SF_KS; ++kk) {
      const int co = k4 + 4 * kk, p = 16 * (wave + SF_NW * u) + col;
      const bool present = co < g.Co && p < npix;
      xo[u][kk] = present ? (uint32_t)(co * npix + p) : 0u;
      if (present) pmask |= 1u << (u * SF_KS + kk);
    }
  auto present_at = [&](int u, int kk) { return ((pmask >> (u * SF_KS + kk)) & 1u) != 0; };
  // the taps of output pixel o_j = tid + SF_NT j, in the order (kh, kw) of conv_t_small_kernel
  int off[SF_PPT][4];
#pragma unroll
  for (int j = 0; j < SF_PPT; ++j) {
    const int o = tid + SF_NT * j;
#pragma unroll
    for (int t = 0; t < 4; ++t) off[j][t] = zero_cell;
    if (o < HW) {
      const int oh = o / g.Wi, ow = o - oh * g.Wi;
      const int qh = (oh + g.ph) / g.sh, qw = (ow + g.pw) / g.sw;
      const int kh0 = oh + g.ph - qh * g.sh, kw0 = ow + g.pw - qw * g.sw;
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int kh = kh0 + g.sh * a, kw = kw0 + g.sw * b, ih = qh - a, iw = qw - b;
          if (kh < g.KH && kw < g.KW && ih >= 0 && ih < g.Ho && iw >= 0 && iw < g.Wo)
            off[j][2 * a + b] = (kh * g.KW + kw) * SF_PITCHZ + ih * g.Wo + iw;
        }
    }
  }

  const int64_t r0 = (int64_t)blockIdx.x * g.rows_per_wg;
  const int64_t r_end = r0 + g.rows_per_wg < g.R ? r0 + g.rows_per_wg : g.R;
  float xv[SF_UB][SF_KS];
  auto load_row = [&](int64_t r) {
    const float* __restrict__ xr = X + r * (int64_t)nin;
#pragma unroll
    for (int u = 0; u < SF_UB; ++u)
#pragma unroll
      for (int kk = 0; kk < SF_KS; ++kk) xv[u][kk] = xr[xo[u][kk]];
  };
  // per element of the cached domain: the slopes for v >= 0 and v < 0 on this side, the
  // intercepts for v >= 0 and v < 0 (ip, in), the split term, the center projection; the bias map
  float sp[SF_UB][SF_KS], sn[SF_UB][SF_KS], ip[SF_UB][SF_KS], in_[SF_UB][SF_KS];
  float adc[SF_UB][SF_KS], cvc[SF_UB][SF_KS], kbc[SF_UB][SF_KS];
  if constexpr (RELAX) {
#pragma unroll
    for (int u = 0; u < SF_UB; ++u)
#pragma unroll
      for (int kk = 0; kk < SF_KS; ++kk) kbc[u][kk] = (rx.kbias && present_at(u, kk)) ? rx.kbias[xo[u][kk]] : 0.f;
  }
  // domain of the current row, and the row's index inside it
  int64_t d = r0 / g.S;
  int64_t s_in = r0 - d * g.S;
  int64_t d_cached = -1;
  if (r0 < r_end) load_row(r0);
  for (int64_t r = r0; r < r_end; ++r) {
    float bop[SF_UB][SF_KS];
    if constexpr (RELAX) {
      if (d != d_cached) {   // uniform
        d_cached = d;
        const int64_t dn = d * (int64_t)nin;
#pragma unroll
        for (int u = 0; u < SF_UB; ++u)
#pragma unroll
          for (int kk = 0; kk < SF_KS; ++kk) {
            // opaque to the optimizer: the element addresses are formed here, once per domain,
            // rather than hoisted out of the row loop as live 64-bit registers
            uint32_t e = xo[u][kk];
            asm volatile("" : "+v"(e));
            const bool pr = present_at(u, kk);
            float4 t = make_float4(1.f, 0.f, 1.f, 0.f);
            if (SRC == 2) {
              t = make_float4(rx.pl[0][dn + e], rx.pl[1][dn + e], rx.pl[2][dn + e], rx.pl[3][dn + e]);
            } else if (rx.lo) {
              const bool has_alpha = rx.alpha != nullptr;
              const Relax rr = relu_relax(rx.lo[dn + e], rx.hi[dn + e], has_alpha,
                                          has_alpha ? clamp01(rx.alpha[d * rx.alpha_ld + e]) : 0.f);
              t = make_float4(rr.au, rr.bu, rr.al, rr.bl);
            }
            // lower: A' = A (al | au), A * (bl | bu); upper: A' = A (au | al), A * (bu | bl)  (v >= 0 | v < 0)
            sp[u][kk] = pr ? (lower ? t.z : t.x) : 0.f;
            sn[u][kk] = pr ? (lower ? t.x : t.z) : 0.f;
            ip[u][kk] = pr ? (lower ? t.w : t.y) : 0.f;
            in_[u][kk] = pr ? (lower ? t.y : t.w) : 0.f;
            adc[u][kk] = (pr && lower && rx.add) ? rx.add[d * rx.add_ld + e] : 0.f;
            cvc[u][kk] = (pr && rx.cvec) ? rx.cvec[dn + e] : 0.f;
          }
      }
      float sb = 0.f, sk = 0.f, sc = 0.f;
#pragma unroll
      for (int u = 0; u < SF_UB; ++u)
#pragma unroll
        for (int kk = 0; kk < SF_KS; ++kk) {
          // relax_element's arithmetic: a slot past the map has zero slopes and terms
          const float v = xv[u][kk];
          const bool nn = v >= 0.f;
          float o = v * (nn ? sp[u][kk] : sn[u][kk]);
          sb += v * (nn ? ip[u][kk] : in_[u][kk]);
          if (lower && rx.add) o = o + adc[u][kk];
          if (rx.kbias) sk += o * kbc[u][kk];
          if (rx.cvec) sc += o * cvc[u][kk];
          if (relaxed && present_at(u, kk)) relaxed[r * (int64_t)nin + xo[u][kk]] = o;
          bop[u][kk] = o;
        }
      sb = wave_sum(sb);
      sk = wave_sum(sk);
      sc = wave_sum(sc);
      if (lane == 0) {
        rred[wave][0] = sb;
        rred[wave][1] = sk;
        rred[wave][2] = sc;
      }
    } else {
#pragma unroll
      for (int u = 0; u < SF_UB; ++u)
#pragma unroll
        for (int kk = 0; kk < SF_KS; ++kk) bop[u][kk] = present_at(u, kk) ? xv[u][kk] : 0.f;
    }
    // tap products of every output channel: Z_n[tap 4 k4 + q][pixel 16 jb + col] = acc[q]
#pragma unroll
    for (int n = 0; n < SF_CI; ++n) {
      if (n >= g.Ci) break;   // uniform
      float wr[SF_KS];
#pragma unroll
      for (int kk = 0; kk < SF_KS; ++kk) wr[kk] = Ws[(n * SF_KS + kk) * 64 + lane];
#pragma unroll
      for (int u = 0; u < SF_UB; ++u) {
        const int jb = wave + SF_NW * u;
        if (jb >= g.nblk) break;   // uniform
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < SF_KS; ++kk)
          if (kk < ksteps) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wr[kk], bop[u][kk], acc, 0, 0, 0);
        float* zr = Zs + n * SF_ZSZ + (4 * k4) * SF_PITCHZ + 16 * jb + col;
#pragma unroll
        for (int q = 0; q < 4; ++q) zr[q * SF_PITCHZ] = acc[q];
      }
    }
    if (r + 1 < r_end) load_row(r + 1);
    __syncthreads();   // Z of every channel written; the row sums of every wave posted
    float row_b = 0.f, row_c = 0.f;   // the row's bias and center sums (thread 0)
    if constexpr (RELAX) {
      if (tid == 0) {
        float tb = 0.f, tk = 0.f, tcs = 0.f;
        for (int q = 0; q < SF_NW; ++q) {
          tb += rred[q][0];
          tk += rred[q][1];
          tcs += rred[q][2];
        }
        row_b = ((rx.b_in[z] ? rx.b_in[z][r] : 0.f) + tb) + tk;
        row_c = tcs;
        if (rx.b_out[z]) rx.b_out[z][r] = row_b;
        if (rx.c_out[z]) rx.c_out[z][r] = row_c;
      }
    }
    const float hs = (lower && g.h_out) ? g.h_scale[r] : 0.f;
    float s = 0.f;
#pragma unroll
    for (int n = 0; n < SF_CI; ++n) {
      if (n >= g.Ci) break;   // uniform
      const float* __restrict__ zn = Zs + n * SF_ZSZ;
#pragma unroll
      for (int j = 0; j < SF_PPT; ++j) {
        const int o = tid + SF_NT * j;
        if (o >= HW) break;
        float v = 0.f;
        v += zn[off[j][0]];
        v += zn[off[j][1]];
        v += zn[off[j][2]];
        v += zn[off[j][3]];
        const int64_t oidx = (int64_t)n * HW + o;
        if (y) y[r * nout + oidx] = v;
        if (nrm) {
          const float wgt = g.wv ? g.wv[d * g.w_ld + oidx] : 1.f;
          s = norm_step(s, v, wgt, g.wv != nullptr, g.nkind);
          if (lower && g.h_out) {
            const float sg = (v > 0.f) ? 1.f : ((v < 0.f) ? -1.f : 0.f);
            g.h_out[r * nout + oidx] = g.wv ? hs * sg * wgt : hs * sg;
          }
        }
      }
    }
    if (nrm) {
      s = norm_wave_xor(s, g.nkind);
      if (lane == 0) red[wave] = s;
    }
    __syncthreads();   // every wave's taps gathered (Z free for the next row); the norms posted
    if (nrm && tid == 0) {
      float tsum = 0.f;
      for (int q = 0; q < SF_NW; ++q) tsum = norm_join(tsum, red[q], g.nkind);
      nrm[r] = tsum;
      if constexpr (RELAX) {
        // the bound of the row, as concretize_finalize_kernel forms it from this one partial norm
        if (g.bnd[z]) {
          const float fin = g.nkind == 2 ? sqrtf(tsum) : tsum;
          g.bnd[z][r] = lower ? (row_c - g.eps * fin) + row_b : (row_c + g.eps * fin) + row_b;
        }
      }
    }
    if (++s_in == g.S) {
      s_in = 0;
      ++d;
    }
  }
}

// Plan of conv_t_small_fast_kernel over a conv_t_small_kernel plan; false when it does not apply.
static bool conv_t_small_fast_plan(SmallTArgs& g, size_t* lds_bytes) {
  if (g.Co > 4 * SF_KS || g.nblk > SF_NW * SF_UB || g.Ci > SF_CI || g.Hi * g.Wi > SF_PPT * SF_NT) return false;
  if ((g.KH + g.sh - 1) / g.sh > 2 || (g.KW + g.sw - 1) / g.sw > 2) return false;
  *lds_bytes = sizeof(float) * (size_t)(SF_WS + SF_CI * SF_ZSZ);
  return true;
}

// Rows per workgroup of conv_t_small_fast_kernel: one round of one workgroup per CU.
static int small_fast_rows_per_wg(int64_t work) {
  const int64_t rpw = (work + 255) / 256;
  return rpw < 1 ? 1 : (rpw > 64 ? 64 : (int)rpw);
}

// BOUNDFLOW_CONV_T_SMALL=generic keeps every shape on conv_t_small_kernel (for
// measurement); read once when the library is loaded.
static bool small_fast_disabled_from_env() {
  const char* v = std::getenv("BOUNDFLOW_CONV_T_SMALL");
  return v != nullptr && std::strcmp(v, "generic") == 0;
}
static const bool kSmallFastDisabled = small_fast_disabled_from_env();


static int gather_rows_per_wg(int64_t work);

// Launch of the tap-product transposed conv over a conv_t_small_kernel plan: the
// register form where it applies, else the generic kernel (which takes the
// relaxation from the pre-activation box only).
template <bool RELAX>
static int small_t_launch(SmallTArgs& g, const ConvRelax& rx, unsigned nz, size_t glds, const char* who,
                          hipStream_t stream, bool* fast = nullptr) {
  size_t flds = 0;
  if (fast) *fast = false;
  if (!kSmallFastDisabled && conv_t_small_fast_plan(g, &flds)) {
    if (fast) *fast = true;
    BF_REQUIRE(g.R * (int64_t)g.Co * g.npix < (1LL << 62) && (int64_t)g.Co * g.npix < (1LL << 31),
               "%s: rows too large", who);
    const int rpw = small_fast_rows_per_wg(g.R * nz);
    g.rows_per_wg = rpw;
    BF_REQUIRE((g.R + rpw - 1) / rpw < (1LL << 31), "%s: too many rows", who);
    const dim3 grid((unsigned)((g.R + rpw - 1) / rpw), nz);
    if (!RELAX)
      hipLaunchKernelGGL(conv_t_small_fast_kernel<0>, grid, dim3(SF_NT), flds, stream, g, rx);
    else if (rx.pl[0])
      hipLaunchKernelGGL(conv_t_small_fast_kernel<2>, grid, dim3(SF_NT), flds, stream, g, rx);
    else
      hipLaunchKernelGGL(conv_t_small_fast_kernel<1>, grid, dim3(SF_NT), flds, stream, g, rx);
    BF_LAUNCH_CHECK(who);
    return BF_OK;
  }
  BF_REQUIRE(!RELAX || rx.pl[0] == nullptr, "%s: relaxation planes need the register form of the kernel", who);
  const int rpw = gather_rows_per_wg(g.R * nz);
  g.rows_per_wg = rpw;
  BF_REQUIRE((g.R + rpw - 1) / rpw < (1LL << 31), "%s: too many rows", who);
  hipLaunchKernelGGL(conv_t_small_kernel<RELAX>, dim3((unsigned)((g.R + rpw - 1) / rpw), nz), dim3(GTM), glds, stream,
                     g, rx);
  BF_LAUNCH_CHECK(who);
  return BF_OK;
}

// Plan of conv_t_small_kernel; false when it does not apply.
static bool conv_t_small_plan(SmallTArgs& g, int64_t R, int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh,
                              int sw, int ph, int pw, int Hi, int Wi, size_t* lds_bytes) {
  if (Ci > 4 || KH * KW > 16 || ph < 0 || pw < 0) return false;
  g.R = R;
  g.Co = Co; g.Ho = Ho; g.Wo = Wo; g.Ci = Ci; g.KH = KH; g.KW = KW; g.sh = sh; g.sw = sw; g.ph = ph; g.pw = pw;
  g.Hi = Hi; g.Wi = Wi;
  g.Co4 = (Co + 3) / 4 * 4;
  g.npix = Ho * Wo;
  g.nblk = (g.npix + 15) / 16;
  const size_t lds = sizeof(float) * ((size_t)Ci * g.Co4 * 16 + (size_t)g.Co4 * g.nblk * 16 + (size_t)16 * g.nblk * 16);
  if (lds > 64 * 1024 || Hi * Wi >= 65536 || Hi + ph >= 65536 || Wi + pw >= 65536) return false;
  *lds_bytes = lds;
  g.f_Wi = make_fdiv(Wi);
  g.f_sh = make_fdiv(sh);
  g.f_sw = make_fdiv(sw);
  g.f_pitch = make_fdiv(g.nblk * 16);
  return true;
}

// floor / ceil of x / y for y > 0 and any sign of x
static inline int fdiv(int x, int y) { return x >= 0 ? x / y : -((-x + y - 1) / y); }
static inline int cdiv(int x, int y) { return x >= 0 ? (x + y - 1) / y : -((-x) / y); }

// Build the class decomposition; returns false when the MFMA path does not apply.
static bool conv_t_mfma_plan(GatherArgs& g, int64_t R, int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh,
                             int sw, int ph, int pw, int Hi, int Wi, size_t* lds_bytes) {
  if (KH % sh || KW % sw || sh * sw > GMAX_CLASSES) return false;
  g.Cm = Co; g.Hm = Ho; g.Wm = Wo; g.Cin = Ci; g.nch = Ci; g.HWout = Hi * Wi;
  g.KH = KH; g.KW = KW; g.sh = sh; g.sw = sw;
  g.nA = KH / sh; g.nB = KW / sw; g.T = g.nA * g.nB;
  g.Kc = Co * g.T;
  g.Kc4 = (g.Kc + 15) / 16 * 16;
  g.npad = (Ci + 15) / 16 * 16;
  g.nblk = g.npad / 16;
  g.nclasses = sh * sw;
  int umin_all = 1 << 30, umax_all = -(1 << 30), vmin_all = 1 << 30, vmax_all = -(1 << 30);
  int umin[GMAX_CLASSES], vmin[GMAX_CLASSES], nu[GMAX_CLASSES], nv[GMAX_CLASSES];
  for (int c = 0; c < g.nclasses; ++c) {
    const int al = c / sw, be = c % sw;
    umin[c] = cdiv(ph - al, sh);
    vmin[c] = cdiv(pw - be, sw);
    const int umax = fdiv(Hi - 1 + ph - al, sh), vmax = fdiv(Wi - 1 + pw - be, sw);
    nu[c] = umax >= umin[c] ? umax - umin[c] + 1 : 0;
    nv[c] = vmax >= vmin[c] ? vmax - vmin[c] + 1 : 0;
    if (nu[c] && nv[c]) {
      umin_all = umin[c] < umin_all ? umin[c] : umin_all;
      vmin_all = vmin[c] < vmin_all ? vmin[c] : vmin_all;
      umax_all = umax > umax_all ? umax : umax_all;
      vmax_all = vmax > vmax_all ? vmax : vmax_all;
    }
  }
  if (umax_all < 0) return false;
  // halo so that u - a and v - b (a < nA, b < nB) always index inside the padded map
  g.pad_h = (g.nA - 1) - umin_all > 0 ? (g.nA - 1) - umin_all : 0;
  g.pad_w = (g.nB - 1) - vmin_all > 0 ? (g.nB - 1) - vmin_all : 0;
  g.Hp = (Ho > umax_all + 1 ? Ho : umax_all + 1) + g.pad_h;
  g.Wp = (Wo > vmax_all + 1 ? Wo : vmax_all + 1) + g.pad_w;
  int ntasks = 0;
  for (int c = 0; c < g.nclasses; ++c) {
    GatherClass& C = g.cls[c];
    const int al = c / sw, be = c % sw;
    C.np = nu[c] * nv[c];
    C.n2 = nv[c] > 0 ? nv[c] : 1;
    C.poff0 = (umin[c] + g.pad_h) * g.Wp + vmin[c] + g.pad_w;
    C.s1 = g.Wp;
    C.s2 = 1;
    C.out0 = (sh * umin[c] + al - ph) * Wi + sw * vmin[c] + be - pw;
    C.o1 = sh * Wi;
    C.o2 = sw;
    C.tbase = ntasks;
    ntasks += (C.np + 15) / 16 * g.nblk;
  }
  g.ntasks = ntasks;
  const size_t lds = sizeof(float) * ((size_t)g.nclasses * g.Kc4 * g.npad + g.Kc4 + (size_t)Co * g.Hp * g.Wp);
  if (lds > 64 * 1024) return false;
  *lds_bytes = lds;
  g.R = R;
  g.in_div = 1;
  gather_fdivs(g);
  return true;
}

// The channel-last variant of the transposed-conv gather-GEMM (conv_t_hwc_kernel):
// the parity classes of conv_t_mfma_plan, Co a multiple of 16, map indices below
// 2^16 (exact FastDiv) and the stage within 64 KB.
static bool conv_t_hwc_plan(GatherArgs& g, int64_t R, int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw,
                            int ph, int pw, int Hi, int Wi, size_t* lds_bytes) {
  if (Co % 16 != 0 || (int64_t)Co * Ho * Wo >= (1 << 16)) return false;
  size_t base_lds = 0;
  if (!conv_t_mfma_plan(g, R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &base_lds)) return false;
  const size_t lds = sizeof(float) * ((size_t)g.nclasses * g.Kc4 * g.npad + (size_t)g.Hp * g.Wp * (Co + 4));
  if (lds > 64 * 1024) return false;
  *lds_bytes = lds;
  g.f_HWm = make_fdiv(Ho * Wo);
  g.f_Wm = make_fdiv(Wo);
  return true;
}

// conv2d as one gather class; returns false when the LDS stage does not fit.
static bool conv_f_mfma_plan(GatherArgs& g, int64_t R, int Ci, int Hi, int Wi, int Co, int KH, int KW, int sh,
                             int sw, int ph, int pw, int Ho, int Wo, size_t* lds_bytes) {
  g.Cm = Ci; g.Hm = Hi; g.Wm = Wi; g.Cin = Ci; g.nch = Co; g.HWout = Ho * Wo;
  g.KH = KH; g.KW = KW; g.sh = sh; g.sw = sw;
  g.Kc = Ci * KH * KW;
  g.Kc4 = (g.Kc + 15) / 16 * 16;
  g.npad = (Co + 15) / 16 * 16;
  g.nblk = g.npad / 16;
  g.nclasses = 1;
  // padded map coordinate hp = hi + ph = ho*sh + kh
  g.pad_h = ph;
  g.pad_w = pw;
  const int need_h = (Ho - 1) * sh + KH, need_w = (Wo - 1) * sw + KW;
  g.Hp = Hi + ph > need_h ? Hi + ph : need_h;
  g.Wp = Wi + pw > need_w ? Wi + pw : need_w;
  GatherClass& C = g.cls[0];
  C.np = Ho * Wo;
  C.n2 = Wo;
  C.poff0 = 0;
  C.s1 = sh * g.Wp;
  C.s2 = sw;
  C.out0 = 0;
  C.o1 = Wo;
  C.o2 = 1;
  C.tbase = 0;
  g.ntasks = (C.np + 15) / 16 * g.nblk;
  const size_t lds = sizeof(float) * ((size_t)g.Kc4 * g.npad + g.Kc4 + (size_t)Ci * g.Hp * g.Wp);
  if (lds > 64 * 1024) return false;
  *lds_bytes = lds;
  g.R = R;
  gather_fdivs(g);
  return true;
}

// rows per workgroup: amortize the weight stage, keep >= ~3 workgroups per CU
static int gather_rows_per_wg(int64_t work) {
  int64_t rpw = work / 768;
  return rpw < 1 ? 1 : (rpw > 8 ? 8 : (int)rpw);
}


// Launch of the channel-last gather-GEMM over a conv_t_hwc plan (lds: its LDS footprint).
template <bool RELAX>
static int hwc_launch(GatherArgs& g, const ConvRelax& rx, unsigned nz, size_t lds, const char* who,
                      hipStream_t stream) {
  const int rpw = gather_rows_per_wg(g.R * nz);
  g.rows_per_wg = rpw;
  BF_REQUIRE((g.R + rpw - 1) / rpw < (1LL << 31), "%s: too many rows", who);
  hipLaunchKernelGGL(conv_t_hwc_kernel<RELAX>, dim3((unsigned)((g.R + rpw - 1) / rpw), nz), dim3(GTM), lds, stream, g,
                     rx);
  BF_LAUNCH_CHECK(who);
  return BF_OK;
}

int ibp_center_radius(const float* lo, const float* hi, int64_t n, int apply_relu, float* mid, float* rad,
                      hipStream_t stream);
int ibp_finalize(const float* c, const float* r, const float* rownorm, float eps, const float* bias,
                 int64_t bias_div, const int8_t* split, int64_t split_ld, int64_t B, int64_t N, float* lo, float* hi,
                 int* infeasible, hipStream_t stream);
int fill_value(float* p, int64_t n, float v, hipStream_t stream);
int lp_seed_rows(float* h, int64_t M, int64_t I, const float* h_scale, int norm_p, hipStream_t stream);
int concretize_finalize(const float* pu, const float* pl, int nparts, int64_t M, const float* cu, const float* cl,
                        const float* bu, const float* bl, float eps, int norm_p, float* lb, float* ub,
                        hipStream_t stream);

// conv2d of rows; with x2/y2 a second operand pair (abs_w2 for its weights) runs in
// the same launch (blockIdx.y = 1), e.g. the center and the radius of an IBP layer.
static int conv2d_launch(const float* x, int64_t in_div, int64_t R, int Ci, int Hi, int Wi, const float* W, int abs_w,
                         int Co, int KH, int KW, int sh, int sw, int ph, int pw, int Ho, int Wo, float* y,
                         const float* rs, const float* v, int64_t v_div, int64_t v_ld, hipStream_t stream,
                         const float* x2 = nullptr, float* y2 = nullptr, int abs_w2 = 0) {
  const int nz = x2 ? 2 : 1;
  {
    GatherArgs g;
    memset(&g, 0, sizeof(g));
    size_t glds = 0;
    if (conv_f_mfma_plan(g, R, Ci, Hi, Wi, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, &glds)) {
      g.X[0] = x;
      g.y[0] = y;
      g.X[1] = x2;
      g.y[1] = y2;
      g.W = W;
      g.abs_w = (abs_w ? 1 : 0) | (abs_w2 ? 2 : 0);   // bit z: operand pair z uses |W|
      g.in_div = in_div;
      g.rs = rs;
      g.v = v;
      g.v_div = v_div;
      g.v_ld = v_ld;
      g.S = 1;
      g.rows_per_wg = gather_rows_per_wg(R * nz);
      const int rpw = g.rows_per_wg;
      BF_REQUIRE((R + rpw - 1) / rpw < (1LL << 31), "conv2d: too many rows");
      hipLaunchKernelGGL(conv_mfma_kernel<MODE_F>, dim3((unsigned)((R + rpw - 1) / rpw), nz), dim3(GTM), glds, stream,
                         g);
      BF_LAUNCH_CHECK("conv_mfma_kernel<conv2d>");
      return BF_OK;
    }
  }
  if (x2) {
    const int rc = conv2d_launch(x, in_div, R, Ci, Hi, Wi, W, abs_w, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, y, rs, v,
                                 v_div, v_ld, stream);
    if (rc) return rc;
    return conv2d_launch(x2, in_div, R, Ci, Hi, Wi, W, abs_w2, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, y2, rs, v, v_div,
                         v_ld, stream);
  }
  const size_t lds = sizeof(float) * (size_t)Ci * Hi * Wi;
  BF_REQUIRE(R < (1LL << 31), "conv2d: too many rows");
  BF_REQUIRE((int64_t)Ci * Hi * Wi < (1LL << 31) && (int64_t)Co * Ho * Wo < (1LL << 31), "conv2d: map too large");
  if (lds <= 64 * 1024)
    hipLaunchKernelGGL(conv2d_rows_kernel<true>, dim3((unsigned)R), dim3(CT), lds, stream, x, in_div, Ci, Hi, Wi, W,
                       abs_w, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, y, rs, v, v_div, v_ld);
  else   // a map beyond the LDS row stage: the taps read it from global memory
    hipLaunchKernelGGL(conv2d_rows_kernel<false>, dim3((unsigned)R), dim3(CT), 0, stream, x, in_div, Ci, Hi, Wi, W,
                       abs_w, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, y, rs, v, v_div, v_ld);
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

static int conv_transpose_rows_launch(const float* A_u, const float* A_l, int64_t R, int Co, int Ho, int Wo,
                                      const float* W, int Ci, int KH, int KW, int sh, int sw, int ph, int pw, int Hi,
                                      int Wi, float* y_u, float* y_l, int64_t S, const float* wvec, int64_t w_ld,
                                      int norm_p, float* norm_u, float* norm_l, const float* h_scale, float* h_out,
                                      hipStream_t stream) {
  const unsigned nz = (A_u && A_l) ? 2u : 1u;
  {
    SmallTArgs g;
    memset(&g, 0, sizeof(g));
    size_t glds = 0;
    if (conv_t_small_plan(g, R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &glds)) {
      int nzi = 0;
      if (A_u) { g.X[nzi] = A_u; g.y[nzi] = y_u; g.nrm[nzi] = norm_u; ++nzi; }
      if (A_l) { g.X[nzi] = A_l; g.y[nzi] = y_l; g.nrm[nzi] = norm_l; ++nzi; }
      g.z_lower_first = A_u ? 0 : 1;
      g.W = W;
      g.wv = wvec;
      g.w_ld = w_ld;
      g.nkind = norm_p;
      g.h_scale = h_scale;
      g.h_out = h_out;
      g.S = S;
      g.vec = (g.npix % 16 == 0) && (((uintptr_t)(A_u ? A_u : A_l) & 15) == 0) &&
              (A_u == nullptr || A_l == nullptr || ((uintptr_t)A_l & 15) == 0) ? 1 : 0;
      ConvRelax rx;
      memset(&rx, 0, sizeof(rx));
      return small_t_launch<false>(g, rx, nz, glds, "bf_conv_transpose_rows (tap products)", stream);
    }
  }
  {
    GatherArgs g;
    memset(&g, 0, sizeof(g));
    size_t glds = 0;
    if (conv_t_hwc_plan(g, R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &glds)) {
      int nzi = 0;
      if (A_u) { g.X[nzi] = A_u; g.y[nzi] = y_u; g.nrm[nzi] = norm_u; ++nzi; }
      if (A_l) { g.X[nzi] = A_l; g.y[nzi] = y_l; g.nrm[nzi] = norm_l; ++nzi; }
      g.z_lower_first = A_u ? 0 : 1;
      g.W = W;
      g.wv = wvec;
      g.w_ld = w_ld;
      g.nkind = norm_p;
      g.h_scale = h_scale;
      g.h_out = h_out;
      g.S = S;
      ConvRelax rx;
      memset(&rx, 0, sizeof(rx));
      return hwc_launch<false>(g, rx, nz, glds, "bf_conv_transpose_rows (channel-last gather-GEMM)", stream);
    }
  }
  {
    GatherArgs g;
    memset(&g, 0, sizeof(g));
    size_t glds = 0;
    if (conv_t_mfma_plan(g, R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &glds)) {
      int nzi = 0;
      if (A_u) { g.X[nzi] = A_u; g.y[nzi] = y_u; g.nrm[nzi] = norm_u; ++nzi; }
      if (A_l) { g.X[nzi] = A_l; g.y[nzi] = y_l; g.nrm[nzi] = norm_l; ++nzi; }
      g.z_lower_first = A_u ? 0 : 1;
      g.W = W;
      g.wv = wvec;
      g.w_ld = w_ld;
      g.nkind = norm_p;
      g.h_scale = h_scale;
      g.h_out = h_out;
      g.S = S;
      const int rpw = gather_rows_per_wg(R * nz);
      g.rows_per_wg = rpw;
      BF_REQUIRE((R + rpw - 1) / rpw < (1LL << 31), "bf_conv_transpose_rows: too many rows");
      hipLaunchKernelGGL(conv_mfma_kernel<MODE_T>, dim3((unsigned)((R + rpw - 1) / rpw), nz), dim3(GTM), glds, stream,
                         g);
      BF_LAUNCH_CHECK("conv_mfma_kernel<conv_transpose2d>");
      return BF_OK;
    }
  }
  const size_t lds = sizeof(float) * (size_t)Co * Ho * Wo;
  BF_REQUIRE(R < (1LL << 31), "bf_conv_transpose_rows: too many rows");
  BF_REQUIRE((int64_t)Co * Ho * Wo < (1LL << 31) && (int64_t)Ci * Hi * Wi < (1LL << 31),
             "bf_conv_transpose_rows: map too large");
  if (lds <= 64 * 1024)
    hipLaunchKernelGGL(conv_transpose_rows_kernel<true>, dim3((unsigned)R, nz), dim3(CT), lds, stream, A_u, A_l, Co,
                       Ho, Wo, W, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, y_u, y_l, S, wvec, w_ld, norm_p, norm_u, norm_l,
                       h_scale, h_out);
  else   // a map beyond the LDS row stage: the taps read it from global memory
    hipLaunchKernelGGL(conv_transpose_rows_kernel<false>, dim3((unsigned)R, nz), dim3(CT), 0, stream, A_u, A_l, Co,
                       Ho, Wo, W, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, y_u, y_l, S, wvec, w_ld, norm_p, norm_u, norm_l,
                       h_scale, h_out);
  BF_LAUNCH_CHECK("conv_transpose_rows_kernel");
  return BF_OK;
}

int bf_conv_transpose_rows(const float* A_u, const float* A_l, int64_t R, int Co, int Ho, int Wo, const float* W,
                           int Ci, int KH, int KW, int sh, int sw, int ph, int pw, int Hi, int Wi, float* y_u,
                           float* y_l, int64_t S, const float* wvec, int64_t w_ld, int norm_p, float* norm_u,
                           float* norm_l, const float* h_scale, float* h_out, hipStream_t stream) {
  BF_REQUIRE(R >= 0 && Co > 0 && Ci > 0 && KH > 0 && KW > 0 && sh > 0 && sw > 0 && Hi > 0 && Wi > 0 && S > 0,
             "bf_conv_transpose_rows: bad sizes");
  BF_REQUIRE(norm_p >= 0 && norm_p <= 2 && (norm_p == 0 || wvec == nullptr),
             "bf_conv_transpose_rows: norm_p is 0, 1 or 2; 1 and 2 take no weights");
  if (R == 0) return BF_OK;
  BF_REQUIRE(W && (A_u || A_l), "bf_conv_transpose_rows: null pointer");
  BF_REQUIRE((A_u == nullptr) == (y_u == nullptr && norm_u == nullptr) && (A_l == nullptr) == (y_l == nullptr && norm_l == nullptr),
             "bf_conv_transpose_rows: each given coefficient needs an output or a norm");
  BF_REQUIRE((h_out == nullptr) == (h_scale == nullptr) && (h_out == nullptr || norm_l != nullptr),
             "bf_conv_transpose_rows: h_out needs h_scale and the lower norm");
  if (norm_p == 0 || h_out == nullptr)
    return conv_transpose_rows_launch(A_u, A_l, R, Co, Ho, Wo, W, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, y_u, y_l, S,
                                      wvec, w_ld, norm_p, norm_u, norm_l, h_scale, h_out, stream);
  // L1/L2 seeds need each row's whole norm: the lower rows are stored into h_out, then made into the seed
  BF_REQUIRE(y_l == nullptr, "bf_conv_transpose_rows: with norm_p 1 or 2, h_out takes the place of y_l");
  const int rc = conv_transpose_rows_launch(A_u, A_l, R, Co, Ho, Wo, W, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, y_u,
                                            h_out, S, nullptr, 0, norm_p, norm_u, norm_l, nullptr, nullptr, stream);
  if (rc) return rc;
  return lp_seed_rows(h_out, R, (int64_t)Ci * Hi * Wi, h_scale, norm_p, stream);
}

int bf_conv_transpose_hwc_supported(int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw, int ph, int pw,
                                    int Hi, int Wi) {
  if (Co <= 0 || Ci <= 0 || KH <= 0 || KW <= 0 || sh <= 0 || sw <= 0 || Hi <= 0 || Wi <= 0 || Ho <= 0 || Wo <= 0)
    return 0;
  GatherArgs g;
  memset(&g, 0, sizeof(g));
  size_t lds = 0;
  return conv_t_hwc_plan(g, 1, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &lds) ? 1 : 0;
}

int64_t bf_conv_transpose_packed_floats(int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw, int ph,
                                        int pw, int Hi, int Wi) {
  GatherArgs g;
  memset(&g, 0, sizeof(g));
  size_t lds = 0;
  if (!conv_t_hwc_plan(g, 1, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &lds)) return 0;
  return (int64_t)g.nclasses * g.Kc4 * g.npad;
}

int bf_conv_transpose_pack_weights(const float* W, int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw,
                                   int ph, int pw, int Hi, int Wi, float* out, hipStream_t stream) {
  BF_REQUIRE(W && out, "bf_conv_transpose_pack_weights: null pointer");
  GatherArgs g;
  memset(&g, 0, sizeof(g));
  size_t lds = 0;
  if (!conv_t_hwc_plan(g, 1, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &lds)) {
    set_error("bf_conv_transpose_pack_weights: shape not supported (bf_conv_transpose_hwc_supported)");
    return BF_EINVAL;
  }
  g.W = W;
  const int total = g.nclasses * g.Kc4 * g.npad;
  hipLaunchKernelGGL(conv_t_hwc_pack_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, stream, g, out);
  BF_LAUNCH_CHECK("conv_t_hwc_pack_kernel");
  return BF_OK;
}

int bf_crown_relu_conv_transpose(const float* A_u, const float* A_l, int64_t D, int64_t S, int Co, int Ho, int Wo,
                                 const float* pre_lo, const float* pre_hi, const float* alpha, int64_t alpha_ld,
                                 const float* add_l, int64_t add_ld, const float* kbias, const float* b_u_in,
                                 const float* b_l_in, const float* W, const float* w_packed, int Ci, int KH, int KW,
                                 int sh, int sw, int ph, int pw, int Hi, int Wi, float* y_u, float* y_l,
                                 float* b_u_out, float* b_l_out, float* relaxed_u, float* relaxed_l,
                                 hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0 && Co > 0 && Ci > 0, "bf_crown_relu_conv_transpose: bad sizes");
  const int64_t R = D * S;
  if (R == 0) return BF_OK;
  BF_REQUIRE(W && (A_u || A_l), "bf_crown_relu_conv_transpose: null pointer");
  BF_REQUIRE((A_u == nullptr) == (y_u == nullptr) && (A_l == nullptr) == (y_l == nullptr),
             "bf_crown_relu_conv_transpose: each given coefficient needs an output");
  BF_REQUIRE((pre_lo == nullptr) == (pre_hi == nullptr), "bf_crown_relu_conv_transpose: pre_lo and pre_hi go together");
  GatherArgs g;
  memset(&g, 0, sizeof(g));
  size_t glds = 0;
  if (!conv_t_hwc_plan(g, R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &glds)) {
    set_error("bf_crown_relu_conv_transpose: shape not supported (bf_conv_transpose_hwc_supported)");
    return BF_EINVAL;
  }
  const unsigned nz = (A_u && A_l) ? 2u : 1u;
  ConvRelax rx;
  memset(&rx, 0, sizeof(rx));
  rx.lo = pre_lo;
  rx.hi = pre_hi;
  rx.alpha = alpha;
  rx.alpha_ld = alpha_ld;
  rx.add = add_l;
  rx.add_ld = add_ld;
  rx.kbias = kbias;
  int nzi = 0;
  if (A_u) {
    g.X[nzi] = A_u; g.y[nzi] = y_u;
    rx.b_in[nzi] = b_u_in; rx.b_out[nzi] = b_u_out; rx.relaxed[nzi] = relaxed_u;
    ++nzi;
  }
  if (A_l) {
    g.X[nzi] = A_l; g.y[nzi] = y_l;
    rx.b_in[nzi] = b_l_in; rx.b_out[nzi] = b_l_out; rx.relaxed[nzi] = relaxed_l;
    ++nzi;
  }
  g.z_lower_first = A_u ? 0 : 1;
  g.W = W;
  g.wpack = ((uintptr_t)w_packed & 15) == 0 ? w_packed : nullptr;
  g.S = S;
  return hwc_launch<true>(g, rx, nz, glds, "bf_crown_relu_conv_transpose", stream);
}

int bf_crown_relu_planes_conv_transpose(const float* A_u, const float* A_l, int64_t D, int64_t S, int Co, int Ho,
                                        int Wo, const float* alpha_u, const float* beta_u, const float* alpha_l,
                                        const float* beta_l, const float* kbias, const float* b_u_in,
                                        const float* b_l_in, const float* W, const float* w_packed, int Ci, int KH,
                                        int KW, int sh, int sw, int ph, int pw, int Hi, int Wi, float* y_u,
                                        float* y_l, float* b_u_out, float* b_l_out, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0 && Co > 0 && Ci > 0, "bf_crown_relu_planes_conv_transpose: bad sizes");
  const int64_t R = D * S;
  if (R == 0) return BF_OK;
  BF_REQUIRE(W && (A_u || A_l), "bf_crown_relu_planes_conv_transpose: null pointer");
  BF_REQUIRE(alpha_u && beta_u && alpha_l && beta_l, "bf_crown_relu_planes_conv_transpose: null relaxation plane");
  BF_REQUIRE((A_u == nullptr) == (y_u == nullptr) && (A_l == nullptr) == (y_l == nullptr),
             "bf_crown_relu_planes_conv_transpose: each given coefficient needs an output");
  const unsigned nz = (A_u && A_l) ? 2u : 1u;
  ConvRelax rx;
  memset(&rx, 0, sizeof(rx));
  rx.pl[0] = alpha_u;
  rx.pl[1] = beta_u;
  rx.pl[2] = alpha_l;
  rx.pl[3] = beta_l;
  rx.kbias = kbias;
  {
    // few output channels (an input layer): the tap-product kernel in its register form
    SmallTArgs sg;
    memset(&sg, 0, sizeof(sg));
    size_t slds = 0, flds = 0;
    if (!kSmallFastDisabled && conv_t_small_plan(sg, R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &slds) &&
        conv_t_small_fast_plan(sg, &flds)) {
      int nzi = 0;
      if (A_u) {
        sg.X[nzi] = A_u; sg.y[nzi] = y_u;
        rx.b_in[nzi] = b_u_in; rx.b_out[nzi] = b_u_out;
        ++nzi;
      }
      if (A_l) {
        sg.X[nzi] = A_l; sg.y[nzi] = y_l;
        rx.b_in[nzi] = b_l_in; rx.b_out[nzi] = b_l_out;
        ++nzi;
      }
      sg.z_lower_first = A_u ? 0 : 1;
      sg.W = W;
      sg.S = S;
      return small_t_launch<true>(sg, rx, nz, slds, "bf_crown_relu_planes_conv_transpose", stream);
    }
  }
  GatherArgs g;
  memset(&g, 0, sizeof(g));
  size_t glds = 0;
  if (!conv_t_hwc_plan(g, R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &glds)) {
    set_error("bf_crown_relu_planes_conv_transpose: shape not supported (bf_conv_transpose_hwc_supported)");
    return BF_EINVAL;
  }
  int nzi = 0;
  if (A_u) {
    g.X[nzi] = A_u; g.y[nzi] = y_u;
    rx.b_in[nzi] = b_u_in; rx.b_out[nzi] = b_u_out;
    ++nzi;
  }
  if (A_l) {
    g.X[nzi] = A_l; g.y[nzi] = y_l;
    rx.b_in[nzi] = b_l_in; rx.b_out[nzi] = b_l_out;
    ++nzi;
  }
  g.z_lower_first = A_u ? 0 : 1;
  g.W = W;
  g.wpack = ((uintptr_t)w_packed & 15) == 0 ? w_packed : nullptr;
  g.S = S;
  return hwc_launch<true>(g, rx, nz, glds, "bf_crown_relu_planes_conv_transpose", stream);
}

int bf_conv_transpose_small_supported(int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw, int ph,
                                      int pw, int Hi, int Wi) {
  if (Co <= 0 || Ci <= 0 || KH <= 0 || KW <= 0 || sh <= 0 || sw <= 0 || Hi <= 0 || Wi <= 0 || Ho <= 0 || Wo <= 0)
    return 0;
  SmallTArgs g;
  memset(&g, 0, sizeof(g));
  size_t lds = 0;
  return conv_t_small_plan(g, 1, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &lds) ? 1 : 0;
}

int bf_crown_relu_conv_transpose_concretize(const float* A_u, const float* A_l, int64_t D, int64_t S, int Co, int Ho,
                                            int Wo, const float* pre_lo, const float* pre_hi, const float* alpha,
                                            int64_t alpha_ld, const float* add_l, int64_t add_ld, const float* kbias,
                                            const float* cvec, const float* b_u_in, const float* b_l_in,
                                            const float* W, int Ci, int KH, int KW, int sh, int sw, int ph, int pw,
                                            int Hi, int Wi, const float* wvec, int64_t w_ld, int norm_p,
                                            const float* h_scale, float* h_out, float* norm_u, float* norm_l,
                                            float* b_u_out,
                                            float* b_l_out, float* c_u_out, float* c_l_out, float* relaxed_u,
                                            float* relaxed_l, float eps, float* lb, float* ub, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0 && Co > 0 && Ci > 0, "bf_crown_relu_conv_transpose_concretize: bad sizes");
  BF_REQUIRE((lb == nullptr || (A_l && norm_l && b_l_out && c_l_out)) &&
                 (ub == nullptr || (A_u && norm_u && b_u_out && c_u_out)),
             "bf_crown_relu_conv_transpose_concretize: a bound needs its coefficient, norm, bias and center outputs");
  const int64_t R = D * S;
  if (R == 0) return BF_OK;
  BF_REQUIRE(W && (A_u || A_l), "bf_crown_relu_conv_transpose_concretize: null pointer");
  BF_REQUIRE((A_u == nullptr) == (norm_u == nullptr) && (A_l == nullptr) == (norm_l == nullptr),
             "bf_crown_relu_conv_transpose_concretize: each given coefficient needs its norm output");
  BF_REQUIRE((pre_lo == nullptr) == (pre_hi == nullptr),
             "bf_crown_relu_conv_transpose_concretize: pre_lo and pre_hi go together");
  BF_REQUIRE(norm_p >= 0 && norm_p <= 2 && (norm_p == 0 || wvec == nullptr),
             "bf_crown_relu_conv_transpose_concretize: norm_p is 0, 1 or 2; 1 and 2 take no weights");
  BF_REQUIRE((h_out == nullptr) == (h_scale == nullptr) && (h_out == nullptr || norm_l != nullptr),
             "bf_crown_relu_conv_transpose_concretize: h_out needs h_scale and the lower norm");
  SmallTArgs g;
  memset(&g, 0, sizeof(g));
  size_t glds = 0;
  if (!conv_t_small_plan(g, R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, &glds)) {
    set_error("bf_crown_relu_conv_transpose_concretize: shape not supported (bf_conv_transpose_small_supported)");
    return BF_EINVAL;
  }
  const unsigned nz = (A_u && A_l) ? 2u : 1u;
  ConvRelax rx;
  memset(&rx, 0, sizeof(rx));
  rx.lo = pre_lo;
  rx.hi = pre_hi;
  rx.alpha = alpha;
  rx.alpha_ld = alpha_ld;
  rx.add = add_l;
  rx.add_ld = add_ld;
  rx.kbias = kbias;
  rx.cvec = cvec;
  int nzi = 0;
  if (A_u) {
    g.X[nzi] = A_u; g.nrm[nzi] = norm_u;
    rx.b_in[nzi] = b_u_in; rx.b_out[nzi] = b_u_out; rx.c_out[nzi] = c_u_out; rx.relaxed[nzi] = relaxed_u;
    ++nzi;
  }
  if (A_l) {
    g.X[nzi] = A_l; g.nrm[nzi] = norm_l;
    rx.b_in[nzi] = b_l_in; rx.b_out[nzi] = b_l_out; rx.c_out[nzi] = c_l_out; rx.relaxed[nzi] = relaxed_l;
    ++nzi;
  }
  g.z_lower_first = A_u ? 0 : 1;
  g.W = W;
  g.wv = wvec;
  g.w_ld = w_ld;
  g.nkind = norm_p;
  // L1/L2 seeds need each row's whole norm: the lower rows go to h_out, made into the seed after the launch
  const bool lp_seed = norm_p != 0 && h_out != nullptr;
  if (lp_seed) g.y[A_u ? 1 : 0] = h_out;
  g.h_scale = lp_seed ? nullptr : h_scale;
  g.h_out = lp_seed ? nullptr : h_out;
  g.S = S;
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  g.vec = (g.npix % 16 == 0) && al16(A_u) && al16(A_l) && al16(pre_lo) && al16(pre_hi) && al16(alpha) &&
          al16(add_l) && al16(kbias) && al16(cvec) && al16(relaxed_u) && al16(relaxed_l) &&
          (alpha == nullptr || alpha_ld % 4 == 0) && (add_l == nullptr || add_ld % 4 == 0) ? 1 : 0;
  {
    int zi = 0;
    if (A_u) g.bnd[zi++] = ub;
    if (A_l) g.bnd[zi++] = lb;
  }
  g.eps = eps;
  bool fast = false;
  const int rc = small_t_launch<true>(g, rx, nz, glds, "bf_crown_relu_conv_transpose_concretize", stream, &fast);
  if (rc) return rc;
  if (!fast && (lb || ub)) {
    // the generic kernel writes the norms, centers and biases: the bounds from them
    const int rcf = concretize_finalize(norm_u, norm_l, 1, R, c_u_out, c_l_out, b_u_out, b_l_out, eps, norm_p,
                                        lb, ub, stream);
    if (rcf) return rcf;
  }
  if (lp_seed) return lp_seed_rows(h_out, R, (int64_t)Ci * Hi * Wi, h_scale, norm_p, stream);
  return BF_OK;
}

// The center and radius products of an IBP conv layer in one launch of the forward
// gather-GEMM, the operands made from the input set while each row's map is staged
// (ivl: IVL_BOX [| IVL_RELU] from lo / hi, or IVL_BALL from the center and eps).  Returns
// BF_OK with *planned false, launching nothing, for shapes the gather-GEMM does not take.
static int conv2d_ivl_launch(const float* lo, const float* hi, int ivl, float eps, int64_t R, int Ci, int Hi, int Wi,
                             const float* W, int Co, int KH, int KW, int sh, int sw, int ph, int pw, int Ho, int Wo,
                             float* yc, float* yr, bool* planned, hipStream_t stream) {
  GatherArgs g;
  memset(&g, 0, sizeof(g));
  size_t glds = 0;
  *planned = conv_f_mfma_plan(g, R, Ci, Hi, Wi, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, &glds);
  if (!*planned) return BF_OK;
  g.X[0] = lo;
  g.X[1] = lo;
  g.y[0] = yc;
  g.y[1] = yr;
  g.W = W;
  g.abs_w = 2;   // the radius product takes |W|
  g.in_div = 1;
  g.S = 1;
  g.ivl = ivl;
  g.ivl_hi = hi;
  g.ivl_eps = eps;
  g.rows_per_wg = gather_rows_per_wg(R * 2);
  const int rpw = g.rows_per_wg;
  BF_REQUIRE((R + rpw - 1) / rpw < (1LL << 31), "conv2d: too many rows");
  hipLaunchKernelGGL(conv_mfma_kernel<MODE_F>, dim3((unsigned)((R + rpw - 1) / rpw), 2), dim3(GTM), glds, stream, g);
  BF_LAUNCH_CHECK("conv_mfma_kernel<conv2d, interval>");
  return BF_OK;
}

// IBP of a conv layer in one launch of conv_ibp_kernel; BF_OK with *planned false, launching
// nothing, for shapes it does not take (the two maps and this half's weights above 64 KB).
static int conv_ibp_fused_launch(const float* lo, const float* hi, int ivl, float eps, int64_t R, int Ci, int Hi,
                                 int Wi, const float* W, int Co, int KH, int KW, int sh, int sw, int ph, int pw,
                                 int Ho, int Wo, const IbpConvOut& o, bool* planned, hipStream_t stream) {
  GatherArgs g;
  memset(&g, 0, sizeof(g));
  size_t one_map_lds = 0;
  *planned = false;
  if (!conv_f_mfma_plan(g, R, Ci, Hi, Wi, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, &one_map_lds)) return BF_OK;
  const bool cb_split = g.nblk % 2 == 0;
  const int nloc = (cb_split ? g.nblk / 2 : g.nblk) * 16;
  const size_t map = (size_t)Ci * g.Hp * g.Wp;
  const size_t lds = sizeof(float) * ((size_t)g.Kc4 * nloc + g.Kc4 + 2 * map);
  if (lds > 64 * 1024) return BF_OK;
  *planned = true;
  g.X[0] = lo;
  g.W = W;
  g.ivl = ivl;
  g.ivl_hi = hi;
  g.ivl_eps = eps;
  g.rows_per_wg = gather_rows_per_wg(R * 2);
  const int rpw = g.rows_per_wg;
  BF_REQUIRE((R + rpw - 1) / rpw < (1LL << 31), "conv2d: too many rows");
  const dim3 grid((unsigned)((R + rpw - 1) / rpw), 2);
  if (cb_split)
    hipLaunchKernelGGL(conv_ibp_kernel<true>, grid, dim3(GTM), lds, stream, g, o);
  else
    hipLaunchKernelGGL(conv_ibp_kernel<false>, grid, dim3(GTM), lds, stream, g, o);
  BF_LAUNCH_CHECK("conv_ibp_kernel");
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
  bool planned = false;
  if (input_kind == 1 || in_hi) {
    // both products and the finalize in one launch
    IbpConvOut o;
    o.bias = bias;
    o.split = split;
    o.split_ld = split_ld;
    o.lo = out_lo;
    o.hi = out_hi;
    o.c_out = center_out;
    o.infeasible = infeasible;
    rc = conv_ibp_fused_launch(in_lo, in_hi, input_kind == 1 ? IVL_BALL : (IVL_BOX | (apply_relu ? IVL_RELU : 0)),
                               eps, B, Ci, Hi, Wi, W, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, o, &planned, stream);
    if (rc || planned) return rc;
  }
  // the center (W) and the radius (|W|) products in one launch, the center and radius made
  // from the input set while the gather-GEMM stages each row
  if (input_kind == 1 || in_hi) {
    rc = conv2d_ivl_launch(in_lo, in_hi, input_kind == 1 ? IVL_BALL : (IVL_BOX | (apply_relu ? IVL_RELU : 0)), eps, B,
                           Ci, Hi, Wi, W, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, cdst, r, &planned, stream);
    if (rc) return rc;
  }
  if (planned) {
    rc = BF_OK;
  } else if (input_kind == 1) {
    // center x0 conv W; the radius map is eps everywhere inside the image (padding has none)
    rc = fill_value(rad, B * nin, eps, stream);
    if (rc) return rc;
    rc = conv2d_launch(in_lo, 1, B, Ci, Hi, Wi, W, 0, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, cdst, nullptr, nullptr, 1, 0,
                       stream, rad, r, 1);
  } else {
    BF_REQUIRE(in_hi, "bf_ibp_conv2d: interval input needs in_hi");
    rc = ibp_center_radius(in_lo, in_hi, B * nin, apply_relu, mid, rad, stream);
    if (rc) return rc;
    rc = conv2d_launch(mid, 1, B, Ci, Hi, Wi, W, 0, Co, KH, KW, sh, sw, ph, pw, Ho, Wo, cdst, nullptr, nullptr, 1, 0,
                       stream, rad, r, 1);
  }
  if (rc) return rc;
  return ibp_finalize(cdst, r, nullptr, 0.f, bias, (int64_t)Ho * Wo, split, split_ld, B, nout, out_lo, out_hi,
                      infeasible, stream);
}

int64_t bf_ibp_conv2d_workspace(int64_t B, int64_t nin, int64_t nout) { return 2 * B * nin + 2 * B * nout; }

}  // extern "C"
