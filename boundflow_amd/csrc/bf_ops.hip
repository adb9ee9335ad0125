// Bandwidth-bound kernels and the C-ABI of the boundflow HIP library.
//
// Every extern "C" entry point takes device pointers, int64 sizes, scalar
// parameters and a hipStream_t; it launches asynchronously on that stream,
// never allocates or synchronizes, and returns 0 on success or a nonzero
// status with a message retrievable through bf_last_error().

#include "bf_common.h"

#include <cstring>
#include <mutex>

namespace bf {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace bf

#include "bf_gemm_args.h"

namespace bf {

int gemm_dispatch(const GemmArgs& a, int pro, int epi, int nz, hipStream_t stream);
int gemm_tile_choice(int64_t M, int64_t N, int nz, int64_t ks, int pro, bool dl);
int concretize_finalize(const float* pu, const float* pl, int nparts, int64_t M, const float* cu, const float* cl,
                        const float* bu, const float* bl, float eps, int norm_p, float* lb, float* ub,
                        hipStream_t stream);
int gemm_partial_count(int64_t N);
int gemm_norm_partial_count(int64_t M, int64_t N, int pro);
int rows_finalize(const float* b_src, const float* pb, const float* pc, int nparts, int64_t M, float* b_out,
                  float* c_out, hipStream_t stream);
int gemm_ksplit(int64_t M, int64_t N, int64_t K, int64_t* kchunk);
int splitk_reduce(const float* part, int ks, int64_t M, int64_t N, float* C, int64_t ldc, const float* r_row,
                  const float* v_col, int64_t v_ld, int64_t S, hipStream_t stream);
int relax_table(const float* lo, const float* hi, const float* alpha, int64_t alpha_ld, int64_t D, int64_t K,
                float4* out, hipStream_t stream);
int relax_table_multi(int count, const float* const* lo, const float* const* hi, const float* const* alpha,
                      const int64_t* alpha_ld, int64_t D, const int64_t* K, float* const* out, hipStream_t stream);
int lp_seed_rows(float* h, int64_t M, int64_t I, const float* h_scale, int norm_p, hipStream_t stream);

// ---------------------------------------------------------------------------
// IBP helpers (center/radius form)

// mid = (relu?(l) + relu?(u)) / 2, rad = (relu?(u) - relu?(l)) / 2
__global__ void ibp_center_radius_kernel(const float* __restrict__ lo, const float* __restrict__ hi, int64_t n,
                                         int apply_relu, float* __restrict__ mid, float* __restrict__ rad) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float l = lo[i], u = hi[i];
  if (apply_relu) {
    l = fmaxf(l, 0.f);
    u = fmaxf(u, 0.f);
  }
  if (mid) mid[i] = (l + u) / 2.0f;
  if (rad) rad[i] = (u - l) / 2.0f;
}

int ibp_center_radius(const float* lo, const float* hi, int64_t n, int apply_relu, float* mid, float* rad,
                      hipStream_t stream) {
  if (n == 0) return BF_OK;
  hipLaunchKernelGGL(ibp_center_radius_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, lo, hi, n,
                     apply_relu, mid, rad);
  BF_LAUNCH_CHECK("ibp_center_radius_kernel");
  return BF_OK;
}

// Row norm of the input layer's weight under the input ball (perturbation.py:127-136):
// kind 0 sum_i |W[o, i]| (Linf ball), 1 max_i |W[o, i]| (L1 ball), 2 sqrt(sum_i W[o, i]^2) (L2 ball);
// the per-thread partials combined by a fixed tree.
__global__ void row_norm_kernel(const float* __restrict__ W, int64_t O, int64_t I, int kind, float* __restrict__ out) {
  int64_t o = (int64_t)blockIdx.x;
  if (o >= O) return;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < I; i += blockDim.x) {
    const float w = W[o * I + i];
    s = kind == 1 ? fmaxf(s, fabsf(w)) : (kind == 2 ? s + w * w : s + fabsf(w));
  }
  __shared__ float sh[256];
  sh[threadIdx.x] = s;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w)
      sh[threadIdx.x] = kind == 1 ? fmaxf(sh[threadIdx.x], sh[threadIdx.x + w]) : sh[threadIdx.x] + sh[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[o] = kind == 2 ? sqrtf(sh[0]) : sh[0];
}

// lo = (c - dev) + b, hi = (c + dev) + b, then the ReLU split of the consumer
// (crown_ibp.py:70-98): active -> lo = max(lo, 0); inactive -> hi = min(hi, 0);
// a domain with lo > hi anywhere is flagged infeasible.  With `part`, c (and r
// when two products were taken) are the split-K partial products [z][s][B*N],
// summed here in chunk order (the order of splitk_reduce_kernel), and c is also
// written to c_out when given.
__global__ void ibp_finalize_kernel(const float* __restrict__ c, const float* __restrict__ r,
                                    const float* __restrict__ part, int ks, int two, float* __restrict__ c_out,
                                    const float* __restrict__ rownorm, float eps, const float* __restrict__ bias,
                                    int64_t bias_div, const int8_t* __restrict__ split, int64_t split_ld, int64_t B,
                                    int64_t N, float* __restrict__ lo, float* __restrict__ hi,
                                    int* __restrict__ infeasible) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * N) return;
  const int64_t b = div_rows(i, N, B * N < (1LL << 31)), n = i - b * N;
  float cv, rv = 0.f;
  if (part) {
    // the K chunks summed in order, their loads issued eight at a time
    const int64_t BN = B * N;
    const float* __restrict__ pc = part + i;
    const float* __restrict__ pr = part + (int64_t)ks * BN + i;
    cv = pc[0];
    if (two) rv = pr[0];
    int s = 1;
    for (; s + 8 <= ks; s += 8) {
      float tc[8], tr[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        tc[q] = pc[(int64_t)(s + q) * BN];
        tr[q] = two ? pr[(int64_t)(s + q) * BN] : 0.f;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        cv += tc[q];
        rv += tr[q];
      }
    }
    for (; s < ks; ++s) {
      cv += pc[(int64_t)s * BN];
      if (two) rv += pr[(int64_t)s * BN];
    }
    if (c_out) c_out[i] = cv;
  } else {
    cv = c[i];
    if (r) rv = r[i];
  }
  float dev = rownorm ? eps * rownorm[n] : rv;
  float l = cv - dev;
  float u = cv + dev;
  if (bias) {
    l = l + bias[n / bias_div];
    u = u + bias[n / bias_div];
  }
  if (split) {
    int8_t s = split[b * split_ld + n];
    if (s > 0) l = fmaxf(l, 0.f);
    if (s < 0) u = fminf(u, 0.f);
    if (l > u && infeasible) infeasible[b] = 1;
  }
  lo[i] = l;
  hi[i] = u;
}

// Products of a small output (few 16 x 16 tiles: a small batch) in one launch, with no
// split of the reduction: workgroup t owns output tile t (16 rows x 16 columns) and takes
// the whole reduction, its 16 waves taking the 16-wide steps of k in turn (wave w: steps
// w, w + 16, ...; the loads of four steps issued together).  The waves' partial tiles are
// added in LDS in wave order and the workgroup applies the epilogue, so no partial buffer
// and no second launch is needed.  Modes:
//  * SM_INTERVAL / SM_BALL -- IBP of a linear layer: the center Xc . W^T and the radius
//    Xr . |W|^T of an interval input (center and radius made from [lo, hi] as they are
//    loaded, of the ReLU when relu, with the arithmetic of ibp_center_radius_kernel), or
//    the center and eps times the row norm of W (norm code nk as row_norm_kernel) of a
//    ball; the epilogue is ibp_finalize_kernel's arithmetic.  With rad_out (interval
//    input without ReLU) the first column of tiles also writes the box radius.
//  * SM_GEMM -- C = A . W^T (+ r_row[m] v_col[(m / S) v_ld + n]), the rank-1 term added
//    as splitk_reduce_kernel adds it.
typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr int ISM_WAVES = 16;
constexpr int ISM_GROUP = 4;
constexpr int64_t ISM_MAX_TILES = 1024;
enum : int { SM_INTERVAL = 0, SM_BALL = 1, SM_GEMM = 2 };

struct SmallOutArgs {
  const float* lo;        // left operand rows (the interval's lower bounds, the ball's center, or A)
  const float* hi;        // the interval's upper bounds (SM_INTERVAL)
  int64_t lda;            // row stride of lo / hi
  const float* W;         // [N, ldw] rows
  int64_t ldw;
  int64_t B, K, N;        // output rows, reduction, output columns
  int relu, nk;
  float eps;
  const float* bias;      // IBP outputs
  const int8_t* split;
  int64_t split_ld;
  float* out_lo;
  float* out_hi;
  float* c_out;
  int* infeasible;
  float* rad_out;
  float* C;               // SM_GEMM output
  int64_t ldc;
  const float* r_row;
  const float* v_col;
  int64_t v_ld, S;
};

// Four k of one row, zero where ok is false or k runs past K.  Branch-free: every load is
// issued (from a clamped address inside the row) and masked afterwards, so the loads of a
// group stay in flight together.  VEC: K % 4 == 0 and 16-byte rows (a quad is whole or past K).
template <bool VEC>
__device__ __forceinline__ float4 ism_load4(const float* __restrict__ p, int64_t k, int64_t K, bool ok) {
  if constexpr (VEC) {
    const bool in = ok && k < K;
    const float4 v = *reinterpret_cast<const float4*>(p + (in ? k : 0));
    return in ? v : make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    const bool i0 = ok && k < K, i1 = ok && k + 1 < K, i2 = ok && k + 2 < K, i3 = ok && k + 3 < K;
    const float x0 = p[i0 ? k : 0], x1 = p[i1 ? k + 1 : 0], x2 = p[i2 ? k + 2 : 0], x3 = p[i3 ? k + 3 : 0];
    return make_float4(i0 ? x0 : 0.f, i1 ? x1 : 0.f, i2 ? x2 : 0.f, i3 ? x3 : 0.f);
  }
}

__device__ __forceinline__ float ism_center(float l, float u, bool relu) {
  if (relu) {
    l = fmaxf(l, 0.f);
    u = fmaxf(u, 0.f);
  }
  return (l + u) / 2.0f;
}
__device__ __forceinline__ float ism_radius(float l, float u, bool relu) {
  if (relu) {
    l = fmaxf(l, 0.f);
    u = fmaxf(u, 0.f);
  }
  return (u - l) / 2.0f;
}
__device__ __forceinline__ float ism_norm_step(float s, float w, int nk) {
  return nk == 1 ? fmaxf(s, fabsf(w)) : (nk == 2 ? s + w * w : s + fabsf(w));
}

template <int MODE, bool VEC>
__global__ void __launch_bounds__(64 * ISM_WAVES)
small_out_kernel(SmallOutArgs a) {
  constexpr bool BALL = MODE == SM_BALL, IVL = MODE == SM_INTERVAL;
  __shared__ float red_c[ISM_WAVES][256];
  __shared__ float red_r[IVL ? ISM_WAVES : 1][256];
  __shared__ float red_n[BALL ? ISM_WAVES : 1][64];
  const int64_t B = a.B, K = a.K, N = a.N;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t ntn = (N + 15) / 16;
  const int64_t b0 = (int64_t)(blockIdx.x / ntn) * 16, n0 = (int64_t)(blockIdx.x % ntn) * 16;
  // MFMA lanes: i = lane & 15 is the row of the A operand and the column of the B
  // operand, g = lane >> 4 the k slot; a lane's float4 at k = 16 s + 4 g holds the four
  // k of its slot for the four MFMAs of step s
  const int i = lane & 15, g = lane >> 4;
  const bool bok = b0 + i < B, nok = n0 + i < N;
  const bool rl = a.relu != 0;
  const float* __restrict__ xl = a.lo + (bok ? b0 + i : 0) * a.lda;
  const float* __restrict__ xh = IVL ? a.hi + (bok ? b0 + i : 0) * a.lda : a.lo;
  const float* __restrict__ wr = a.W + (nok ? n0 + i : 0) * a.ldw;
  floatx4 acc_c = {0.f, 0.f, 0.f, 0.f};
  floatx4 acc_r = {0.f, 0.f, 0.f, 0.f};
  float nrm = 0.f;
  const int64_t nsteps = (K + 15) / 16;
  // rad_out (interval input without ReLU): the first column of tiles writes the box radius
  // (u - l) / 2 of its rows from the loaded bounds (the arithmetic of ibp_center_radius_kernel)
  const bool put_rad = IVL && a.rad_out != nullptr && n0 == 0 && bok;
  float* __restrict__ rrow = put_rad ? a.rad_out + (b0 + i) * K : nullptr;
  for (int64_t s0 = wave; s0 < nsteps; s0 += (int64_t)ISM_WAVES * ISM_GROUP) {
    float4 al[ISM_GROUP], ah[ISM_GROUP], w4[ISM_GROUP];
#pragma unroll
    for (int q = 0; q < ISM_GROUP; ++q) {
      const int64_t s = s0 + (int64_t)q * ISM_WAVES;
      const int64_t k = s * 16 + 4 * g;
      const bool sok = s < nsteps;
      al[q] = ism_load4<VEC>(xl, k, K, bok && sok);
      if (IVL) ah[q] = ism_load4<VEC>(xh, k, K, bok && sok);
      w4[q] = ism_load4<VEC>(wr, k, K, nok && sok);
    }
#pragma unroll
    for (int q = 0; q < ISM_GROUP; ++q) {
      if constexpr (!IVL) {
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(al[q].x, w4[q].x, acc_c, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(al[q].y, w4[q].y, acc_c, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(al[q].z, w4[q].z, acc_c, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(al[q].w, w4[q].w, acc_c, 0, 0, 0);
        if constexpr (BALL) {
          nrm = ism_norm_step(nrm, w4[q].x, a.nk);
          nrm = ism_norm_step(nrm, w4[q].y, a.nk);
          nrm = ism_norm_step(nrm, w4[q].z, a.nk);
          nrm = ism_norm_step(nrm, w4[q].w, a.nk);
        }
      } else {
        if (put_rad) {
          const int64_t k = (s0 + (int64_t)q * ISM_WAVES) * 16 + 4 * g;
          const float4 rv = make_float4(ism_radius(al[q].x, ah[q].x, false), ism_radius(al[q].y, ah[q].y, false),
                                        ism_radius(al[q].z, ah[q].z, false), ism_radius(al[q].w, ah[q].w, false));
          if constexpr (VEC) {
            if (k < K) *reinterpret_cast<float4*>(rrow + k) = rv;
          } else {
            if (k + 0 < K) rrow[k + 0] = rv.x;
            if (k + 1 < K) rrow[k + 1] = rv.y;
            if (k + 2 < K) rrow[k + 2] = rv.z;
            if (k + 3 < K) rrow[k + 3] = rv.w;
          }
        }
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(ism_center(al[q].x, ah[q].x, rl), w4[q].x, acc_c, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(ism_center(al[q].y, ah[q].y, rl), w4[q].y, acc_c, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(ism_center(al[q].z, ah[q].z, rl), w4[q].z, acc_c, 0, 0, 0);
        acc_c = __builtin_amdgcn_mfma_f32_16x16x4f32(ism_center(al[q].w, ah[q].w, rl), w4[q].w, acc_c, 0, 0, 0);
        acc_r = __builtin_amdgcn_mfma_f32_16x16x4f32(ism_radius(al[q].x, ah[q].x, rl), fabsf(w4[q].x), acc_r, 0, 0, 0);
        acc_r = __builtin_amdgcn_mfma_f32_16x16x4f32(ism_radius(al[q].y, ah[q].y, rl), fabsf(w4[q].y), acc_r, 0, 0, 0);
        acc_r = __builtin_amdgcn_mfma_f32_16x16x4f32(ism_radius(al[q].z, ah[q].z, rl), fabsf(w4[q].z), acc_r, 0, 0, 0);
        acc_r = __builtin_amdgcn_mfma_f32_16x16x4f32(ism_radius(al[q].w, ah[q].w, rl), fabsf(w4[q].w), acc_r, 0, 0, 0);
      }
    }
  }
  // lane's acc[r] is tile element (row 4 g + r, column i)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    red_c[wave][(4 * g + r) * 16 + i] = acc_c[r];
    if constexpr (IVL) red_r[wave][(4 * g + r) * 16 + i] = acc_r[r];
  }
  if constexpr (BALL) red_n[wave][lane] = nrm;
  __syncthreads();
  if (tid >= 256) return;
  const int mr = tid >> 4, nc = tid & 15;
  const int64_t b = b0 + mr, n = n0 + nc;
  float cv = red_c[0][tid];
  for (int w = 1; w < ISM_WAVES; ++w) cv += red_c[w][tid];
  if constexpr (MODE == SM_GEMM) {
    if (b >= B || n >= N) return;
    float v = cv;
    if (a.r_row) v = v + a.r_row[b] * a.v_col[(b / a.S) * a.v_ld + n];
    a.C[b * a.ldc + n] = v;
  } else {
    float dev;
    if constexpr (BALL) {
      float sn = 0.f;
      for (int w = 0; w < ISM_WAVES; ++w)
        for (int q = 0; q < 4; ++q) {
          const float v = red_n[w][16 * q + nc];
          sn = a.nk == 1 ? fmaxf(sn, v) : sn + v;
        }
      dev = a.eps * (a.nk == 2 ? sqrtf(sn) : sn);
    } else {
      dev = red_r[0][tid];
      for (int w = 1; w < ISM_WAVES; ++w) dev += red_r[w][tid];
    }
    if (b >= B || n >= N) return;
    float l = cv - dev;
    float u = cv + dev;
    if (a.bias) {
      l = l + a.bias[n];
      u = u + a.bias[n];
    }
    if (a.split) {
      const int8_t sp = a.split[b * a.split_ld + n];
      if (sp > 0) l = fmaxf(l, 0.f);
      if (sp < 0) u = fminf(u, 0.f);
      if (l > u && a.infeasible) a.infeasible[b] = 1;
    }
    const int64_t o = b * N + n;
    a.out_lo[o] = l;
    a.out_hi[o] = u;
    if (a.c_out) a.c_out[o] = cv;
  }
}

// True when small_out_kernel takes a B x N output.
bool small_out_route(int64_t B, int64_t N) { return ceil_div(B, 16) * ceil_div(N, 16) <= ISM_MAX_TILES; }

static int small_out_launch(int mode, const SmallOutArgs& a, hipStream_t stream) {
  const unsigned tiles = (unsigned)(ceil_div(a.B, 16) * ceil_div(a.N, 16));
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool vec = (a.K % 4 == 0) && (a.lda % 4 == 0) && (a.ldw % 4 == 0) && al16(a.lo) && al16(a.hi) && al16(a.W) &&
                   al16(a.rad_out);
  auto launch = [&](auto kern) { hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * ISM_WAVES), 0, stream, a); };
  if (mode == SM_INTERVAL) {
    if (vec) launch(small_out_kernel<SM_INTERVAL, true>);
    else launch(small_out_kernel<SM_INTERVAL, false>);
  } else if (mode == SM_BALL) {
    if (vec) launch(small_out_kernel<SM_BALL, true>);
    else launch(small_out_kernel<SM_BALL, false>);
  } else {
    if (vec) launch(small_out_kernel<SM_GEMM, true>);
    else launch(small_out_kernel<SM_GEMM, false>);
  }
  BF_LAUNCH_CHECK("small_out_kernel");
  return BF_OK;
}

int ibp_linear_small(const float* lo, const float* hi, int relu, int nk, float eps, const float* W, const float* bias,
                     int64_t B, int64_t K, int64_t N, const int8_t* split, int64_t split_ld, float* out_lo,
                     float* out_hi, float* c_out, int* infeasible, float* rad_out, hipStream_t stream) {
  SmallOutArgs a;
  memset(&a, 0, sizeof(a));
  a.lo = lo;
  a.hi = hi;
  a.lda = K;
  a.W = W;
  a.ldw = K;
  a.B = B;
  a.K = K;
  a.N = N;
  a.relu = relu;
  a.nk = nk;
  a.eps = eps;
  a.bias = bias;
  a.split = split;
  a.split_ld = split_ld;
  a.out_lo = out_lo;
  a.out_hi = out_hi;
  a.c_out = c_out;
  a.infeasible = infeasible;
  a.rad_out = rad_out;
  return small_out_launch(hi ? SM_INTERVAL : SM_BALL, a, stream);
}

// The relaxation table {alpha_u, beta_u, alpha_l, beta_l} from the four separate tensors
// of a FusedReluAffineRequest: one 16-byte store per entry.
__global__ void planes_table_kernel(const float* __restrict__ au, const float* __restrict__ bu,
                                    const float* __restrict__ al, const float* __restrict__ bl, int64_t n,
                                    float4* __restrict__ table) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) table[i] = make_float4(au[i], bu[i], al[i], bl[i]);
}

__global__ void fill_kernel(float* __restrict__ p, int64_t n, float v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

int fill_value(float* p, int64_t n, float v, hipStream_t stream) {
  if (n == 0) return BF_OK;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, p, n, v);
  BF_LAUNCH_CHECK("fill_kernel");
  return BF_OK;
}

int ibp_center_radius(const float* lo, const float* hi, int64_t n, int apply_relu, float* mid, float* rad,
                      hipStream_t stream);

static int ibp_finalize_parts(const float* c, const float* r, const float* part, int ks, int two, float* c_out,
                              const float* rownorm, float eps, const float* bias, int64_t bias_div,
                              const int8_t* split, int64_t split_ld, int64_t B, int64_t N, float* lo, float* hi,
                              int* infeasible, hipStream_t stream) {
  if (B * N == 0) return BF_OK;
  hipLaunchKernelGGL(ibp_finalize_kernel, dim3((unsigned)ceil_div(B * N, 256)), dim3(256), 0, stream, c, r, part, ks,
                     two, c_out, rownorm, eps, bias, bias_div, split, split_ld, B, N, lo, hi, infeasible);
  BF_LAUNCH_CHECK("ibp_finalize_kernel");
  return BF_OK;
}

int ibp_finalize(const float* c, const float* r, const float* rownorm, float eps, const float* bias,
                 int64_t bias_div, const int8_t* split, int64_t split_ld, int64_t B, int64_t N, float* lo, float* hi,
                 int* infeasible, hipStream_t stream) {
  return ibp_finalize_parts(c, r, nullptr, 1, 0, nullptr, rownorm, eps, bias, bias_div, split, split_ld, B, N, lo,
                            hi, infeasible, stream);
}

// Intersect with external constraints (crown_ibp.py:186-209) and apply a split.
__global__ void interval_clip_kernel(float* __restrict__ lo, float* __restrict__ hi, const float* __restrict__ clo,
                                     const float* __restrict__ chi, const int8_t* __restrict__ split,
                                     int64_t split_ld, int64_t B, int64_t N, int* __restrict__ infeasible) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * N) return;
  int64_t b = i / N, n = i % N;
  float l = lo[i], u = hi[i];
  if (clo) {
    l = fmaxf(l, clo[i]);
    u = fminf(u, chi[i]);
  }
  if (split) {
    int8_t s = split[b * split_ld + n];
    if (s > 0) l = fmaxf(l, 0.f);
    if (s < 0) u = fminf(u, 0.f);
  }
  if (l > u && infeasible) infeasible[b] = 1;
  lo[i] = l;
  hi[i] = u;
}

// ---------------------------------------------------------------------------
// Op-by-op interval kernels of the IBP task executor
// (boundflow/runtime/task_executor.py:360-563).

// relu(l), relu(u)  (domains/interval.py:88-91)
__global__ void interval_relu_kernel(const float* __restrict__ lo, const float* __restrict__ hi, int64_t n,
                                     float* __restrict__ olo, float* __restrict__ ohi) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  olo[i] = fmaxf(lo[i], 0.f);
  ohi[i] = fmaxf(hi[i], 0.f);
}

// [a_l + b_l, a_u + b_u]  (task_executor.py:476-490)
__global__ void interval_add_kernel(const float* __restrict__ alo, const float* __restrict__ ahi,
                                    const float* __restrict__ blo, const float* __restrict__ bhi, int64_t n,
                                    float* __restrict__ olo, float* __restrict__ ohi) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  olo[i] = alo[i] + blo[i];
  ohi[i] = ahi[i] + bhi[i];
}

// Interval product (domains/interval.py:102-112): min / max over the four endpoint
// products; a NaN among them propagates, as in torch.min / torch.max over a stack.
__device__ __forceinline__ float nan_min(float m, float c) { return (c < m || c != c) ? c : m; }
__device__ __forceinline__ float nan_max(float m, float c) { return (c > m || c != c) ? c : m; }

__global__ void interval_mul_kernel(const float* __restrict__ alo, const float* __restrict__ ahi,
                                    const float* __restrict__ blo, const float* __restrict__ bhi, int64_t n,
                                    float* __restrict__ olo, float* __restrict__ ohi) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float al = alo[i], au = ahi[i], bl = blo[i], bu = bhi[i];
  const float c0 = al * bl, c1 = al * bu, c2 = au * bl, c3 = au * bu;
  olo[i] = nan_min(nan_min(nan_min(c0, c1), c2), c3);
  ohi[i] = nan_max(nan_max(nan_max(c0, c1), c2), c3);
}

// spec_linear (task_executor.py:423-439): lb = sum_o C+ l + C- u, ub = sum_o C+ u + C- l; one thread per (b, s)
__global__ void spec_linear_kernel(const float* __restrict__ C, const float* __restrict__ lo,
                                   const float* __restrict__ hi, int64_t B, int64_t S, int64_t O,
                                   float* __restrict__ olo, float* __restrict__ ohi) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * S) return;
  const int64_t b = i / S;
  float sl = 0.f, su = 0.f;
  for (int64_t o = 0; o < O; ++o) {
    const float c = C[i * O + o];
    const float cp = fmaxf(c, 0.f), cn = fminf(c, 0.f);
    const float l = lo[b * O + o], u = hi[b * O + o];
    sl += cp * l + cn * u;
    su += cp * u + cn * l;
  }
  olo[i] = sl;
  ohi[i] = su;
}

// Batched linear with per-sample weights W[b] [O, I] (the spec-fused last layer of
// planner/interval_v1.py:85-164), center/radius form (task_executor.py:445-458):
// lb = mid . W[b, o] - rad . |W[b, o]| + bias[b, o].  One wave64 per (b, o).
__global__ void __launch_bounds__(256)
ibp_batched_linear_kernel(const float* __restrict__ lo, const float* __restrict__ hi, int64_t B, int64_t I,
                          const float* __restrict__ W, const float* __restrict__ bias, int64_t O,
                          float* __restrict__ olo, float* __restrict__ ohi) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r >= B * O) return;
  const int64_t b = r / O;
  float c = 0.f, d = 0.f;
  for (int64_t i = lane; i < I; i += 64) {
    const float l = lo[b * I + i], u = hi[b * I + i];
    const float mid = (l + u) / 2.0f, rad = (u - l) / 2.0f;
    const float w = W[r * I + i];
    c += mid * w;
    d += rad * fabsf(w);
  }
  for (int off = 32; off >= 1; off >>= 1) {
    c += __shfl_xor(c, off, 64);
    d += __shfl_xor(d, off, 64);
  }
  if (lane == 0) {
    const float bb = bias ? bias[r] : 0.f;
    olo[r] = (c - d) + bb;
    ohi[r] = (c + d) + bb;
  }
}

// ---------------------------------------------------------------------------
// Where a relaxation pass reads the slopes/intercepts {alpha_u, beta_u, alpha_l,
// beta_l} of (domain d, neuron k): a table of bf_relu_relax_table, or computed in
// place from the pre-activation box [lo, hi] and the optional lower-slope
// override with the table kernel's own arithmetic (relu_relax), which reads 8-12
// contiguous bytes per neuron instead of a 16-byte entry.  Neither: identity.
struct RelaxSrc {
  const float4* table;   // [D, K]
  const float* lo;       // [D, K]
  const float* hi;
  const float* alpha;    // [D, K] (alpha_ld K) or shared (alpha_ld 0)
  int64_t alpha_ld;

  __device__ __forceinline__ float4 at(int64_t d, int64_t K, int64_t k) const {
    if (table) return table[d * K + k];
    if (!lo) return make_float4(1.f, 0.f, 1.f, 0.f);
    const bool has_alpha = alpha != nullptr;
    const Relax r = relu_relax(lo[d * K + k], hi[d * K + k], has_alpha,
                               has_alpha ? clamp01(alpha[d * alpha_ld + k]) : 0.f);
    return make_float4(r.au, r.bu, r.al, r.bl);
  }

  // entries of k .. k + 3 (16-byte aligned operands)
  __device__ __forceinline__ void quad(int64_t d, int64_t K, int64_t k, float4 (&e)[4]) const {
    if (table) {
#pragma unroll
      for (int q = 0; q < 4; ++q) e[q] = table[d * K + k + q];
      return;
    }
    if (!lo) {
#pragma unroll
      for (int q = 0; q < 4; ++q) e[q] = make_float4(1.f, 0.f, 1.f, 0.f);
      return;
    }
    const float4 l4 = *reinterpret_cast<const float4*>(lo + d * K + k);
    const float4 u4 = *reinterpret_cast<const float4*>(hi + d * K + k);
    const bool has_alpha = alpha != nullptr;
    const float4 a4 = has_alpha ? *reinterpret_cast<const float4*>(alpha + d * alpha_ld + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, uv[4] = {u4.x, u4.y, u4.z, u4.w}, av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const Relax r = relu_relax(lv[q], uv[q], has_alpha, has_alpha ? clamp01(av[q]) : 0.f);
      e[q] = make_float4(r.au, r.bu, r.al, r.bl);
    }
  }
};

// ---------------------------------------------------------------------------
// Standalone ReLU relaxation pass (north-star kernel #3 in its unfused form):
// one wave64 per coefficient row, float loads strided by 64 lanes, wave
// reduction of the bias terms.  Writes A' for both bounds and
//   b_out = (b_in + sum_k A * beta_sel)  [+ sum_k A' * kbias if kbias].
__global__ void __launch_bounds__(256)
relu_relax_rows_kernel(const float* __restrict__ Au, const float* __restrict__ Al, int64_t a_dstride, int64_t M,
                       int64_t S, int64_t K,
                       RelaxSrc relax, const float* __restrict__ add_l, int64_t add_ld,
                       const float* __restrict__ kbias, const float* __restrict__ cvec,
                       const float* __restrict__ bu_in, const float* __restrict__ bl_in, float* __restrict__ Au_out,
                       float* __restrict__ Al_out, float* __restrict__ bu_out, float* __restrict__ bl_out,
                       float* __restrict__ cu_out, float* __restrict__ cl_out) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (m >= M) return;
  const int64_t d = m / S;
  const int64_t a_row = d * a_dstride + (m - d * S) * K;   // input row (shared by all domains when a_dstride = 0)
  float su = 0.f, sl = 0.f, ku = 0.f, kl = 0.f, cu = 0.f, cl = 0.f;
  for (int64_t k = lane; k < K; k += 64) {
    // {alpha_u, beta_u, alpha_l, beta_l}; no source = no ReLU (identity)
    const float4 r = relax.at(d, K, k);
    if (Au) {
      float v = Au[a_row + k];
      bool nn = v >= 0.f;
      float o = v * (nn ? r.x : r.z);
      su += v * (nn ? r.y : r.w);
      if (kbias) ku += o * kbias[k];
      if (cvec) cu += o * cvec[d * K + k];
      if (Au_out) Au_out[m * K + k] = o;
    }
    if (Al) {
      float v = Al[a_row + k];
      bool nn = v >= 0.f;
      float o = v * (nn ? r.z : r.x);
      sl += v * (nn ? r.w : r.y);
      if (add_l) o = o + add_l[d * add_ld + k];
      if (kbias) kl += o * kbias[k];
      if (cvec) cl += o * cvec[d * K + k];
      if (Al_out) Al_out[m * K + k] = o;
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    su += __shfl_xor(su, off, 64);
    sl += __shfl_xor(sl, off, 64);
    ku += __shfl_xor(ku, off, 64);
    kl += __shfl_xor(kl, off, 64);
    cu += __shfl_xor(cu, off, 64);
    cl += __shfl_xor(cl, off, 64);
  }
  if (lane == 0) {
    if (bu_out) bu_out[m] = ((bu_in ? bu_in[m] : 0.f) + su) + ku;
    if (bl_out) bl_out[m] = ((bl_in ? bl_in[m] : 0.f) + sl) + kl;
    if (cu_out) cu_out[m] = cu;
    if (cl_out) cl_out[m] = cl;
  }
}

// The same pass, vectorized: TPR threads per row (256 / TPR rows per
// workgroup), each thread handling 4 consecutive k per step, so a row of K
// coefficients is covered in ceil(K / (4 TPR)) steps with two 16-byte loads per
// bound and four table entries in flight per thread.  Needs K % 4 == 0 and
// 16-byte aligned rows.  Row sums: per-thread partials in k order, then a fixed
// tree (wave shuffles, then the workgroup's waves through LDS when TPR > 64).
template <int TPR>
__global__ void __launch_bounds__(256)
relu_relax_rows4_kernel(const float* __restrict__ Au, const float* __restrict__ Al, int64_t a_dstride, int64_t M,
                        int64_t S, int64_t K,
                        RelaxSrc relax, const float* __restrict__ add_l, int64_t add_ld,
                        const float* __restrict__ kbias, const float* __restrict__ cvec,
                        const float* __restrict__ bu_in, const float* __restrict__ bl_in, float* __restrict__ Au_out,
                        float* __restrict__ Al_out, float* __restrict__ bu_out, float* __restrict__ bl_out,
                        float* __restrict__ cu_out, float* __restrict__ cl_out) {
  constexpr int RPB = 256 / TPR;   // rows per workgroup
  constexpr int WPR = TPR / 64;    // waves per row
  __shared__ float red[6][256 / 64];
  const int t = threadIdx.x % TPR;
  // the row is uniform per wave (TPR >= 64): its index and address arithmetic stay scalar
  const int64_t m = (int64_t)blockIdx.x * RPB + __builtin_amdgcn_readfirstlane(threadIdx.x / TPR);
  const bool live = m < M;
  float s[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};   // su, sl, ku, kl, cu, cl
  if (live) {
    const int64_t d = div_rows(m, S, M < (1LL << 31));
    const int64_t a_row = d * a_dstride + (m - d * S) * K;   // input row (shared by all domains when a_dstride = 0)
    for (int64_t k = 4 * (int64_t)t; k < K; k += 4 * TPR) {
      float4 r[4];
      relax.quad(d, K, k, r);
      const float4 kb = kbias ? *reinterpret_cast<const float4*>(kbias + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 cv = cvec ? *reinterpret_cast<const float4*>(cvec + d * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float kbv[4] = {kb.x, kb.y, kb.z, kb.w};
      const float cvv[4] = {cv.x, cv.y, cv.z, cv.w};
      // one load serves both bounds when they share the coefficient (the first region of a C = I query)
      const float4 vu4 = Au ? *reinterpret_cast<const float4*>(Au + a_row + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      if (Au) {
        const float4 v4 = vu4;
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool nn = v[e] >= 0.f;
          o[e] = v[e] * (nn ? r[e].x : r[e].z);
          s[0] += v[e] * (nn ? r[e].y : r[e].w);
          if (kbias) s[2] += o[e] * kbv[e];
          if (cvec) s[4] += o[e] * cvv[e];
        }
        if (Au_out) *reinterpret_cast<float4*>(Au_out + m * K + k) = make_float4(o[0], o[1], o[2], o[3]);
      }
      if (Al) {
        const float4 v4 = Al == Au ? vu4 : *reinterpret_cast<const float4*>(Al + a_row + k);
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        const float4 ad =
            add_l ? *reinterpret_cast<const float4*>(add_l + d * add_ld + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float adv[4] = {ad.x, ad.y, ad.z, ad.w};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool nn = v[e] >= 0.f;
          o[e] = v[e] * (nn ? r[e].z : r[e].x);
          s[1] += v[e] * (nn ? r[e].w : r[e].y);
          if (add_l) o[e] = o[e] + adv[e];
          if (kbias) s[3] += o[e] * kbv[e];
          if (cvec) s[5] += o[e] * cvv[e];
        }
        if (Al_out) *reinterpret_cast<float4*>(Al_out + m * K + k) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  // the sums this call needs (conditions uniform over the launch)
  const bool need[6] = {Au != nullptr, Al != nullptr, Au && kbias, Al && kbias, Au && cvec, Al && cvec};
#pragma unroll
  for (int q = 0; q < 6; ++q)
    if (need[q]) s[q] = wave_sum(s[q]);
  if (WPR > 1) {
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0)
#pragma unroll
      for (int q = 0; q < 6; ++q) red[q][w] = s[q];
    __syncthreads();
    if (t == 0)
#pragma unroll
      for (int q = 0; q < 6; ++q) {
        float v = red[q][w];
        for (int i = 1; i < WPR; ++i) v += red[q][w + i];
        s[q] = v;
      }
  }
  if (live && t == 0) {
    if (bu_out) bu_out[m] = ((bu_in ? bu_in[m] : 0.f) + s[0]) + s[2];
    if (bl_out) bl_out[m] = ((bl_in ? bl_in[m] : 0.f) + s[1]) + s[3];
    if (cu_out) cu_out[m] = s[4];
    if (cl_out) cl_out[m] = s[5];
  }
}

// The same pass over a coefficient shared by every domain (a_dstride 0: the first region
// of a C = I query, rows of K <= 256 NQ), or over a per-domain one of many rows: a
// workgroup takes rows_per_wg rows of one domain, and each lane keeps that domain's
// operands of its NQ quads of k (k = 4 lane + 256 q: the relaxation entries, split term,
// center and bias) in registers across all of them, so a row costs one read of its
// coefficient row (for a shared one, L2-resident) and the writes of its relaxed rows.  Per-lane partials in k order and the wave sum: the sums of
// relu_relax_rows4_kernel<64>, bit for bit.
template <int NQ>
__global__ void __launch_bounds__(256)
relu_relax_shared_kernel(const float* __restrict__ Au, const float* __restrict__ Al, int64_t a_dstride, int64_t S,
                         int64_t K, int64_t chunks, int rows_per_wg, RelaxSrc relax, const float* __restrict__ add_l,
                         int64_t add_ld, const float* __restrict__ kbias, const float* __restrict__ cvec,
                         const float* __restrict__ bu_in, const float* __restrict__ bl_in,
                         float* __restrict__ Au_out, float* __restrict__ Al_out, float* __restrict__ bu_out,
                         float* __restrict__ bl_out, float* __restrict__ cu_out, float* __restrict__ cl_out) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t d = (int64_t)blockIdx.x / chunks;
  const int64_t s0 = ((int64_t)blockIdx.x - d * chunks) * rows_per_wg;
  const int64_t s_end = s0 + rows_per_wg < S ? s0 + rows_per_wg : S;
  float4 e[NQ][4];
  float kbv[NQ][4], cvv[NQ][4], adv[NQ][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int64_t k = 4 * ((int64_t)lane + 64 * q);
    const bool ok = k < K;
    if (ok) {
      relax.quad(d, K, k, e[q]);
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) e[q][u] = make_float4(1.f, 0.f, 1.f, 0.f);
    }
    const float4 kb = (ok && kbias) ? *reinterpret_cast<const float4*>(kbias + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 cv = (ok && cvec) ? *reinterpret_cast<const float4*>(cvec + d * K + k)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 ad = (ok && add_l) ? *reinterpret_cast<const float4*>(add_l + d * add_ld + k)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
    kbv[q][0] = kb.x; kbv[q][1] = kb.y; kbv[q][2] = kb.z; kbv[q][3] = kb.w;
    cvv[q][0] = cv.x; cvv[q][1] = cv.y; cvv[q][2] = cv.z; cvv[q][3] = cv.w;
    adv[q][0] = ad.x; adv[q][1] = ad.y; adv[q][2] = ad.z; adv[q][3] = ad.w;
  }
  const bool need[6] = {Au != nullptr, Al != nullptr, Au && kbias, Al && kbias, Au && cvec, Al && cvec};
  for (int64_t srow = s0 + wave; srow < s_end; srow += 4) {
    const int64_t m = d * S + srow;
    const float* __restrict__ au = Au + d * a_dstride + srow * K;
    const float* __restrict__ al = Al + d * a_dstride + srow * K;
    float4 vu4[NQ], vl4[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int64_t k = 4 * ((int64_t)lane + 64 * q);
      const bool ok = k < K;
      vu4[q] = (ok && Au) ? *reinterpret_cast<const float4*>(au + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      vl4[q] = (ok && Al && Al != Au) ? *reinterpret_cast<const float4*>(al + k) : vu4[q];
    }
    float s[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};   // su, sl, ku, kl, cu, cl
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int64_t k = 4 * ((int64_t)lane + 64 * q);
      if (k >= K) continue;
      if (Au) {
        const float v[4] = {vu4[q].x, vu4[q].y, vu4[q].z, vu4[q].w};
        float o[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const bool nn = v[u] >= 0.f;
          o[u] = v[u] * (nn ? e[q][u].x : e[q][u].z);
          s[0] += v[u] * (nn ? e[q][u].y : e[q][u].w);
          if (kbias) s[2] += o[u] * kbv[q][u];
          if (cvec) s[4] += o[u] * cvv[q][u];
        }
        if (Au_out) *reinterpret_cast<float4*>(Au_out + m * K + k) = make_float4(o[0], o[1], o[2], o[3]);
      }
      if (Al) {
        const float v[4] = {vl4[q].x, vl4[q].y, vl4[q].z, vl4[q].w};
        float o[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const bool nn = v[u] >= 0.f;
          o[u] = v[u] * (nn ? e[q][u].z : e[q][u].x);
          s[1] += v[u] * (nn ? e[q][u].w : e[q][u].y);
          if (add_l) o[u] = o[u] + adv[q][u];
          if (kbias) s[3] += o[u] * kbv[q][u];
          if (cvec) s[5] += o[u] * cvv[q][u];
        }
        if (Al_out) *reinterpret_cast<float4*>(Al_out + m * K + k) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
#pragma unroll
    for (int q = 0; q < 6; ++q)
      if (need[q]) s[q] = wave_sum(s[q]);
    if (lane == 0) {   // wave_sum returns the total to every lane
      if (bu_out) bu_out[m] = ((bu_in ? bu_in[m] : 0.f) + s[0]) + s[2];
      if (bl_out) bl_out[m] = ((bl_in ? bl_in[m] : 0.f) + s[1]) + s[3];
      if (cu_out) cu_out[m] = s[4];
      if (cl_out) cl_out[m] = s[5];
    }
  }
}

// ---------------------------------------------------------------------------
// Dense concretization (north-star kernel #4): one wave64 per row
//   center = sum_i A[m,i] * c[d,i];  norm = sum_i |A[m,i]| (* rad[d,i])  (norm_p 0: Linf ball, box),
//   max_i |A[m,i]| (1: L1 ball), sqrt(sum_i A[m,i]^2) (2: L2 ball);
//   lb = (center - eps*norm) + b ; box: eps = 1 with radius weights.
__global__ void __launch_bounds__(256)
concretize_rows_kernel(const float* __restrict__ A, int64_t M, int64_t S, int64_t I, const float* __restrict__ cen,
                       const float* __restrict__ rad, float eps, int norm_p, const float* __restrict__ b,
                       int is_lower, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (m >= M) return;
  const int64_t d = m / S;
  float c = 0.f, nrm = 0.f;
  const float* __restrict__ row = A + m * I;
  const float* __restrict__ cr = cen + d * I;
  if ((I & 3) == 0) {
    const float4* row4 = reinterpret_cast<const float4*>(row);
    const float4* c4 = reinterpret_cast<const float4*>(cr);
    const float4* r4 = rad ? reinterpret_cast<const float4*>(rad + d * I) : nullptr;
    for (int64_t q = lane; q < I / 4; q += 64) {
      float4 a = row4[q], x = c4[q];
      c += a.x * x.x + a.y * x.y + a.z * x.z + a.w * x.w;
      if (r4) {
        float4 w = r4[q];
        nrm += fabsf(a.x) * w.x + fabsf(a.y) * w.y + fabsf(a.z) * w.z + fabsf(a.w) * w.w;
      } else if (norm_p == 1) {
        nrm = fmaxf(nrm, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
      } else if (norm_p == 2) {
        nrm += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
      } else {
        nrm += fabsf(a.x) + fabsf(a.y) + fabsf(a.z) + fabsf(a.w);
      }
    }
  } else {
    for (int64_t i = lane; i < I; i += 64) {
      float a = row[i];
      c += a * cr[i];
      if (rad) nrm += fabsf(a) * rad[d * I + i];
      else if (norm_p == 1) nrm = fmaxf(nrm, fabsf(a));
      else if (norm_p == 2) nrm += a * a;
      else nrm += fabsf(a);
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    c += __shfl_xor(c, off, 64);
    const float o = __shfl_xor(nrm, off, 64);
    nrm = norm_p == 1 ? fmaxf(nrm, o) : nrm + o;
  }
  if (lane == 0) {
    float dev = eps * (norm_p == 2 ? sqrtf(nrm) : nrm);
    float v = is_lower ? c - dev : c + dev;
    out[m] = b ? v + b[m] : v;
  }
}

// ---------------------------------------------------------------------------
// Branching heuristic update for one ReLU layer (alpha_beta_crown.py:145-182):
// per domain, widest ambiguous neuron (first index on ties); replaces the
// running best only when strictly wider (earlier layers win ties).
__global__ void branch_update_kernel(const float* __restrict__ lo, const float* __restrict__ hi, int64_t D,
                                     int64_t N, int layer, float* __restrict__ best_gap, int* __restrict__ best_layer,
                                     int* __restrict__ best_idx) {
  const int lane = threadIdx.x & 63;
  const int64_t d = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (d >= D) return;
  float g = -INFINITY;
  int idx = 0;
  bool any = false;
  for (int64_t n = lane; n < N; n += 64) {
    float l = lo[d * N + n], u = hi[d * N + n];
    bool amb = (l < 0.f) && (u > 0.f);
    if (amb) {
      any = true;
      float gap = fmaxf(u - l, 0.f);
      if (gap > g) {
        g = gap;
        idx = (int)n;
      }
    }
  }
  // reduce (max gap, then min index)
  for (int off = 32; off >= 1; off >>= 1) {
    float og = __shfl_xor(g, off, 64);
    int oi = __shfl_xor(idx, off, 64);
    int oa = __shfl_xor((int)any, off, 64);
    if (oa) {
      if (!any || og > g || (og == g && oi < idx)) {
        g = og;
        idx = oi;
      }
      any = true;
    }
  }
  if (lane == 0 && any) {
    if (g > best_gap[d]) {
      best_gap[d] = g;
      best_layer[d] = layer;
      best_idx[d] = idx;
    }
  }
}

// ---------------------------------------------------------------------------
// torch.optim.Adam step (defaults: no weight decay, no amsgrad) followed by
// clamp_(lo, hi), applied in place.  Matches the single-tensor update order:
//   m = lerp(m, g, 1 - b1); v = v * b2 + (1 - b2) * g * g;
//   p -= (lr / (1 - b1^t)) * m / (sqrt(v) / sqrt(1 - b2^t) + eps)
__device__ __forceinline__ void adam_clamp_one(float* __restrict__ p, float* __restrict__ m, float* __restrict__ v,
                                               const float* __restrict__ g, int64_t i, float w1, float b2, float w2,
                                               float eps, float neg_step, float bc2_sqrt, float lo, float hi,
                                               int clamp_hi, bool fresh) {
  // fresh (step 1): torch.optim.Adam's state starts at zero, so the moments are not read
  const float gi = g[i];
  float mi = fresh ? 0.f : m[i];
  // exp_avg.lerp_(grad, 1 - beta1): torch's vectorized CPU lerp is fma(w, g - m, m) for w < 0.5
  mi = (w1 < 0.5f) ? fmaf(w1, gi - mi, mi) : fmaf(w1 - 1.0f, gi - mi, gi);
  float vi = (fresh ? 0.f : v[i]) * b2;                                       // exp_avg_sq.mul_(beta2)
  vi = vi + w2 * gi * gi;                                                     //   .addcmul_(g, g, 1 - beta2)
  m[i] = mi;
  v[i] = vi;
  const float denom = sqrtf(vi) / bc2_sqrt + eps;                             // (sqrt(v) / bc2_sqrt).add_(eps)
  float pi = p[i] + neg_step * mi / denom;                                    // addcdiv_(m, denom, -step_size)
  pi = fmaxf(pi, lo);
  if (clamp_hi) pi = fminf(pi, hi);
  p[i] = pi;
}

__global__ void adam_clamp_kernel(float* __restrict__ p, float* __restrict__ m, float* __restrict__ v,
                                  const float* __restrict__ g, int64_t n, float w1, float b2, float w2, float eps,
                                  float neg_step, float bc2_sqrt, float lo, float hi, int clamp_hi, int fresh) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  adam_clamp_one(p, m, v, g, i, w1, b2, w2, eps, neg_step, bc2_sqrt, lo, hi, clamp_hi, fresh != 0);
}

// Several tensors in one launch.  Workgroups are dealt to the tensors in order
// (tensor s owns blocks bstart[s] .. bstart[s + 1] - 1), so a workgroup's tensor
// is uniform and its pointers are scalar loads.
constexpr int BF_SEG_MAX = 16;

struct AdamSegs {
  float* p[BF_SEG_MAX];
  float* m[BF_SEG_MAX];
  float* v[BF_SEG_MAX];
  const float* g[BF_SEG_MAX];
  float* best[BF_SEG_MAX];   // best-of copy before the step (null: none)
  int64_t ncol[BF_SEG_MAX];  // row length of the copy's mask rows
  int64_t n[BF_SEG_MAX];
  float lo[BF_SEG_MAX], hi[BF_SEG_MAX];
  int clamp_hi[BF_SEG_MAX];
  int64_t bstart[BF_SEG_MAX + 1];
  int count;
};

__device__ __forceinline__ int seg_of_block(const int64_t* bstart, int count) {
  int s = 0;
  while (s + 1 < count && (int64_t)blockIdx.x >= bstart[s + 1]) ++s;
  return s;
}

// improved (with best): row i / ncol of every tensor improved at the evaluation the step
// follows, so the parameter is first copied to its best-of tensor (the copy of
// masked_copy_rows_multi_kernel, taken from the same values before they are stepped).
__global__ void adam_clamp_multi_kernel(AdamSegs a, float w1, float b2, float w2, float eps, float neg_step,
                                        float bc2_sqrt, const int* __restrict__ improved, int fresh) {
  const int s = seg_of_block(a.bstart, a.count);
  const int64_t i = ((int64_t)blockIdx.x - a.bstart[s]) * 256 + threadIdx.x;
  if (i >= a.n[s]) return;
  if (a.best[s] && improved[div_rows(i, a.ncol[s], a.n[s] < (1LL << 31))]) a.best[s][i] = a.p[s][i];
  adam_clamp_one(a.p[s], a.m[s], a.v[s], a.g[s], i, w1, b2, w2, eps, neg_step, bc2_sqrt, a.lo[s], a.hi[s],
                 a.clamp_hi[s], fresh != 0);
}

// dst[s][d, j] = src[s][d, j] where mask[d] (the best-of copy of several parameters)
struct CopySegs {
  float* dst[BF_SEG_MAX];
  const float* src[BF_SEG_MAX];
  int64_t ncol[BF_SEG_MAX];
  int64_t bstart[BF_SEG_MAX + 1];
  int count;
};

// QUAD: every segment's row length is a multiple of 4 and its rows 16-byte aligned, and a
// thread moves one float4; the row index is a 32-bit division when the segment fits.
template <bool QUAD>
__global__ void masked_copy_rows_multi_kernel(CopySegs c, int64_t D, const int* __restrict__ mask) {
  const int s = seg_of_block(c.bstart, c.count);
  const int64_t i = ((int64_t)blockIdx.x - c.bstart[s]) * 256 + threadIdx.x;
  const int64_t N = QUAD ? c.ncol[s] / 4 : c.ncol[s];
  const int64_t total = D * N;
  if (i >= total) return;
  if (!mask[div_rows(i, N, total < (1LL << 31))]) return;
  if constexpr (QUAD)
    reinterpret_cast<float4*>(c.dst[s])[i] = reinterpret_cast<const float4*>(c.src[s])[i];
  else
    c.dst[s][i] = c.src[s][i];
}

// out[s][d, j] = -beta[s][d, j] * split[s][d, j] * 1(split != 0) for several ReLUs
struct BetaSegs {
  const float* beta[BF_SEG_MAX];
  int64_t beta_ld[BF_SEG_MAX];
  const int8_t* split[BF_SEG_MAX];
  int64_t split_ld[BF_SEG_MAX];
  int64_t ncol[BF_SEG_MAX];
  float* out[BF_SEG_MAX];
  int64_t bstart[BF_SEG_MAX + 1];
  int count;
};

__device__ __forceinline__ float beta_term(float beta, int8_t sp) {
  return (-beta * (float)sp) * (sp != 0 ? 1.f : 0.f);
}

// QUAD: every segment's row length and strides are multiples of 4 with aligned rows, and a
// thread writes four consecutive entries of one row (a float4 of beta, four split bytes).
template <bool QUAD>
__global__ void beta_coeff_multi_kernel(BetaSegs b, int64_t D) {
  const int s = seg_of_block(b.bstart, b.count);
  const int64_t i = ((int64_t)blockIdx.x - b.bstart[s]) * 256 + threadIdx.x;
  const int64_t N = QUAD ? b.ncol[s] / 4 : b.ncol[s];
  if (i >= D * N) return;
  const int64_t d = div_rows(i, N, D * N < (1LL << 31)), q = i - d * N;
  if constexpr (QUAD) {
    const int64_t n = 4 * q;
    const float4 bv = *reinterpret_cast<const float4*>(b.beta[s] + d * b.beta_ld[s] + n);
    const char4 sv = *reinterpret_cast<const char4*>(b.split[s] + d * b.split_ld[s] + n);
    *reinterpret_cast<float4*>(b.out[s] + 4 * i) =
        make_float4(beta_term(bv.x, sv.x), beta_term(bv.y, sv.y), beta_term(bv.z, sv.z), beta_term(bv.w, sv.w));
  } else {
    b.out[s][i] = beta_term(b.beta[s][d * b.beta_ld[s] + q], b.split[s][d * b.split_ld[s] + q]);
  }
}

// ---------------------------------------------------------------------------
// The two-region step of bf_crown_relu_linear_relu_fwd when the contraction is
// short (N <= SMALLK_MAX: the first region C x W of the output layer) and A needs
// no prologue relaxation.  The tiled contraction would run one wave of workgroups
// whose fixed latencies never overlap; here a wave takes the S rows of one domain
// over 256 output columns (4 per lane), keeps the weight columns and the next
// ReLU's relaxation entries of its columns in registers, reads each coefficient
// row with scalar loads, and stores A_next (and A_pre) as 16-byte vectors.  The
// four waves of a workgroup take four domains of one column chunk and stage that
// chunk's weights in LDS once, with coalesced loads.  Row
// sums per 256-column chunk go to the workspace, summed in chunk order by
// rows_finalize like the tiled path's per-tile partials.
constexpr int SMALLK_MAX = 16;
constexpr int SMALLK_ROWS = 256;

__global__ void __launch_bounds__(256)
small_k_relax_epi_kernel(const float* __restrict__ A0, const float* __restrict__ A1, int64_t a_dstride, int64_t D,
                         int64_t S, int N, const float* __restrict__ Wt, int64_t P, const float* __restrict__ bias,
                         const float* __restrict__ b_in0, const float* __restrict__ b_in1,
                         const float4* __restrict__ relax_next, const float* __restrict__ add_next,
                         int64_t add_next_ld, const float* __restrict__ bias_next, const float* __restrict__ cvec_next,
                         int64_t cvec_next_ld, float* __restrict__ An0, float* __restrict__ An1,
                         float* __restrict__ Ap0, float* __restrict__ Ap1, float* __restrict__ bo0,
                         float* __restrict__ bo1, float* __restrict__ pb0, float* __restrict__ pb1,
                         float* __restrict__ pc0, float* __restrict__ pc1, int z_lower_first, int nchunks) {
  const int z = blockIdx.y;
  const bool lower = z_lower_first ? (z == 0) : (z == 1);
  const float* __restrict__ A = z == 0 ? A0 : A1;
  const float* __restrict__ b_in = z == 0 ? b_in0 : b_in1;
  float* __restrict__ An = z == 0 ? An0 : An1;
  float* __restrict__ Ap = z == 0 ? Ap0 : Ap1;
  float* __restrict__ bo = z == 0 ? bo0 : bo1;
  float* __restrict__ pb = z == 0 ? pb0 : pb1;
  float* __restrict__ pc = z == 0 ? pc0 : pc1;
  __shared__ float Ws[256 * SMALLK_MAX];   // the chunk's weight rows [256 columns][N]
  __shared__ float Asm[4][SMALLK_ROWS];    // each wave's domain block of A [S][N] when S N <= SMALLK_ROWS
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int chunk = (int)(blockIdx.x % nchunks);
  const int64_t d = (int64_t)(blockIdx.x / nchunks) * 4 + wave;
  const int64_t cols = P - (int64_t)chunk * 256 < 256 ? P - (int64_t)chunk * 256 : 256;
  for (int64_t i = threadIdx.x; i < cols * N; i += 256) Ws[i] = Wt[(int64_t)chunk * 256 * N + i];
  const bool a_lds = S * N <= SMALLK_ROWS;   // uniform
  if (a_lds && d < D)
    for (int64_t i = lane; i < S * N; i += 64) Asm[wave][i] = A[d * a_dstride + i];
  __syncthreads();
  if (d >= D) return;   // whole wave
  const int64_t M = D * S;
  const int64_t p0 = (int64_t)chunk * 256 + 4 * lane;
  const bool act = p0 < P;   // P % 4 == 0: the whole quad is inside
  float wv[4][SMALLK_MAX];
  float4 e[4];
  float ad[4] = {0.f, 0.f, 0.f, 0.f}, kb[4] = {0.f, 0.f, 0.f, 0.f}, cv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int n = 0; n < SMALLK_MAX; ++n) wv[q][n] = (act && n < N) ? Ws[(4 * lane + q) * N + n] : 0.f;
    e[q] = act ? relax_next[d * P + p0 + q] : make_float4(1.f, 0.f, 1.f, 0.f);
    if (act && lower && add_next) ad[q] = add_next[d * add_next_ld + p0 + q];
    if (act && bias_next) kb[q] = bias_next[p0 + q];
    if (act && cvec_next) cv[q] = cvec_next[d * cvec_next_ld + p0 + q];
  }
  float bv[SMALLK_MAX];
#pragma unroll
  for (int n = 0; n < SMALLK_MAX; ++n) bv[n] = (bo && n < N) ? bias[n] : 0.f;
  for (int64_t s_ = 0; s_ < S; ++s_) {
    const int64_t m = d * S + s_;
    // the row from LDS (a broadcast read) or, for a large domain block, from global memory
    float a[SMALLK_MAX];
    if (a_lds) {
      const float* ar = &Asm[wave][s_ * N];
#pragma unroll
      for (int n = 0; n < SMALLK_MAX; ++n) a[n] = n < N ? ar[n] : 0.f;
    } else {
      const float* __restrict__ ar = A + d * a_dstride + s_ * N;
#pragma unroll
      for (int n = 0; n < SMALLK_MAX; ++n) a[n] = n < N ? ar[n] : 0.f;
    }
    float acc[4], out[4];
    float sb = 0.f, sc = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float v = 0.f;
#pragma unroll
      for (int n = 0; n < SMALLK_MAX; ++n) v += a[n] * wv[q][n];
      acc[q] = v;
      // upper: C >= 0 -> (alpha_u, beta_u) else (alpha_l, beta_l); lower mirrored
      const bool use_u = lower ? !(v >= 0.f) : (v >= 0.f);
      float o = v * (use_u ? e[q].x : e[q].z);
      const float be = use_u ? e[q].y : e[q].w;
      if (lower && add_next) o = o + ad[q];
      sb += v * be;
      if (bias_next) sb += o * kb[q];
      if (cvec_next) sc += o * cv[q];
      out[q] = o;
    }
    if (act) {
      if (Ap) *reinterpret_cast<float4*>(Ap + m * P + p0) = make_float4(acc[0], acc[1], acc[2], acc[3]);
      *reinterpret_cast<float4*>(An + m * P + p0) = make_float4(out[0], out[1], out[2], out[3]);
    }
    // fixed-order DPP wave sums (VALU only, no LDS round trips)
    sb = wave_sum(sb);
    if (cvec_next) sc = wave_sum(sc);
    if (lane == 0) {
      pb[(int64_t)chunk * M + m] = sb;
      if (cvec_next) pc[(int64_t)chunk * M + m] = sc;
      if (bo && chunk == 0) {
        // the affine bias of this region: b += A . bias
        float sk = 0.f;
#pragma unroll
        for (int n = 0; n < SMALLK_MAX; ++n)
          if (n < N) sk += a[n] * bv[n];
        bo[m] = ((b_in ? b_in[m] : 0.f) + 0.f) + sk;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The same concretization without a caller workspace, for callers that cannot
// allocate (graph capture, serving loops that forbid it).  Its workspace -- the
// per-column-tile partial norms, the center and bias sums -- lives in a
// file-scope device array of kConcretizeScratchFloats floats (16 MiB), one copy
// per GPU for the life of the process.  The kernels write every element they
// later read (each column tile its partial norm of every row, the first column
// tile the center and bias sums), so nothing is cleared between calls.  Calls
// that overlap on one GPU share the array and race: serialise them (one stream,
// or events) as for any buffer they would share.

constexpr int64_t kConcretizeScratchFloats = (int64_t)4 << 20;
static __device__ __align__(256) float scratch[kConcretizeScratchFloats];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_dev[kMaxDevices] = {};   // device address of `scratch` on each GPU

// Address of the current device's copy of `scratch`, looked up once per device
// (the host symbol itself is not a device address).
static int concretize_scratch(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("bf_crown_relu_linear_concretize_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return BF_ELAUNCH;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("bf_crown_relu_linear_concretize_noalloc: device %d beyond %d", dev, kMaxDevices);
    return BF_ERANGE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("bf_crown_relu_linear_concretize_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return BF_ELAUNCH;
    }
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_dev[dev];
  return BF_OK;
}

}  // namespace bf

using namespace bf;

extern "C" {

int bf_abi_version(void) { return 1; }

const char* bf_last_error(void) { return g_err; }

int bf_gemm_tile_config(int64_t M, int64_t N, int nz, int ksplit, int relax_prologue, int dl_operands) {
  if (M <= 0 || N <= 0 || nz < 1 || nz > 2 || ksplit < 1) return 0;
  return gemm_tile_choice(M, N, nz, ksplit, relax_prologue ? PRO_RELAX : PRO_PLAIN, dl_operands != 0);
}

int bf_gemm(const float* A, int64_t lda, const float* B, int64_t ldb, int trans_b, int abs_b, float* C, int64_t ldc,
            int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  BF_REQUIRE(M >= 0 && N >= 0 && K >= 0, "bf_gemm: negative size");
  if (M == 0 || N == 0) return BF_OK;
  BF_REQUIRE(A && B && C, "bf_gemm: null pointer");
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A[0] = A;
  a.C[0] = C;
  a.lda = lda;
  a.lda_d = lda;
  a.ldc = ldc;
  a.B = B;
  a.ldb = ldb;
  a.trans_b = trans_b;
  a.abs_b = abs_b ? 1 : 0;
  a.M = M;
  a.N = N;
  a.K = K;
  a.S = 1;
  return gemm_dispatch(a, PRO_PLAIN, EPI_STORE, 1, stream);
}

int64_t bf_gemm_rank1_workspace(int64_t M, int64_t N, int64_t K) {
  int64_t kchunk;
  const int ks = gemm_ksplit(M, N, K, &kchunk);
  return ks > 1 ? (int64_t)ks * M * N : 0;
}

int bf_gemm_rank1(const float* A, int64_t lda, const float* B, int64_t ldb, int trans_b, float* C, int64_t ldc,
                  int64_t M, int64_t N, int64_t K, int64_t S, const float* r_row, const float* v_col, int64_t v_ld,
                  float* workspace, int64_t workspace_floats, hipStream_t stream) {
  BF_REQUIRE(M >= 0 && N >= 0 && K >= 0 && S > 0, "bf_gemm_rank1: bad sizes");
  if (M == 0 || N == 0) return BF_OK;
  BF_REQUIRE(A && B && C && ((r_row == nullptr) == (v_col == nullptr)), "bf_gemm_rank1: null pointer");
  int64_t kchunk = K;
  int ks = gemm_ksplit(M, N, K, &kchunk);
  if (ks > 1 && trans_b && small_out_route(M, N)) {
    // a small output whose contraction would be split: the whole reduction per 16 x 16 tile
    // in one launch, the rank-1 term in its epilogue
    SmallOutArgs s;
    memset(&s, 0, sizeof(s));
    s.lo = A;
    s.lda = lda;
    s.W = B;
    s.ldw = ldb;
    s.B = M;
    s.K = K;
    s.N = N;
    s.C = C;
    s.ldc = ldc;
    s.r_row = r_row;
    s.v_col = v_col;
    s.v_ld = v_ld;
    s.S = S;
    return small_out_launch(SM_GEMM, s, stream);
  }
  if (ks > 1 && (workspace == nullptr || workspace_floats < (int64_t)ks * M * N)) ks = 1;   // no split without room
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A[0] = A;
  a.C[0] = C;
  a.lda = lda;
  a.lda_d = lda * S;
  a.ldc = ldc;
  a.B = B;
  a.ldb = ldb;
  a.trans_b = trans_b;
  a.M = M;
  a.N = N;
  a.K = K;
  a.S = S;
  a.r1_row = r_row;
  a.r1_col = v_col;
  a.r1_ld = v_ld;
  if (ks == 1) return gemm_dispatch(a, PRO_PLAIN, EPI_STORE, 1, stream);
  a.ksplit = ks;
  a.kchunk = kchunk;
  a.part = workspace;
  const int rc = gemm_dispatch(a, PRO_PLAIN, EPI_STORE, 1, stream);
  if (rc) return rc;
  return splitk_reduce(workspace, ks, M, N, C, ldc, r_row, v_col, v_ld, S, stream);
}

int bf_concretize_finalize(const float* partial_u, const float* partial_l, int nparts, int64_t M,
                           const float* cen_u, const float* cen_l, const float* b_u, const float* b_l, float eps,
                           int norm_p, float* lb, float* ub, hipStream_t stream) {
  BF_REQUIRE(M >= 0 && nparts >= 1, "bf_concretize_finalize: bad sizes");
  BF_REQUIRE((lb == nullptr || (partial_l && cen_l && b_l)) && (ub == nullptr || (partial_u && cen_u && b_u)),
             "bf_concretize_finalize: null pointer");
  return concretize_finalize(partial_u, partial_l, nparts, M, cen_u, cen_l, b_u, b_l, eps, norm_p, lb, ub, stream);
}

int bf_relu_relax_table_from_planes(const float* alpha_u, const float* beta_u, const float* alpha_l,
                                    const float* beta_l, int64_t n, float* table, hipStream_t stream) {
  BF_REQUIRE(n >= 0, "bf_relu_relax_table_from_planes: bad size");
  if (n == 0) return BF_OK;
  BF_REQUIRE(alpha_u && beta_u && alpha_l && beta_l && table, "bf_relu_relax_table_from_planes: null pointer");
  BF_REQUIRE(((uintptr_t)table & 15) == 0, "bf_relu_relax_table_from_planes: table must be 16-byte aligned");
  const int64_t blocks = (n + 255) / 256;
  BF_REQUIRE(blocks < (1LL << 31), "bf_relu_relax_table_from_planes: too many entries");
  hipLaunchKernelGGL(planes_table_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, alpha_u, beta_u, alpha_l,
                     beta_l, n, reinterpret_cast<float4*>(table));
  BF_LAUNCH_CHECK("planes_table_kernel");
  return BF_OK;
}

int bf_relu_relax_table(const float* pre_lo, const float* pre_hi, const float* alpha, int64_t alpha_ld, int64_t D,
                        int64_t K, float* table, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && K >= 0, "bf_relu_relax_table: bad sizes");
  if (D * K == 0) return BF_OK;
  BF_REQUIRE(pre_lo && pre_hi && table, "bf_relu_relax_table: null pointer");
  BF_REQUIRE(((uintptr_t)table & 15) == 0, "bf_relu_relax_table: table must be 16-byte aligned");
  return relax_table(pre_lo, pre_hi, alpha, alpha_ld, D, K, reinterpret_cast<float4*>(table), stream);
}

int bf_relu_relax_table_multi(int count, const float* const* pre_lo, const float* const* pre_hi,
                              const float* const* alpha, const int64_t* alpha_ld, int64_t D, const int64_t* K,
                              float* const* table, hipStream_t stream) {
  BF_REQUIRE(count >= 0 && D >= 0, "bf_relu_relax_table_multi: bad sizes");
  if (count == 0 || D == 0) return BF_OK;
  BF_REQUIRE(pre_lo && pre_hi && alpha && alpha_ld && K && table, "bf_relu_relax_table_multi: null array");
  for (int j = 0; j < count; ++j) {
    BF_REQUIRE(K[j] >= 0, "bf_relu_relax_table_multi: bad size of table %d", j);
    if (K[j] == 0) continue;
    BF_REQUIRE(pre_lo[j] && pre_hi[j] && table[j], "bf_relu_relax_table_multi: null pointer in table %d", j);
    BF_REQUIRE(((uintptr_t)table[j] & 15) == 0, "bf_relu_relax_table_multi: table %d must be 16-byte aligned", j);
  }
  return relax_table_multi(count, pre_lo, pre_hi, alpha, alpha_ld, D, K, table, stream);
}

static int relax_pass(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t K,
                      const RelaxSrc& src, const float* add_l, int64_t add_ld, const float* kbias, const float* cvec,
                      const float* b_u_in, const float* b_l_in, float* A_u_out, float* A_l_out, float* b_u_out,
                      float* b_l_out, float* c_u_out, float* c_l_out, hipStream_t stream, bool sums_only);

int bf_crown_relu_linear_fwd(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t N,
                             const float* relax, const float* add_l, int64_t add_ld, const float* W, int64_t P,
                             int w_trans, const float* bias, const float* b_u_in, const float* b_l_in,
                             float* A_prev_u, float* A_prev_l, float* b_u_out, float* b_l_out, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S >= 0 && N > 0 && P > 0, "bf_crown_relu_linear_fwd: bad sizes");
  const int64_t M = D * S;
  if (M == 0) return BF_OK;
  BF_REQUIRE(W != nullptr, "bf_crown_relu_linear_fwd: null weight");
  BF_REQUIRE(((uintptr_t)relax & 15) == 0, "bf_crown_relu_linear_fwd: relax table must be 16-byte aligned");
  BF_REQUIRE((A_u != nullptr) == (A_prev_u != nullptr) && (A_l != nullptr) == (A_prev_l != nullptr),
             "bf_crown_relu_linear_fwd: input/output pointer mismatch");
  BF_REQUIRE(A_u || A_l, "bf_crown_relu_linear_fwd: no coefficient");
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  int nz = 0;
  // z order: upper first when present
  if (A_u) {
    a.A[nz] = A_u; a.C[nz] = A_prev_u; a.b_in[nz] = b_u_in; a.b_out[nz] = b_u_out; ++nz;
  }
  if (A_l) {
    a.A[nz] = A_l; a.C[nz] = A_prev_l; a.b_in[nz] = b_l_in; a.b_out[nz] = b_l_out; ++nz;
  }
  a.z_lower_first = (A_u == nullptr) ? 1 : 0;
  a.lda = N;
  a.lda_d = a_dstride;
  a.ldc = P;
  a.B = W;
  a.trans_b = w_trans ? 1 : 0;
  a.ldb = w_trans ? N : P;
  a.M = M;
  a.N = P;
  a.K = N;
  a.S = S;
  a.relax = reinterpret_cast<const float4*>(relax);
  a.add_l = add_l;
  a.add_ld = add_ld;
  a.kbias = bias;
  // Bias rows alone (nothing to relax) on a grid of fewer 128 x 128 tiles than the device
  // has CUs: the row sums in a pass of their own (A read once, no coefficient written),
  // then the plain contraction, whose 64 x 64 tiles spread the short grid over four times
  // as many CUs as the relaxation prologue's tiles (a K loop of a few tiles keeps the
  // one-launch form).
  if (!relax && !add_l && bias && N >= 32 && ceil_div(M, 128) * ceil_div(P, 128) * nz < 256) {
    if (b_u_out || b_l_out) {
      const RelaxSrc none{nullptr, nullptr, nullptr, nullptr, 0};
      const int rc = relax_pass(A_u, A_l, a_dstride, D, S, N, none, nullptr, 0, bias, nullptr, b_u_in, b_l_in, nullptr,
                                nullptr, b_u_out, b_l_out, nullptr, nullptr, stream, true);
      if (rc) return rc;
    }
    return gemm_dispatch(a, PRO_PLAIN, EPI_STORE, nz, stream);
  }
  if (relax || add_l || bias) return gemm_dispatch(a, PRO_RELAX, EPI_STORE, nz, stream);
  // nothing to relax (A already relaxed): the plain contraction, b_out = b_in
  const int rc = gemm_dispatch(a, PRO_PLAIN, EPI_STORE, nz, stream);
  for (int z = 0; z < nz && rc == 0; ++z) {
    if (a.b_out[z]) {
      const int r2 = rows_finalize(a.b_in[z], nullptr, nullptr, 0, M, a.b_out[z], nullptr, stream);
      if (r2) return r2;
    }
  }
  return rc;
}

int bf_crown_relu_linear_concretize(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t N,
                                    const float* relax, const float* add_l, int64_t add_ld, const float* W, int64_t I,
                                    int w_trans, const float* bias, const float* cvec, const float* rad, float eps,
                                    int norm_p, const float* b_u_in, const float* b_l_in, const float* h_scale,
                                    float* h_out, float* workspace, float* lb, float* ub, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S >= 0 && N > 0 && I > 0, "bf_crown_relu_linear_concretize: bad sizes");
  BF_REQUIRE(norm_p >= 0 && norm_p <= 2 && (norm_p == 0 || rad == nullptr),
             "bf_crown_relu_linear_concretize: norm_p %d (0 Linf/box, 1 L1, 2 L2; the box radius goes with 0 only)",
             norm_p);
  const int64_t M = D * S;
  if (M == 0) return BF_OK;
  BF_REQUIRE(W && cvec && workspace, "bf_crown_relu_linear_concretize: null pointer");
  BF_REQUIRE(((uintptr_t)relax & 15) == 0, "bf_crown_relu_linear_concretize: relax table must be 16-byte aligned");
  BF_REQUIRE((A_u != nullptr) == (ub != nullptr) && (A_l != nullptr) == (lb != nullptr),
             "bf_crown_relu_linear_concretize: input/output pointer mismatch");
  const int nparts = gemm_norm_partial_count(M, I, PRO_RELAX);
  // workspace layout: partial_u [nparts*M], partial_l [nparts*M], cen_u [M], cen_l [M], bout_u [M], bout_l [M]
  float* pu = workspace;
  float* pl = pu + (int64_t)nparts * M;
  float* cu = pl + (int64_t)nparts * M;
  float* cl = cu + M;
  float* bu = cl + M;
  float* bl = bu + M;
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  int nz = 0;
  if (A_u) {
    a.A[nz] = A_u; a.b_in[nz] = b_u_in; a.b_out[nz] = bu; a.c_out[nz] = cu; a.partial[nz] = pu; ++nz;
  }
  if (A_l) {
    a.A[nz] = A_l; a.b_in[nz] = b_l_in; a.b_out[nz] = bl; a.c_out[nz] = cl; a.partial[nz] = pl; ++nz;
  }
  a.z_lower_first = (A_u == nullptr) ? 1 : 0;
  a.lda = N;
  a.lda_d = a_dstride;
  a.B = W;
  a.trans_b = w_trans ? 1 : 0;
  a.ldb = w_trans ? N : I;
  a.M = M;
  a.N = I;
  a.K = N;
  a.S = S;
  a.relax = reinterpret_cast<const float4*>(relax);
  a.add_l = add_l;
  a.add_ld = add_ld;
  a.kbias = bias;
  a.cvec = cvec;
  a.cvec_ld = N;
  a.wvec = rad;
  a.w_ld = I;
  BF_REQUIRE((h_out == nullptr) == (h_scale == nullptr) && (h_out == nullptr || A_l != nullptr),
             "bf_crown_relu_linear_concretize: h_out needs h_scale and the lower coefficient");
  a.h_scale = h_scale;
  a.h_out = h_out;
  a.norm_kind = norm_p;
  int rc = gemm_dispatch(a, PRO_RELAX, EPI_ABSSUM, nz, stream);
  if (rc) return rc;
  if (h_out && norm_p != 0) {
    rc = lp_seed_rows(h_out, M, I, h_scale, norm_p, stream);   // h_out holds the lower coefficient A'W
    if (rc) return rc;
  }
  return concretize_finalize(pu, pl, nparts, M, cu, cl, bu, bl, rad ? 1.0f : eps, norm_p, lb, ub, stream);
}

int64_t bf_crown_relu_linear_concretize_workspace(int64_t D, int64_t S, int64_t I) {
  const int64_t M = D * S;
  return (2 * (int64_t)gemm_norm_partial_count(M, I, PRO_RELAX) + 4) * M;
}

int bf_crown_relu_linear_concretize_noalloc(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D,
                                            int64_t S, int64_t N, const float* relax, const float* add_l,
                                            int64_t add_ld, const float* W, int64_t I, int w_trans, const float* bias,
                                            const float* cvec, const float* rad, float eps, int norm_p,
                                            const float* b_u_in, const float* b_l_in, const float* h_scale,
                                            float* h_out, float* lb, float* ub, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S >= 0 && N > 0 && I > 0, "bf_crown_relu_linear_concretize_noalloc: bad sizes");
  if (D * S == 0) return BF_OK;
  const int64_t need = bf_crown_relu_linear_concretize_workspace(D, S, I);
  if (need > kConcretizeScratchFloats) {
    set_error("bf_crown_relu_linear_concretize_noalloc: %lld rows of %lld columns need %lld workspace floats, the "
              "fixed scratch holds %lld (at most %lld rows at this width); use bf_crown_relu_linear_concretize",
              (long long)(D * S), (long long)I, (long long)need, (long long)kConcretizeScratchFloats,
              (long long)(kConcretizeScratchFloats / (2 * (int64_t)gemm_norm_partial_count(D * S, I, PRO_RELAX) + 4)));
    return BF_ERANGE;
  }
  float* ws = nullptr;
  const int rc = concretize_scratch(&ws);
  if (rc) return rc;
  return bf_crown_relu_linear_concretize(A_u, A_l, a_dstride, D, S, N, relax, add_l, add_ld, W, I, w_trans, bias,
                                         cvec, rad, eps, norm_p, b_u_in, b_l_in, h_scale, h_out, ws, lb, ub, stream);
}

int bf_crown_relu_linear_relu_fwd(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S,
                                  int64_t N, const float* relax, const float* add_l, int64_t add_ld,
                                  const float* W_t, int64_t P, const float* bias, const float* b_u_in,
                                  const float* b_l_in, const float* relax_next, const float* add_next,
                                  int64_t add_next_ld, const float* bias_next, const float* cvec_next,
                                  int64_t cvec_next_ld, float* workspace, float* A_next_u, float* A_next_l,
                                  float* A_pre_u, float* A_pre_l, float* b_u_out, float* b_l_out, float* c_u_out,
                                  float* c_l_out, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0 && N > 0 && P > 0, "bf_crown_relu_linear_relu_fwd: bad sizes");
  const int64_t M = D * S;
  if (M == 0) return BF_OK;
  BF_REQUIRE(W_t && relax_next && workspace, "bf_crown_relu_linear_relu_fwd: null weight, table or workspace");
  BF_REQUIRE(((uintptr_t)relax & 15) == 0 && ((uintptr_t)relax_next & 15) == 0,
             "bf_crown_relu_linear_relu_fwd: relaxation tables must be 16-byte aligned");
  BF_REQUIRE((A_u != nullptr) == (A_next_u != nullptr) && (A_u != nullptr) == (b_u_out != nullptr) &&
                 (A_l != nullptr) == (A_next_l != nullptr) && (A_l != nullptr) == (b_l_out != nullptr),
             "bf_crown_relu_linear_relu_fwd: input/output pointer mismatch");
  BF_REQUIRE(A_u || A_l, "bf_crown_relu_linear_relu_fwd: no coefficient");
  BF_REQUIRE(cvec_next == nullptr || ((A_u == nullptr || c_u_out) && (A_l == nullptr || c_l_out)),
             "bf_crown_relu_linear_relu_fwd: center sums need c_out");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (N <= SMALLK_MAX && relax == nullptr && add_l == nullptr && P % 4 == 0 && al16(A_next_u) && al16(A_next_l) &&
      al16(A_pre_u) && al16(A_pre_l)) {
    const int nchunks = (int)ceil_div(P, 256);
    const int nz = (A_u ? 1 : 0) + (A_l ? 1 : 0);
    const float* As[2] = {A_u ? A_u : A_l, A_l};
    const float* bi[2] = {A_u ? b_u_in : b_l_in, b_l_in};
    float* an[2] = {A_u ? A_next_u : A_next_l, A_next_l};
    float* ap[2] = {A_u ? A_pre_u : A_pre_l, A_pre_l};
    float* bo[2] = {A_u ? b_u_out : b_l_out, b_l_out};
    float* co[2] = {A_u ? c_u_out : c_l_out, c_l_out};
    float* pbz[2], *pcz[2];
    for (int z = 0; z < 2; ++z) {
      pbz[z] = workspace + (int64_t)(2 * z) * nchunks * M;
      pcz[z] = workspace + (int64_t)(2 * z + 1) * nchunks * M;
    }
    const bool bias_in = bias != nullptr;
    const int64_t wgs = ceil_div(D, 4) * nchunks;
    BF_REQUIRE(wgs < (1LL << 31), "bf_crown_relu_linear_relu_fwd: too many domains");
    hipLaunchKernelGGL(small_k_relax_epi_kernel, dim3((unsigned)wgs, (unsigned)nz), dim3(256), 0,
                       stream, As[0], As[1], a_dstride, D, S, (int)N, W_t, P, bias, bi[0], bi[1],
                       reinterpret_cast<const float4*>(relax_next), add_next, add_next_ld, bias_next, cvec_next,
                       cvec_next_ld, an[0], an[1], ap[0], ap[1], bias_in ? bo[0] : nullptr, bias_in ? bo[1] : nullptr,
                       pbz[0], pbz[1], pcz[0], pcz[1], A_u == nullptr ? 1 : 0, nchunks);
    BF_LAUNCH_CHECK("small_k_relax_epi_kernel");
    for (int z = 0; z < nz; ++z) {
      const int rc = rows_finalize(bias_in ? bo[z] : bi[z], pbz[z], cvec_next ? pcz[z] : nullptr, nchunks, M, bo[z],
                                   cvec_next ? co[z] : nullptr, stream);
      if (rc) return rc;
    }
    return BF_OK;
  }
  const int nparts = gemm_partial_count(P);
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  int nz = 0;
  float* pb[2] = {nullptr, nullptr};
  float* pc[2] = {nullptr, nullptr};
  float* cdst[2] = {nullptr, nullptr};
  const float* bsrc[2] = {nullptr, nullptr};
  float* bdst[2] = {nullptr, nullptr};
  const bool relax_in = relax || add_l || bias;   // prologue relaxation (else A is already relaxed)
  for (int side = 0; side < 2; ++side) {
    const float* Ain = side == 0 ? A_u : A_l;
    if (!Ain) continue;
    a.A[nz] = Ain;
    a.C[nz] = side == 0 ? A_next_u : A_next_l;
    a.C_pre[nz] = side == 0 ? A_pre_u : A_pre_l;
    a.b_in[nz] = side == 0 ? b_u_in : b_l_in;
    bdst[nz] = side == 0 ? b_u_out : b_l_out;
    a.b_out[nz] = relax_in ? bdst[nz] : nullptr;
    bsrc[nz] = relax_in ? bdst[nz] : a.b_in[nz];
    pb[nz] = workspace + (int64_t)(2 * nz) * nparts * M;
    pc[nz] = workspace + (int64_t)(2 * nz + 1) * nparts * M;
    cdst[nz] = cvec_next ? (side == 0 ? c_u_out : c_l_out) : nullptr;
    a.partial[nz] = pb[nz];
    a.partial_c[nz] = pc[nz];
    ++nz;
  }
  a.z_lower_first = (A_u == nullptr) ? 1 : 0;
  a.lda = N;
  a.lda_d = a_dstride;
  a.ldc = P;
  a.B = W_t;
  a.trans_b = 1;
  a.ldb = N;
  a.M = M;
  a.N = P;
  a.K = N;
  a.S = S;
  a.relax = reinterpret_cast<const float4*>(relax);
  a.add_l = add_l;
  a.add_ld = add_ld;
  a.kbias = bias;
  a.e_relax = reinterpret_cast<const float4*>(relax_next);
  a.e_add = add_next;
  a.e_add_ld = add_next_ld;
  a.e_kbias = bias_next;
  a.e_cvec = cvec_next;
  a.e_cvec_ld = cvec_next_ld;
  int rc = gemm_dispatch(a, relax_in ? PRO_RELAX : PRO_PLAIN, EPI_RELAX, nz, stream);
  if (rc) return rc;
  for (int z = 0; z < nz; ++z) {
    rc = rows_finalize(bsrc[z], pb[z], pc[z], nparts, M, bdst[z], cdst[z], stream);
    if (rc) return rc;
  }
  return BF_OK;
}

int64_t bf_crown_relu_linear_relu_fwd_workspace(int64_t D, int64_t S, int64_t P) {
  return 4 * (int64_t)gemm_partial_count(P) * D * S;
}

int bf_crown_linear_concretize(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S,
                               int64_t N, const float* W_t, int64_t I, const float* rad, float eps, int norm_p,
                               const float* cen_u, const float* cen_l, const float* b_u, const float* b_l,
                               const float* h_scale, float* h_out, float* workspace, float* lb, float* ub,
                               hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S > 0 && N > 0 && I > 0, "bf_crown_linear_concretize: bad sizes");
  BF_REQUIRE(norm_p >= 0 && norm_p <= 2 && (norm_p == 0 || rad == nullptr),
             "bf_crown_linear_concretize: norm_p %d (0 Linf/box, 1 L1, 2 L2; the box radius goes with 0 only)",
             norm_p);
  const int64_t M = D * S;
  if (M == 0) return BF_OK;
  BF_REQUIRE(W_t && workspace, "bf_crown_linear_concretize: null weight or workspace");
  BF_REQUIRE((A_u == nullptr || (ub && cen_u && b_u)) && (A_l == nullptr || (lb && cen_l && b_l)) && (A_u || A_l),
             "bf_crown_linear_concretize: missing coefficient, center, bias or output");
  const int nparts = gemm_norm_partial_count(M, I, PRO_PLAIN);
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  int nz = 0;
  float* pu = workspace;
  float* pl = workspace + (int64_t)nparts * M;
  if (A_u) {
    a.A[nz] = A_u; a.partial[nz] = pu; ++nz;
  }
  if (A_l) {
    a.A[nz] = A_l; a.partial[nz] = pl; ++nz;
  }
  a.z_lower_first = (A_u == nullptr) ? 1 : 0;
  a.lda = N;
  a.lda_d = a_dstride;
  a.B = W_t;
  a.trans_b = 1;
  a.ldb = N;
  a.M = M;
  a.N = I;
  a.K = N;
  a.S = S;
  a.wvec = rad;
  a.w_ld = I;
  BF_REQUIRE((h_out == nullptr) == (h_scale == nullptr) && (h_out == nullptr || A_l != nullptr),
             "bf_crown_linear_concretize: h_out needs h_scale and the lower coefficient");
  a.h_scale = h_scale;
  a.h_out = h_out;
  a.norm_kind = norm_p;
  int rc = gemm_dispatch(a, PRO_PLAIN, EPI_ABSSUM, nz, stream);
  if (rc) return rc;
  if (h_out && norm_p != 0) {
    rc = lp_seed_rows(h_out, M, I, h_scale, norm_p, stream);   // h_out holds the lower coefficient A W
    if (rc) return rc;
  }
  return concretize_finalize(A_u ? pu : nullptr, A_l ? pl : nullptr, nparts, M, cen_u, cen_l, b_u, b_l,
                             rad ? 1.0f : eps, norm_p, A_l ? lb : nullptr, A_u ? ub : nullptr, stream);
}

int64_t bf_crown_linear_concretize_workspace(int64_t D, int64_t S, int64_t I) {
  return 2 * (int64_t)gemm_norm_partial_count(D * S, I, PRO_PLAIN) * D * S;
}

// sums_only: the row sums alone, no coefficient written (A_u_out / A_l_out NULL).
static int relax_pass(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t K,
                      const RelaxSrc& src, const float* add_l, int64_t add_ld, const float* kbias, const float* cvec,
                      const float* b_u_in, const float* b_l_in, float* A_u_out, float* A_l_out, float* b_u_out,
                      float* b_l_out, float* c_u_out, float* c_l_out, hipStream_t stream, bool sums_only) {
  BF_REQUIRE(D >= 0 && S >= 0 && K > 0, "bf_crown_relu_relax: bad sizes");
  const int64_t M = D * S;
  if (M == 0) return BF_OK;
  BF_REQUIRE(((uintptr_t)src.table & 15) == 0, "bf_crown_relu_relax: relax table must be 16-byte aligned");
  BF_REQUIRE((src.lo == nullptr) == (src.hi == nullptr), "bf_crown_relu_relax: give both pre_lo and pre_hi");
  BF_REQUIRE(sums_only ? (A_u_out == nullptr && A_l_out == nullptr)
                       : ((A_u == nullptr) == (A_u_out == nullptr) && (A_l == nullptr) == (A_l_out == nullptr)),
             "bf_crown_relu_relax: input/output mismatch");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool vec = (K % 4 == 0) && (a_dstride % 4 == 0) && al16(A_u) && al16(A_l) && al16(A_u_out) &&
                   al16(A_l_out) && al16(kbias) &&
                   al16(cvec) && al16(add_l) && (add_l == nullptr || add_ld % 4 == 0) && al16(src.lo) &&
                   al16(src.hi) && al16(src.alpha) && (src.alpha_ld % 4 == 0);
  if (vec && K <= 512 && (a_dstride == 0 ? S >= 16 : (S >= 8 && M >= 8192))) {
    // a shared coefficient: 16 rows of one domain per workgroup (4 per wave), the
    // domain's operands held in registers across them (C2's 500 x 500 shape: 8, 16 and
    // 64 rows per workgroup measured 150, 129 and 141 us, the per-row kernel 156 us).
    // A per-domain coefficient of many rows takes the same kernel: its rows are read
    // once either way, and the domain's operands are loaded once per wave, not per row.
    const int rpw = S < 16 ? (int)S : 16;
    const int64_t chunks = ceil_div(S, rpw);
    BF_REQUIRE(D * chunks < (1LL << 31), "bf_crown_relu_relax: too many rows");
    if (K <= 256)
      hipLaunchKernelGGL(relu_relax_shared_kernel<1>, dim3((unsigned)(D * chunks)), dim3(256), 0, stream, A_u, A_l,
                         a_dstride, S,
                         K, chunks, rpw, src, add_l, add_ld, kbias, cvec, b_u_in, b_l_in, A_u_out, A_l_out, b_u_out,
                         b_l_out, c_u_out, c_l_out);
    else
      hipLaunchKernelGGL(relu_relax_shared_kernel<2>, dim3((unsigned)(D * chunks)), dim3(256), 0, stream, A_u, A_l,
                         a_dstride, S,
                         K, chunks, rpw, src, add_l, add_ld, kbias, cvec, b_u_in, b_l_in, A_u_out, A_l_out, b_u_out,
                         b_l_out, c_u_out, c_l_out);
    BF_LAUNCH_CHECK("relu_relax_shared_kernel");
  } else if (vec && K >= 1024) {
    hipLaunchKernelGGL(relu_relax_rows4_kernel<256>, dim3((unsigned)M), dim3(256), 0, stream, A_u, A_l, a_dstride, M, S,
                       K, src, add_l, add_ld, kbias, cvec, b_u_in, b_l_in, A_u_out, A_l_out, b_u_out, b_l_out, c_u_out,
                       c_l_out);
    BF_LAUNCH_CHECK("relu_relax_rows4_kernel<256>");
  } else if (vec) {
    hipLaunchKernelGGL(relu_relax_rows4_kernel<64>, dim3((unsigned)ceil_div(M, 4)), dim3(256), 0, stream, A_u, A_l,
                       a_dstride, M, S, K, src, add_l, add_ld, kbias, cvec, b_u_in, b_l_in, A_u_out, A_l_out, b_u_out,
                       b_l_out, c_u_out, c_l_out);
    BF_LAUNCH_CHECK("relu_relax_rows4_kernel<64>");
  } else {
    hipLaunchKernelGGL(relu_relax_rows_kernel, dim3((unsigned)ceil_div(M, 4)), dim3(256), 0, stream, A_u, A_l,
                       a_dstride, M, S, K, src, add_l, add_ld, kbias, cvec, b_u_in, b_l_in, A_u_out, A_l_out, b_u_out,
                       b_l_out, c_u_out, c_l_out);
    BF_LAUNCH_CHECK("relu_relax_rows_kernel");
  }
  return BF_OK;
}

int bf_crown_relu_relax(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t K,
                        const float* relax,
                        const float* add_l, int64_t add_ld, const float* kbias, const float* cvec,
                        const float* b_u_in, const float* b_l_in, float* A_u_out, float* A_l_out, float* b_u_out,
                        float* b_l_out, float* c_u_out, float* c_l_out, hipStream_t stream) {
  const RelaxSrc src{reinterpret_cast<const float4*>(relax), nullptr, nullptr, nullptr, 0};
  return relax_pass(A_u, A_l, a_dstride, D, S, K, src, add_l, add_ld, kbias, cvec, b_u_in, b_l_in, A_u_out, A_l_out,
                    b_u_out, b_l_out, c_u_out, c_l_out, stream, false);
}

int bf_crown_relu_relax_lu(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t K,
                           const float* pre_lo, const float* pre_hi, const float* alpha, int64_t alpha_ld,
                           const float* add_l, int64_t add_ld, const float* kbias, const float* cvec,
                           const float* b_u_in, const float* b_l_in, float* A_u_out, float* A_l_out, float* b_u_out,
                           float* b_l_out, float* c_u_out, float* c_l_out, hipStream_t stream) {
  BF_REQUIRE(alpha == nullptr || alpha_ld == 0 || alpha_ld >= K, "bf_crown_relu_relax_lu: bad alpha_ld");
  const RelaxSrc src{nullptr, pre_lo, pre_hi, alpha, alpha_ld};
  return relax_pass(A_u, A_l, a_dstride, D, S, K, src, add_l, add_ld, kbias, cvec, b_u_in, b_l_in, A_u_out, A_l_out,
                    b_u_out, b_l_out, c_u_out, c_l_out, stream, false);
}

int bf_concretize_dense(const float* A, int64_t D, int64_t S, int64_t I, const float* center, const float* rad,
                        float eps, int norm_p, const float* b, int is_lower, float* out, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && S >= 0 && I > 0, "bf_concretize_dense: bad sizes");
  BF_REQUIRE(norm_p >= 0 && norm_p <= 2 && (norm_p == 0 || rad == nullptr),
             "bf_concretize_dense: norm_p %d (0 Linf/box, 1 L1, 2 L2; the box radius goes with 0 only)", norm_p);
  const int64_t M = D * S;
  if (M == 0) return BF_OK;
  BF_REQUIRE(A && center && out, "bf_concretize_dense: null pointer");
  BF_REQUIRE(((uintptr_t)A % 16) == 0 && ((uintptr_t)center % 16) == 0, "bf_concretize_dense: unaligned");
  hipLaunchKernelGGL(concretize_rows_kernel, dim3((unsigned)ceil_div(M, 4)), dim3(256), 0, stream, A, M, S, I,
                     center, rad, rad ? 1.0f : eps, norm_p, b, is_lower, out);
  BF_LAUNCH_CHECK("concretize_rows_kernel");
  return BF_OK;
}

// c = Xc . W^T and, when Xr is given, r = Xr . |W|^T, as one launch of the
// contraction kernel (product z = blockIdx.y).  An output of few tiles (a small
// batch) is split along K into the partial buffer `part`, whose chunks are added
// in chunk order.
// When K is split (*ks > 1), the partial products stay in `part` ([z][s][B*N]) for
// the finalize kernel to sum; otherwise c (and r) hold the products.
// ivl_hi: xc = xr hold an interval's lower bounds and ivl_hi its upper ones; the products
// read their center and radius (of the ReLU when relu) as the operand tiles are loaded.
static int ibp_products(const float* xc, const float* xr, const float* W, int64_t B, int64_t K, int64_t N, float* c,
                        float* r, float* part, int* ks_out, hipStream_t stream, const float* ivl_hi = nullptr,
                        int relu = 0) {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  const int nz = xr ? 2 : 1;
  a.A[0] = xc;
  a.C[0] = c;
  a.A[1] = xr;
  a.C[1] = r;
  a.ivl_hi = ivl_hi;
  a.ivl_relu = relu;
  a.lda = K;
  a.lda_d = K;
  a.ldc = N;
  a.B = W;
  a.ldb = K;
  a.trans_b = 1;
  a.abs_b = 2;   // product 1 takes |W|
  a.M = B;
  a.N = N;
  a.K = K;
  a.S = 1;
  int64_t kchunk = K;
  const int ks = gemm_ksplit(B, N, K, &kchunk);
  if (ks > 1) {
    a.ksplit = ks;
    a.kchunk = kchunk;
    a.part = part;
  }
  *ks_out = ks;
  return gemm_dispatch(a, PRO_PLAIN, EPI_STORE, nz, stream);
}

int bf_ibp_linear(const float* in_lo, const float* in_hi, int64_t B, int64_t K, int input_kind, float eps,
                  int apply_relu, const float* W, const float* bias, int64_t N, const int8_t* split, int64_t split_ld,
                  float* workspace, float* out_lo, float* out_hi, float* center_out, int* infeasible,
                  float* box_radius_out, hipStream_t stream) {
  // input_kind 0: interval [in_lo, in_hi] (optionally through ReLU) or box; 1: Linf ball around in_lo;
  // 2: L2 ball; 3: L1 ball (the row norm of W is the ball's dual norm, perturbation.py:127-136)
  BF_REQUIRE(B >= 0 && K > 0 && N > 0 && input_kind >= 0 && input_kind <= 3, "bf_ibp_linear: bad sizes or input kind");
  if (B == 0) return BF_OK;
  BF_REQUIRE(in_lo && W && out_lo && out_hi && workspace, "bf_ibp_linear: null pointer");
  // workspace: c [B*N], r [B*N], rownorm [N], split-K partials
  float* c = workspace;
  float* r = c + B * N;
  float* rownorm = r + B * N;
  float* part = rownorm + N;
  float* cdst = center_out ? center_out : c;
  int rc;
  int ks = 1;
  BF_REQUIRE(input_kind >= 1 || in_hi, "bf_ibp_linear: interval input needs in_hi");
  BF_REQUIRE(box_radius_out == nullptr || (input_kind == 0 && apply_relu == 0),
             "bf_ibp_linear: box_radius_out is for a box input without ReLU");
  if (small_out_route(B, N)) {
    // a small output: products and finalize in one launch (row norm code as row_norm_kernel),
    // the box radius written from the loaded bounds
    const int nk = input_kind == 1 ? 0 : (input_kind == 2 ? 2 : 1);
    return ibp_linear_small(in_lo, input_kind >= 1 ? nullptr : in_hi, apply_relu, nk, eps, W, bias, B, K, N, split,
                            split_ld, out_lo, out_hi, center_out, infeasible, box_radius_out, stream);
  }
  if (box_radius_out) {
    rc = ibp_center_radius(in_lo, in_hi, B * K, 0, nullptr, box_radius_out, stream);
    if (rc) return rc;
  }
  if (input_kind >= 1) {
    rc = ibp_products(in_lo, nullptr, W, B, K, N, cdst, nullptr, part, &ks, stream);
    if (rc) return rc;
    const int kind = input_kind == 1 ? 0 : (input_kind == 2 ? 2 : 1);
    hipLaunchKernelGGL(row_norm_kernel, dim3((unsigned)N), dim3(256), 0, stream, W, N, K, kind, rownorm);
    BF_LAUNCH_CHECK("row_norm_kernel");
    return ibp_finalize_parts(cdst, nullptr, ks > 1 ? part : nullptr, ks, 0, center_out, rownorm, eps, bias, 1,
                              split, split_ld, B, N, out_lo, out_hi, infeasible, stream);
  }
  BF_REQUIRE(in_hi, "bf_ibp_linear: interval input needs in_hi");
  // the center and radius (of the ReLU when apply_relu) made as the products load their tiles
  rc = ibp_products(in_lo, in_lo, W, B, K, N, cdst, r, part, &ks, stream, in_hi, apply_relu);
  if (rc) return rc;
  return ibp_finalize_parts(cdst, r, ks > 1 ? part : nullptr, ks, 1, center_out, nullptr, 0.f, bias, 1, split,
                            split_ld, B, N, out_lo, out_hi, infeasible, stream);
}

int64_t bf_ibp_linear_workspace(int64_t B, int64_t K, int64_t N) {
  int64_t kchunk;
  const int ks = gemm_ksplit(B, N, K, &kchunk);
  return 2 * B * N + N + (ks > 1 ? 2 * (int64_t)ks * B * N : 0);
}

int bf_interval_center_radius(const float* lo, const float* hi, int64_t n, int apply_relu, float* mid, float* rad,
                              hipStream_t stream) {
  BF_REQUIRE(n >= 0, "bf_interval_center_radius: bad size");
  if (n == 0 || (mid == nullptr && rad == nullptr)) return BF_OK;
  BF_REQUIRE(lo && hi, "bf_interval_center_radius: null pointer");
  return ibp_center_radius(lo, hi, n, apply_relu, mid, rad, stream);
}

int bf_interval_relu(const float* lo, const float* hi, int64_t n, float* out_lo, float* out_hi, hipStream_t stream) {
  BF_REQUIRE(n >= 0, "bf_interval_relu: bad size");
  if (n == 0) return BF_OK;
  BF_REQUIRE(lo && hi && out_lo && out_hi, "bf_interval_relu: null pointer");
  hipLaunchKernelGGL(interval_relu_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, lo, hi, n, out_lo,
                     out_hi);
  BF_LAUNCH_CHECK("interval_relu_kernel");
  return BF_OK;
}

int bf_interval_add(const float* a_lo, const float* a_hi, const float* b_lo, const float* b_hi, int64_t n,
                    float* out_lo, float* out_hi, hipStream_t stream) {
  BF_REQUIRE(n >= 0, "bf_interval_add: bad size");
  if (n == 0) return BF_OK;
  BF_REQUIRE(a_lo && a_hi && b_lo && b_hi && out_lo && out_hi, "bf_interval_add: null pointer");
  hipLaunchKernelGGL(interval_add_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, a_lo, a_hi, b_lo,
                     b_hi, n, out_lo, out_hi);
  BF_LAUNCH_CHECK("interval_add_kernel");
  return BF_OK;
}

int bf_interval_mul(const float* a_lo, const float* a_hi, const float* b_lo, const float* b_hi, int64_t n,
                    float* out_lo, float* out_hi, hipStream_t stream) {
  BF_REQUIRE(n >= 0, "bf_interval_mul: bad size");
  if (n == 0) return BF_OK;
  BF_REQUIRE(a_lo && a_hi && b_lo && b_hi && out_lo && out_hi, "bf_interval_mul: null pointer");
  hipLaunchKernelGGL(interval_mul_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, a_lo, a_hi, b_lo,
                     b_hi, n, out_lo, out_hi);
  BF_LAUNCH_CHECK("interval_mul_kernel");
  return BF_OK;
}

int bf_spec_linear(const float* C, const float* lo, const float* hi, int64_t B, int64_t S, int64_t O, float* out_lo,
                   float* out_hi, hipStream_t stream) {
  BF_REQUIRE(B >= 0 && S >= 0 && O > 0, "bf_spec_linear: bad sizes");
  if (B * S == 0) return BF_OK;
  BF_REQUIRE(C && lo && hi && out_lo && out_hi, "bf_spec_linear: null pointer");
  hipLaunchKernelGGL(spec_linear_kernel, dim3((unsigned)ceil_div(B * S, 256)), dim3(256), 0, stream, C, lo, hi, B, S,
                     O, out_lo, out_hi);
  BF_LAUNCH_CHECK("spec_linear_kernel");
  return BF_OK;
}

int bf_ibp_batched_linear(const float* lo, const float* hi, int64_t B, int64_t I, const float* W, const float* bias,
                          int64_t O, float* out_lo, float* out_hi, hipStream_t stream) {
  BF_REQUIRE(B >= 0 && I > 0 && O > 0, "bf_ibp_batched_linear: bad sizes");
  if (B == 0) return BF_OK;
  BF_REQUIRE(lo && hi && W && out_lo && out_hi, "bf_ibp_batched_linear: null pointer");
  hipLaunchKernelGGL(ibp_batched_linear_kernel, dim3((unsigned)ceil_div(B * O, 4)), dim3(256), 0, stream, lo, hi, B,
                     I, W, bias, O, out_lo, out_hi);
  BF_LAUNCH_CHECK("ibp_batched_linear_kernel");
  return BF_OK;
}

int bf_interval_clip(float* lo, float* hi, const float* clo, const float* chi, const int8_t* split, int64_t split_ld,
                     int64_t B, int64_t N, int* infeasible, hipStream_t stream) {
  BF_REQUIRE(B >= 0 && N >= 0, "bf_interval_clip: bad sizes");
  if (B * N == 0) return BF_OK;
  BF_REQUIRE(lo && hi && ((clo == nullptr) == (chi == nullptr)), "bf_interval_clip: null pointer");
  hipLaunchKernelGGL(interval_clip_kernel, dim3((unsigned)ceil_div(B * N, 256)), dim3(256), 0, stream, lo, hi, clo,
                     chi, split, split_ld, B, N, infeasible);
  BF_LAUNCH_CHECK("interval_clip_kernel");
  return BF_OK;
}

int bf_branch_update(const float* lo, const float* hi, int64_t D, int64_t N, int layer, float* best_gap,
                     int* best_layer, int* best_idx, hipStream_t stream) {
  BF_REQUIRE(D >= 0 && N >= 0, "bf_branch_update: bad sizes");
  if (D == 0 || N == 0) return BF_OK;
  BF_REQUIRE(lo && hi && best_gap && best_layer && best_idx, "bf_branch_update: null pointer");
  hipLaunchKernelGGL(branch_update_kernel, dim3((unsigned)ceil_div(D, 4)), dim3(256), 0, stream, lo, hi, D, N, layer,
                     best_gap, best_layer, best_idx);
  BF_LAUNCH_CHECK("branch_update_kernel");
  return BF_OK;
}

int bf_adam_clamp_step(float* p, float* m, float* v, const float* g, int64_t n, double lr, double beta1,
                       double beta2, float eps, int step, float clamp_lo, float clamp_hi, int has_clamp_hi,
                       hipStream_t stream) {
  BF_REQUIRE(n >= 0 && step >= 1, "bf_adam_clamp_step: bad arguments");
  if (n == 0) return BF_OK;
  BF_REQUIRE(p && m && v && g, "bf_adam_clamp_step: null pointer");
  // bias corrections in double then rounded, as torch computes them from Python floats
  const double bc1 = 1.0 - __builtin_pow((double)beta1, (double)step);
  const double bc2 = 1.0 - __builtin_pow((double)beta2, (double)step);
  const float neg_step = (float)(-((double)lr / bc1));
  const float bc2_sqrt = (float)__builtin_sqrt(bc2);
  const float w1 = (float)(1.0 - (double)beta1);
  const float w2 = (float)(1.0 - (double)beta2);
  hipLaunchKernelGGL(adam_clamp_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, p, m, v, g, n, w1,
                     beta2, w2, eps, neg_step, bc2_sqrt, clamp_lo, clamp_hi, has_clamp_hi, (int)(step == 1));
  BF_LAUNCH_CHECK("adam_clamp_kernel");
  return BF_OK;
}

static void adam_consts(double lr, double beta1, double beta2, int step, float* w1, float* w2, float* neg_step,
                        float* bc2_sqrt) {
  // bias corrections in double then rounded, as torch computes them from Python floats
  const double bc1 = 1.0 - __builtin_pow((double)beta1, (double)step);
  const double bc2 = 1.0 - __builtin_pow((double)beta2, (double)step);
  *neg_step = (float)(-((double)lr / bc1));
  *bc2_sqrt = (float)__builtin_sqrt(bc2);
  *w1 = (float)(1.0 - (double)beta1);
  *w2 = (float)(1.0 - (double)beta2);
}

int bf_adam_clamp_multi(int count, float* const* p, float* const* m, float* const* v, const float* const* g,
                        const int64_t* n, const float* clamp_lo, const float* clamp_hi, const int* has_clamp_hi,
                        double lr, double beta1, double beta2, float eps, int step, float* const* best,
                        const int* improved, int64_t rows, hipStream_t stream) {
  BF_REQUIRE(count >= 0 && step >= 1, "bf_adam_clamp_multi: bad arguments");
  BF_REQUIRE(count == 0 || (p && m && v && g && n && clamp_lo && clamp_hi && has_clamp_hi),
             "bf_adam_clamp_multi: null array");
  BF_REQUIRE(best == nullptr || (improved && rows > 0), "bf_adam_clamp_multi: the best-of copy needs improved and rows");
  float w1, w2, neg_step, bc2_sqrt;
  adam_consts(lr, beta1, beta2, step, &w1, &w2, &neg_step, &bc2_sqrt);
  for (int base = 0; base < count; base += BF_SEG_MAX) {
    AdamSegs a;
    memset(&a, 0, sizeof(a));
    a.count = count - base < BF_SEG_MAX ? count - base : BF_SEG_MAX;
    int64_t blocks = 0;
    for (int t = 0; t < a.count; ++t) {
      const int k = base + t;
      BF_REQUIRE(n[k] >= 0 && (n[k] == 0 || (p[k] && m[k] && v[k] && g[k])), "bf_adam_clamp_multi: tensor %d", k);
      a.p[t] = p[k]; a.m[t] = m[k]; a.v[t] = v[k]; a.g[t] = g[k]; a.n[t] = n[k];
      if (best) {
        BF_REQUIRE(best[k] && n[k] % rows == 0, "bf_adam_clamp_multi: best-of tensor %d (%lld elements, %lld rows)", k,
                   (long long)n[k], (long long)rows);
        a.best[t] = best[k];
        a.ncol[t] = n[k] / rows;
      }
      a.lo[t] = clamp_lo[k]; a.hi[t] = clamp_hi[k]; a.clamp_hi[t] = has_clamp_hi[k];
      a.bstart[t] = blocks;
      blocks += ceil_div(n[k], 256);
    }
    a.bstart[a.count] = blocks;
    if (blocks == 0) continue;
    BF_REQUIRE(blocks < (1LL << 31), "bf_adam_clamp_multi: too many elements");
    hipLaunchKernelGGL(adam_clamp_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a, w1, (float)beta2,
                       w2, eps, neg_step, bc2_sqrt, improved, (int)(step == 1));
    BF_LAUNCH_CHECK("adam_clamp_multi_kernel");
  }
  return BF_OK;
}

int bf_masked_copy_rows_multi(int count, float* const* dst, const float* const* src, const int64_t* ncol, int64_t D,
                              const int* mask, hipStream_t stream) {
  BF_REQUIRE(count >= 0 && D >= 0, "bf_masked_copy_rows_multi: bad arguments");
  BF_REQUIRE(count == 0 || D == 0 || (dst && src && ncol && mask), "bf_masked_copy_rows_multi: null array");
  for (int base = 0; base < count; base += BF_SEG_MAX) {
    CopySegs c;
    memset(&c, 0, sizeof(c));
    c.count = count - base < BF_SEG_MAX ? count - base : BF_SEG_MAX;
    bool quad = true;
    for (int t = 0; t < c.count; ++t) {
      const int k = base + t;
      BF_REQUIRE(ncol[k] > 0 && dst[k] && src[k], "bf_masked_copy_rows_multi: tensor %d", k);
      c.dst[t] = dst[k]; c.src[t] = src[k]; c.ncol[t] = ncol[k];
      quad = quad && ncol[k] % 4 == 0 && ((uintptr_t)dst[k] & 15) == 0 && ((uintptr_t)src[k] & 15) == 0;
    }
    int64_t blocks = 0;
    for (int t = 0; t < c.count; ++t) {
      c.bstart[t] = blocks;
      blocks += ceil_div(D * (quad ? ncol[base + t] / 4 : ncol[base + t]), 256);
    }
    c.bstart[c.count] = blocks;
    if (blocks == 0) continue;
    BF_REQUIRE(blocks < (1LL << 31), "bf_masked_copy_rows_multi: too many elements");
    if (quad)
      hipLaunchKernelGGL(masked_copy_rows_multi_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, c, D, mask);
    else
      hipLaunchKernelGGL(masked_copy_rows_multi_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, c, D,
                         mask);
    BF_LAUNCH_CHECK("masked_copy_rows_multi_kernel");
  }
  return BF_OK;
}

int bf_beta_coeff_multi(int count, const float* const* beta, const int64_t* beta_ld, const int8_t* const* split,
                        const int64_t* split_ld, const int64_t* ncol, int64_t D, float* const* out,
                        hipStream_t stream) {
  BF_REQUIRE(count >= 0 && D >= 0, "bf_beta_coeff_multi: bad arguments");
  BF_REQUIRE(count == 0 || D == 0 || (beta && beta_ld && split && split_ld && ncol && out),
             "bf_beta_coeff_multi: null array");
  for (int base = 0; base < count; base += BF_SEG_MAX) {
    BetaSegs b;
    memset(&b, 0, sizeof(b));
    b.count = count - base < BF_SEG_MAX ? count - base : BF_SEG_MAX;
    bool quad = true;
    for (int t = 0; t < b.count; ++t) {
      const int k = base + t;
      BF_REQUIRE(ncol[k] > 0 && beta[k] && split[k] && out[k], "bf_beta_coeff_multi: tensor %d", k);
      b.beta[t] = beta[k]; b.beta_ld[t] = beta_ld[k]; b.split[t] = split[k]; b.split_ld[t] = split_ld[k];
      b.ncol[t] = ncol[k]; b.out[t] = out[k];
      quad = quad && ncol[k] % 4 == 0 && beta_ld[k] % 4 == 0 && split_ld[k] % 4 == 0 &&
             ((uintptr_t)beta[k] & 15) == 0 && ((uintptr_t)out[k] & 15) == 0 && ((uintptr_t)split[k] & 3) == 0;
    }
    int64_t blocks = 0;
    for (int t = 0; t < b.count; ++t) {
      b.bstart[t] = blocks;
      blocks += ceil_div(D * (quad ? ncol[base + t] / 4 : ncol[base + t]), 256);
    }
    b.bstart[b.count] = blocks;
    if (blocks == 0) continue;
    BF_REQUIRE(blocks < (1LL << 31), "bf_beta_coeff_multi: too many elements");
    if (quad)
      hipLaunchKernelGGL(beta_coeff_multi_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, b, D);
    else
      hipLaunchKernelGGL(beta_coeff_multi_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, b, D);
    BF_LAUNCH_CHECK("beta_coeff_multi_kernel");
  }
  return BF_OK;
}

}  // extern "C"
