// Dispatch of the fp32 MFMA contraction (bf_gemm_kernel.h) over its tile
// configurations, and the small kernels around it: the relaxation table, the
// concretization finalize and the split-K reduction.

#include <cstdlib>
#include <cstring>

#include "bf_gemm_kernel.h"

namespace bf {

constexpr int RELAX_SEG_MAX = 16;  // tables per relax_table_multi_kernel launch

// The per-column-block partial norms combined in a fixed order -- summed (norm_p 0:
// Linf ball, box), their maximum (1: L1 ball, the dual norm max |A|), the square root
// of their sum (2: L2 ball) -- then
//   lb = (center - eps * norm) + b,   ub = (center + eps * norm) + b
// (perturbation.py:175-222; box: eps = 1 and the norm is already radius-weighted).
__device__ __forceinline__ float combine_parts(const float* __restrict__ part, int nparts, int64_t M, int64_t m,
                                               int norm_p) {
  // the partials' loads issued eight at a time, combined in block order
  float s = 0.f;
  int q = 0;
  for (; q + 8 <= nparts; q += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(q + u) * M + m];
#pragma unroll
    for (int u = 0; u < 8; ++u) s = norm_p == 1 ? fmaxf(s, v[u]) : s + v[u];
  }
  for (; q < nparts; ++q) {
    const float v = part[(int64_t)q * M + m];
    s = norm_p == 1 ? fmaxf(s, v) : s + v;
  }
  return norm_p == 2 ? sqrtf(s) : s;
}

__global__ void concretize_finalize_kernel(const float* __restrict__ partial_u, const float* __restrict__ partial_l,
                                           int nparts, int64_t M, const float* __restrict__ cen_u,
                                           const float* __restrict__ cen_l, const float* __restrict__ b_u,
                                           const float* __restrict__ b_l, float eps, int norm_p,
                                           float* __restrict__ lb, float* __restrict__ ub) {
  int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  if (ub) ub[m] = (cen_u[m] + eps * combine_parts(partial_u, nparts, M, m, norm_p)) + b_u[m];
  if (lb) lb[m] = (cen_l[m] - eps * combine_parts(partial_l, nparts, M, m, norm_p)) + b_l[m];
}

// Slopes/intercepts of the ReLU relaxation per (domain, neuron)
// (crown_ibp.py:722-758, 1176-1208): {alpha_u, beta_u, alpha_l, beta_l}, with the
// optional lower-slope override clamp(alpha, 0, 1) on ambiguous neurons.
__device__ __forceinline__ void relax_table_elem(const float* __restrict__ lo, const float* __restrict__ hi,
                                                 const float* __restrict__ alpha, int64_t alpha_ld, int64_t D,
                                                 int64_t K, float4* __restrict__ out, int64_t i) {
  if (i >= D * K) return;
  const int64_t d = div_rows(i, K, D * K < (1LL << 31)), k = i - d * K;
  const bool has_alpha = alpha != nullptr;
  const float a = has_alpha ? clamp01(alpha[d * alpha_ld + k]) : 0.f;
  const Relax r = relu_relax(lo[i], hi[i], has_alpha, a);
  out[i] = make_float4(r.au, r.bu, r.al, r.bl);
}

__global__ void relax_table_kernel(const float* __restrict__ lo, const float* __restrict__ hi,
                                   const float* __restrict__ alpha, int64_t alpha_ld, int64_t D, int64_t K,
                                   float4* __restrict__ out) {
  relax_table_elem(lo, hi, alpha, alpha_ld, D, K, out, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// Several ReLUs' tables in one launch: table s owns blocks [bstart[s], bstart[s+1]).
struct TableSegs {
  const float* lo[RELAX_SEG_MAX];
  const float* hi[RELAX_SEG_MAX];
  const float* alpha[RELAX_SEG_MAX];
  int64_t alpha_ld[RELAX_SEG_MAX];
  int64_t K[RELAX_SEG_MAX];
  float4* out[RELAX_SEG_MAX];
  int64_t bstart[RELAX_SEG_MAX + 1];
  int count;
};

__global__ void relax_table_multi_kernel(TableSegs t, int64_t D) {
  int s = 0;
  while (s + 1 < t.count && (int64_t)blockIdx.x >= t.bstart[s + 1]) ++s;
  relax_table_elem(t.lo[s], t.hi[s], t.alpha[s], t.alpha_ld[s], D, t.K[s], t.out[s],
                   ((int64_t)blockIdx.x - t.bstart[s]) * blockDim.x + threadIdx.x);
}

// BOUNDFLOW_GEMM_TILE=G, =H, =Q or =S forces one configuration (for measurement);
// read once when the library is loaded, constant afterwards.
static int forced_tile_from_env() {
  const char* v = std::getenv("BOUNDFLOW_GEMM_TILE");
  if (v == nullptr) return 0;
  if (std::strcmp(v, "G") == 0) return 'G';
  if (std::strcmp(v, "H") == 0) return 'H';
  if (std::strcmp(v, "Q") == 0) return 'Q';
  if (std::strcmp(v, "S") == 0) return 'S';
  return 0;
}

// Share of the busiest CU's work that is useful when `tiles` equal tiles are dealt
// over the device's 256 CUs (tiles / 256 per CU on average, the ceiling on the
// busiest one).
static double quantization_efficiency(int64_t tiles) {
  const int64_t per_cu = ceil_div(tiles, (int64_t)256);
  return (double)tiles / (double)(256 * per_cu);
}
static const int kForcedTile = forced_tile_from_env();

// Tile configuration of a contraction: 'G', 'H', 'Q' or 'S'.  ks: K chunks of a split
// contraction (1 when unsplit); dl: the operands suit the direct-to-LDS loop.
int gemm_tile_choice(int64_t M, int64_t N, int nz, int64_t ks, int pro, bool dl) {
  if (kForcedTile) return kForcedTile;
  // measured on the benchmark shapes: the 8-wave TileG at 3 workgroups per CU for
  // every form; a grid with fewer 128 x 128 tiles than the device has CUs takes the
  // 16-wave TileH instead, which spreads each tile's contraction over twice the waves.
  const int64_t wgs = ceil_div(M, 128) * ceil_div(N, 128) * nz * ks;
  // A grid of fewer 128 x 128 tiles than the device has CUs takes, with the plain
  // prologue, the 4-wave 64 x 64 TileS, which deals four times as many tiles over
  // the CUs (C1 0.174 -> 0.164 ms, C3 0.257 -> 0.246, D1 0.771 -> 0.737); with the
  // relaxation prologue (more registers per wave) and for the |A W| and relaxation
  // epilogues (128 columns per tile) the 16-wave TileH.
  if (wgs < 256) return pro == PRO_PLAIN ? 'S' : 'H';
  // A grid whose 128 x 128 tiles leave the CUs unevenly loaded (C5's 576 tiles: 2.25
  // per CU run at the cost of 3) takes the 64 x 128 TileQ, whose twice as many tiles
  // at 6 workgroups per CU even it out (4.5 per CU at the cost of 5); TileQ is a few
  // per cent slower per flop, so only a clear gain in balance picks it.
  const int64_t wgs_q = ceil_div(M, 64) * ceil_div(N, 128) * nz * ks;
  if (pro == PRO_PLAIN && dl && quantization_efficiency(wgs_q) > quantization_efficiency(wgs) + 0.1) return 'Q';
  return 'G';
}

int gemm_norm_cols(int64_t M, int64_t N, int pro);

int gemm_dispatch(const GemmArgs& a, int pro, int epi, int nz, hipStream_t stream) {
  if ((pro != PRO_PLAIN && pro != PRO_RELAX) || (epi != EPI_STORE && epi != EPI_ABSSUM && epi != EPI_RELAX)) {
    set_error("gemm_dispatch: bad mode pro=%d epi=%d", pro, epi);
    return BF_EINVAL;
  }
  const int64_t ks = (pro == PRO_PLAIN && epi == EPI_STORE && a.ksplit > 1) ? a.ksplit : 1;
  const bool dl = gemm_dl_operands(a, nz);
  int t = gemm_tile_choice(a.M, a.N, nz, ks, pro, dl);
  // the norm and relaxation epilogues take 128 columns per tile: a short grid of them runs
  // as the 4-wave 64 x 128 TileQ when the operands suit its direct-to-LDS loop (twice the
  // tiles of TileH over as many CUs, each tile's K loop on one wave per SIMD), else TileH
  if (t == 'S' && epi != EPI_STORE) t = dl ? 'Q' : 'H';
  // the |A W| epilogue's partial norms are per gemm_norm_cols columns: 64 is TileS's width
  if (epi == EPI_ABSSUM && gemm_norm_cols(a.M, a.N, pro) == NORM_BN / 2) t = 'S';
  switch (t) {
    case 'S': return launch_tile<TileS>(a, pro, epi, nz, stream);
    case 'H': return launch_tile<TileH>(a, pro, epi, nz, stream);
    case 'Q': return launch_tile<TileQ>(a, pro, epi, nz, stream);
    default: return launch_tile<TileG>(a, pro, epi, nz, stream);
  }
}

int concretize_finalize(const float* pu, const float* pl, int nparts, int64_t M, const float* cu, const float* cl,
                        const float* bu, const float* bl, float eps, int norm_p, float* lb, float* ub,
                        hipStream_t stream) {
  if (M == 0) return BF_OK;
  BF_REQUIRE(norm_p >= 0 && norm_p <= 2, "concretize: norm_p %d (0 Linf/box, 1 L1, 2 L2)", norm_p);
  hipLaunchKernelGGL(concretize_finalize_kernel, dim3((unsigned)ceil_div(M, 256)), dim3(256), 0, stream, pu, pl,
                     nparts, M, cu, cl, bu, bl, eps, norm_p, lb, ub);
  BF_LAUNCH_CHECK("concretize_finalize_kernel");
  return BF_OK;
}

int relax_table(const float* lo, const float* hi, const float* alpha, int64_t alpha_ld, int64_t D, int64_t K,
                float4* out, hipStream_t stream) {
  if (D * K == 0) return BF_OK;
  hipLaunchKernelGGL(relax_table_kernel, dim3((unsigned)ceil_div(D * K, 256)), dim3(256), 0, stream, lo, hi, alpha,
                     alpha_ld, D, K, out);
  BF_LAUNCH_CHECK("relax_table_kernel");
  return BF_OK;
}

int relax_table_multi(int count, const float* const* lo, const float* const* hi, const float* const* alpha,
                      const int64_t* alpha_ld, int64_t D, const int64_t* K, float* const* out, hipStream_t stream) {
  for (int base = 0; base < count; base += RELAX_SEG_MAX) {
    TableSegs t;
    memset(&t, 0, sizeof(t));
    t.count = count - base < RELAX_SEG_MAX ? count - base : RELAX_SEG_MAX;
    int64_t blocks = 0;
    for (int q = 0; q < t.count; ++q) {
      const int j = base + q;
      t.lo[q] = lo[j];
      t.hi[q] = hi[j];
      t.alpha[q] = alpha[j];
      t.alpha_ld[q] = alpha_ld[j];
      t.K[q] = K[j];
      t.out[q] = reinterpret_cast<float4*>(out[j]);
      t.bstart[q] = blocks;
      blocks += ceil_div(D * K[j], 256);
    }
    t.bstart[t.count] = blocks;
    if (blocks == 0) continue;
    BF_REQUIRE(blocks < (1LL << 31), "relax_table_multi: too many entries");
    hipLaunchKernelGGL(relax_table_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, t, D);
    BF_LAUNCH_CHECK("relax_table_multi_kernel");
  }
  return BF_OK;
}

int gemm_partial_count(int64_t N) { return (int)ceil_div(N, NORM_BN); }

// Columns per partial norm of the |A W| epilogue: 64 (the 64 x 64 TileS, plain prologue)
// when the 64 x 128 tiles of one bound would leave more than half of the device's 256
// CUs idle -- a small batch, where a tile's whole K loop on one wave per SIMD is the
// launch's critical path -- else NORM_BN.
int gemm_norm_cols(int64_t M, int64_t N, int pro) {
  if (pro != PRO_PLAIN || N <= NORM_BN / 2) return NORM_BN;
  return ceil_div(M, (int64_t)64) * ceil_div(N, (int64_t)NORM_BN) < 128 ? NORM_BN / 2 : NORM_BN;
}

int gemm_norm_partial_count(int64_t M, int64_t N, int pro) { return (int)ceil_div(N, (int64_t)gemm_norm_cols(M, N, pro)); }

// Sums of the relaxation epilogue over the column tiles, in tile order:
//   b_out[m] = b_src[m] + sum_t pb[t][m]   (b_src NULL = 0; b_src may alias b_out)
//   c_out[m] = sum_t pc[t][m]              (when c_out)
__global__ void rows_finalize_kernel(const float* b_src, const float* __restrict__ pb, const float* __restrict__ pc,
                                     int nparts, int64_t M, float* b_out, float* __restrict__ c_out) {
  const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  float v = b_src ? b_src[m] : 0.f;
  for (int q = 0; q < nparts; ++q) v += pb[(int64_t)q * M + m];
  b_out[m] = v;
  if (c_out) {
    float c = 0.f;
    for (int q = 0; q < nparts; ++q) c += pc[(int64_t)q * M + m];
    c_out[m] = c;
  }
}

int rows_finalize(const float* b_src, const float* pb, const float* pc, int nparts, int64_t M, float* b_out,
                  float* c_out, hipStream_t stream) {
  if (M == 0) return BF_OK;
  hipLaunchKernelGGL(rows_finalize_kernel, dim3((unsigned)ceil_div(M, 256)), dim3(256), 0, stream, b_src, pb, pc,
                     nparts, M, b_out, c_out);
  BF_LAUNCH_CHECK("rows_finalize_kernel");
  return BF_OK;
}

// Sum of the split-K partial products in chunk order, plus the rank-1 term.
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int ks, int64_t M, int64_t N,
                                     float* __restrict__ C, int64_t ldc, const float* __restrict__ r_row,
                                     const float* __restrict__ v_col, int64_t v_ld, int64_t S) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * N) return;
  const int64_t m = div_rows(i, N, M * N < (1LL << 31)), n = i - m * N;
  const int64_t MN = M * N;
  float v = part[i];
  // the chunks' loads issued eight at a time, their sums still in chunk order
  int s = 1;
  for (; s + 8 <= ks; s += 8) {
    float t[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) t[q] = part[(int64_t)(s + q) * MN + i];
#pragma unroll
    for (int q = 0; q < 8; ++q) v += t[q];
  }
  for (; s < ks; ++s) v += part[(int64_t)s * MN + i];
  if (r_row) v = v + r_row[m] * v_col[div_rows(m, S, M < (1LL << 31)) * v_ld + n];
  C[m * ldc + n] = v;
}

// Split-K plan of a plain contraction: chunks of a multiple of 32 in k, used
// when the output has too few 128 x 128 tiles to fill the device.
int gemm_ksplit(int64_t M, int64_t N, int64_t K, int64_t* kchunk) {
  const int64_t tiles = ceil_div(M, 128) * ceil_div(N, 128);
  *kchunk = K;
  if (tiles >= 128 || K < 256) return 1;
  int64_t ks = ceil_div(512, tiles);
  if (ks > K / 64) ks = K / 64;
  if (ks > 64) ks = 64;
  if (ks < 2) return 1;
  *kchunk = ceil_div(ceil_div(K, ks), 32) * 32;
  return (int)ceil_div(K, *kchunk);
}

int splitk_reduce(const float* part, int ks, int64_t M, int64_t N, float* C, int64_t ldc, const float* r_row,
                  const float* v_col, int64_t v_ld, int64_t S, hipStream_t stream) {
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)ceil_div(M * N, 256)), dim3(256), 0, stream, part, ks, M, N,
                     C, ldc, r_row, v_col, v_ld, S);
  BF_LAUNCH_CHECK("splitk_reduce_kernel");
  return BF_OK;
}

}  // namespace bf
