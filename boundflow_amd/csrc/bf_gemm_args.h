// Argument block of the fp32 MFMA contraction kernel (see bf_gemm.hip).
#pragma once

#include "bf_common.h"

namespace bf {

enum : int { PRO_PLAIN = 0, PRO_RELAX = 1 };
enum : int { EPI_STORE = 0, EPI_ABSSUM = 1, EPI_RELAX = 2 };

struct GemmArgs {
  // Operand pair selected by blockIdx.z (z = 0 "upper", z = 1 "lower").
  const float* A[2];
  float* C[2];
  int64_t lda, ldc;
  int64_t lda_d;    // A row m = d*S + s lives at A + d*lda_d + s*lda (lda_d = S*lda when contiguous,
                    // 0 when every domain shares the same S rows)
  const float* B;   // [K, N] row-major (ldb) or, with trans_b, [N, K] row-major (ldb)
  int64_t ldb;
  int trans_b;
  int abs_b;        // bit z set: product z uses |B| (interval radius products)
  // Interval operand of the IBP products (plain prologue, register-staged loop): A[0] = A[1]
  // hold the lower bounds and ivl_hi the upper ones (same layout); product z = 0 reads the
  // center (l + u) / 2, z = 1 the radius (u - l) / 2, of max(l, 0) and max(u, 0) when ivl_relu.
  const float* ivl_hi;
  int ivl_relu;
  int64_t M, N, K;
  int z_lower_first;  // when 1, blockIdx.z = 0 uses lower semantics (single lower pass)

  // --- ReLU relaxation prologue (PRO_RELAX) ---
  int64_t S;                 // rows per domain
  const float4* relax;       // [D, K] {alpha_u, beta_u, alpha_l, beta_l}; null = identity (row sums only)
  const float* add_l;        // optional coefficient added to the lower A' (beta split term), row stride add_ld
  int64_t add_ld;
  const float* kbias;        // optional [K] bias of the affine layer: sum_k A'[m,k] * kbias[k]
  const float* cvec;         // optional [D, K] center vector: sum_k A'[m,k] * cvec[d,k]
  int64_t cvec_ld;
  const float* b_in[2];      // optional running bias [M]
  float* b_out[2];           // [M] = (b_in + sum A*beta_sel) + sum A'*kbias   (written by blockIdx.y == 0)
  float* c_out[2];           // [M] center sums (written by blockIdx.y == 0)

  // --- |C| row-reduction epilogue (EPI_ABSSUM) ---
  const float* wvec;         // optional [D, N] weights (box radius), row stride w_ld
  int64_t w_ld;
  float* partial[2];         // [gridDim.y, M] partial row sums
  const float* h_scale;      // optional [M]: lower pass also writes h = h_scale[m] * sign(C) * w  (gradient seed;
                             // with norm_kind 1 or 2 it writes C itself, turned into the seed afterwards)
  float* h_out;              // [M, N] row-major (ldh = N)
  int norm_kind;             // the row norm of C: 0 sum |C| (* w) (Linf ball, box); 1 max |C| (L1 ball);
                             // 2 sum C^2, the square root taken by the finalize (L2 ball)

  // --- relaxation epilogue (EPI_RELAX): the ReLU relaxation of the NEXT layer,
  // indexed by the output columns, applied to C before it is stored:
  //   C'[m, n] = C * slope_sel(d, n) (+ e_add[d, n] on the lower pass)
  //   partial[tile_n][m]   = sum over the tile's columns of (C * beta_sel + C' * e_kbias[n])
  //   partial_c[tile_n][m] = sum over the tile's columns of C' * e_cvec[d, n]   (optional)
  const float4* e_relax;     // [D, N] {alpha_u, beta_u, alpha_l, beta_l}
  const float* e_add;        // optional, lower pass only, row stride e_add_ld
  int64_t e_add_ld;
  const float* e_kbias;      // optional [N]
  const float* e_cvec;       // optional [D, N], row stride e_cvec_ld
  int64_t e_cvec_ld;
  float* partial_c[2];
  float* C_pre[2];           // optional: C before the relaxation (same layout as C)

  // --- rank-1 term of the store epilogue: C[m, n] = acc + r1_row[m] * r1_col[(m / S) * r1_ld + n] ---
  const float* r1_row;
  const float* r1_col;
  int64_t r1_ld;

  // --- split K (PRO_PLAIN, EPI_STORE, one operand pair): blockIdx.y = chunk index;
  // chunk s covers k in [s * kchunk, min(K, (s + 1) * kchunk)) and stores its
  // partial product to part + s * M * N (row-major, ld = N, no rank-1 term) ---
  int ksplit;
  int64_t kchunk;
  float* part;
};

}  // namespace bf
