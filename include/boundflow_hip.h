/* boundflow_hip.h -- C ABI of libboundflow_hip.so, the MI355X (gfx950) HIP
 * backend of the bound-propagation hot path.
 *
 * Conventions (all entry points):
 *  - pointers are device pointers (fp32 unless stated; int8 split masks,
 *    int32 flags); tensors are dense row-major;
 *  - "rows" are coefficient rows m = d * S + s (domain d, spec s), M = D * S;
 *    a per-domain vector of length n is addressed vec[d * ld + j] where
 *    ld = n (one per domain) or 0 (shared by all domains);
 *  - work is enqueued on `stream` (torch's current stream by default); no call
 *    synchronizes, allocates or frees -- callers pass outputs and workspaces;
 *  - every int-returning entry returns 0 on success and a nonzero status
 *    (1 invalid argument, 2 launch failure, 3 size limit) with a message from
 *    bf_last_error() (thread-local).  No C++ exception crosses the boundary.
 *
 * Each declaration cites the reference interface it replaces
 * (paths relative to the reference checkout's boundflow/ package).
 */
#ifndef BOUNDFLOW_HIP_H
#define BOUNDFLOW_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

int bf_abi_version(void);
const char* bf_last_error(void);

/* The contraction's tile configuration is chosen per call: 'G', 128 x 128 x 16
 * with 8 waves of 32 x 64 (3 workgroups per CU), for every form; 'H', 128 x 128 x
 * 32 with 16 waves of 32 x 32, when the grid has fewer 128 x 128 tiles (times
 * bounds and split-K chunks) than the device has CUs and the contraction has the
 * relaxation prologue or the |A W| or relaxation epilogue; 'S', 64 x 64 x 32 with
 * 4 waves (4 workgroups per CU), for such a grid with the plain prologue and the
 * store epilogue; 'Q', 64 x 128 x 16 with 4
 * waves (6 workgroups per CU), for a plain-prologue contraction on direct-to-LDS
 * operands (transposed B, 16-byte aligned float4 rows) whose 128 x 128 tiles
 * load the 256 CUs unevenly and whose 64 x 128 tiles load them at least 10
 * points more evenly.  The environment variable BOUNDFLOW_GEMM_TILE=G, =H, =Q or
 * =S, read once when the library is loaded, forces one for measurement ('Q' then
 * refuses other operands; 'S' takes the store epilogue alone, others fall back to 'Q'
 * on direct-to-LDS operands, else 'H').
 * bf_gemm_tile_config returns the configuration ('G', 'H', 'Q' or 'S') a
 * store-epilogue contraction of M x N outputs, nz bounds and ksplit K chunks would
 * take (0 for bad sizes); the other epilogues take 'Q' where it says 'S' when the
 * operands suit the direct-to-LDS loop, else 'H'.
 * No counterpart in the reference: introspection of this build's dispatch. */
int bf_gemm_tile_config(int64_t M, int64_t N, int nz, int ksplit, int relax_prologue, int dl_operands);

/* ---- kernel #1: IBP ---------------------------------------------------- */

/* Interval linear layer in center/radius form, with the consumer ReLU's split
 * applied and per-domain infeasibility flagged.
 * Replaces LpBallPerturbation/BoxPerturbation.concretize_matmul
 * (runtime/perturbation.py:102-173, 282-325) for the input layer and
 * IntervalDomain.affine_transformer (domains/interval.py:79-86) for hidden
 * layers, and _apply_relu_split (runtime/crown_ibp.py:70-98).
 * input_kind 0: [in_lo, in_hi] box (ReLU applied first when apply_relu);
 * input_kind 1: Linf ball of radius eps around in_lo; 2: L2 ball; 3: L1 ball
 * (eps times the dual norm of each W row: sum |w|, the L2 norm, max |w|).
 * workspace: bf_ibp_linear_workspace(B, K, N) floats.  center_out (optional,
 * [B, N]) receives mid @ W^T without bias.  box_radius_out (optional, [B, K],
 * box input without ReLU only) receives the input box radius (in_hi - in_lo) / 2,
 * the weights of the box concretization (perturbation.py:282-325), written from
 * the bounds the products load when the output is small. */
int bf_ibp_linear(const float* in_lo, const float* in_hi, int64_t B, int64_t K, int input_kind, float eps,
                  int apply_relu, const float* W, const float* bias, int64_t N, const int8_t* split,
                  int64_t split_ld, float* workspace, float* out_lo, float* out_hi, float* center_out,
                  int* infeasible, float* box_radius_out, hipStream_t stream);
int64_t bf_ibp_linear_workspace(int64_t B, int64_t K, int64_t N);

/* Interval conv2d (NCHW, groups 1, dilation 1) in center/radius form.
 * Replaces IntervalDomain.affine_transformer conv branch (domains/interval.py:57-74)
 * and the input bounding box of runtime/crown_ibp.py:167-181.
 * workspace: bf_ibp_conv2d_workspace(B, Ci*Hi*Wi, Co*Ho*Wo) floats. */
int bf_ibp_conv2d(const float* in_lo, const float* in_hi, int64_t B, int Ci, int Hi, int Wi, int input_kind,
                  float eps, int apply_relu, const float* W, const float* bias, int Co, int KH, int KW, int sh,
                  int sw, int ph, int pw, int Ho, int Wo, const int8_t* split, int64_t split_ld, float* workspace,
                  float* out_lo, float* out_hi, float* center_out, int* infeasible, hipStream_t stream);
int64_t bf_ibp_conv2d_workspace(int64_t B, int64_t nin, int64_t nout);

/* Intersection with external pre-activation constraints and a split
 * (runtime/crown_ibp.py:186-209), in place; flags infeasible domains. */
int bf_interval_clip(float* lo, float* hi, const float* clo, const float* chi, const int8_t* split,
                     int64_t split_ld, int64_t B, int64_t N, int* infeasible, hipStream_t stream);

/* Op-by-op interval kernels of the IBP task executor (runtime/task_executor.py:360-563):
 * relu (domains/interval.py:88-91), add, mul (four endpoint products, interval.py:102-112),
 * spec_linear (C+ l + C- u, :423-439) and the batched per-sample linear W [B, O, I] in
 * center/radius form (:445-458).  mul expects both operands already broadcast to n elements. */
int bf_interval_relu(const float* lo, const float* hi, int64_t n, float* out_lo, float* out_hi, hipStream_t stream);
/* Center (l + u) / 2 and radius (u - l) / 2 of an interval (of max(., 0) when apply_relu),
 * either output NULL to skip it: the center/radius form of IBP (domains/interval.py:57-86)
 * and the box radius of a concretization (runtime/perturbation.py:327-359, (upper - lower) / 2). */
int bf_interval_center_radius(const float* lo, const float* hi, int64_t n, int apply_relu, float* mid, float* rad,
                              hipStream_t stream);
int bf_interval_add(const float* a_lo, const float* a_hi, const float* b_lo, const float* b_hi, int64_t n,
                    float* out_lo, float* out_hi, hipStream_t stream);
int bf_interval_mul(const float* a_lo, const float* a_hi, const float* b_lo, const float* b_hi, int64_t n,
                    float* out_lo, float* out_hi, hipStream_t stream);
int bf_spec_linear(const float* C, const float* lo, const float* hi, int64_t B, int64_t S, int64_t O, float* out_lo,
                   float* out_hi, hipStream_t stream);
int bf_ibp_batched_linear(const float* lo, const float* hi, int64_t B, int64_t I, const float* W, const float* bias,
                          int64_t O, float* out_lo, float* out_hi, hipStream_t stream);

/* ---- kernels #2 + #3: CROWN backward, fused ReLU relaxation + contraction -- */

/* Slopes/intercepts of the ReLU relaxation per (domain, neuron), as the
 * interleaved table {alpha_u, beta_u, alpha_l, beta_l} [D, K, 4] (16-byte
 * aligned) -- the four tensors of FusedReluAffineRequest
 * (runtime/fused_crown.py:33-48) computed by _relu_backward_relaxation
 * (runtime/crown_ibp.py:722-758, 1176-1208).  alpha: optional lower-slope
 * override [D,K] (alpha_ld K) or shared (alpha_ld 0), clamped to [0,1] and used
 * on ambiguous neurons only. */
int bf_relu_relax_table(const float* pre_lo, const float* pre_hi, const float* alpha, int64_t alpha_ld, int64_t D,
                        int64_t K, float* table, hipStream_t stream);

/* The tables of count ReLUs in one launch (host arrays of device pointers, alpha rows and
 * widths; one domain count D): table j is bf_relu_relax_table(pre_lo[j], pre_hi[j],
 * alpha[j], alpha_ld[j], D, K[j], table[j]) element for element.  Same boundary as
 * bf_relu_relax_table (crown_ibp.py:722-758, 1176-1208), for a backward pass that reads
 * several layers' tables. */
int bf_relu_relax_table_multi(int count, const float* const* pre_lo, const float* const* pre_hi,
                              const float* const* alpha, const int64_t* alpha_ld, int64_t D, const int64_t* K,
                              float* const* table, hipStream_t stream);

/* The same table from the four separate tensors of a FusedReluAffineRequest
 * (runtime/fused_crown.py:33-48: alpha_u, beta_u, alpha_l, beta_l, each n =
 * D*K floats), interleaved in one pass: what HipFusedCrownExecutor hands the
 * contraction of a "fused_relu_linear" region (run, :97-123). */
int bf_relu_relax_table_from_planes(const float* alpha_u, const float* beta_u, const float* alpha_l,
                                    const float* beta_l, int64_t n, float* table, hipStream_t stream);

/* One ReLU -> Linear region: A' = relax(A) (upper: sel(A>=0, alpha_u, alpha_l),
 * lower mirrored, plus the optional beta split coefficient add_l on the lower
 * bound), A_prev = A' @ W on fp32 MFMA, and
 * b_out = (b_in + sum_k A * beta_sel) + sum_k A' * bias.
 * Replaces FusedCrownExecutor.run for "fused_relu_linear"
 * (runtime/fused_crown.py:97-123, reference equations :330-400) and the dense
 * ReLU step + linear step of runtime/crown_ibp.py:1073-1090, 1211-1298.
 * A rows: A + d*a_dstride + s*N (a_dstride = S*N, or 0 when every domain
 * shares the same S rows).  relax: table of bf_relu_relax_table, NULL = no
 * relaxation (identity).  Either bound may be NULL (input and output together).
 * W: the layer weight [N, P] row-major (the reference's [out, in]) when
 * w_trans = 0, or its transpose [P, N] row-major when w_trans = 1 (the faster
 * operand layout: 128-bit loads along the contraction). */
int bf_crown_relu_linear_fwd(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t N,
                             const float* relax, const float* add_l, int64_t add_ld, const float* W, int64_t P,
                             int w_trans, const float* bias, const float* b_u_in, const float* b_l_in,
                             float* A_prev_u, float* A_prev_l, float* b_u_out, float* b_l_out, hipStream_t stream);

/* The input-layer region fused with the concretization (kernel #4):
 * lb = (A' . cvec - eps * sum_i |(A' W)_i| * rad_i) + b, ub mirrored;
 * rad NULL = Lp ball (weights 1, eps used), else box radius [D, I] (eps ignored).
 * norm_p selects the dual norm of the ball's row term: 0 sum |.| (Linf ball or
 * box), 2 the L2 norm (L2 ball), 1 max |.| (L1 ball); 1 and 2 take no rad, and
 * their gradient seed is h = h_scale[m] * d norm / d(A'W) (A'W / |A'W|_2, or
 * sign / ties on the maxima of |A'W|), made after the row's norm is known.
 * cvec = center @ W^T per domain [D, N].  Replaces concretize_affine
 * (runtime/perturbation.py:175-222, 327-359) on RightMatmulLinearOperator
 * (runtime/linear_operator.py:503-586) as called at runtime/crown_ibp.py:2044-2051.
 * h_scale/h_out (optional, lower bound only): h = h_scale[m] * sign(A'W) * rad,
 * the gradient seed of the concretization.  W / w_trans as for bf_crown_relu_linear_fwd.
 * workspace: bf_crown_relu_linear_concretize_workspace(D, S, I) floats. */
int bf_crown_relu_linear_concretize(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S,
                                    int64_t N, const float* relax, const float* add_l, int64_t add_ld, const float* W,
                                    int64_t I, int w_trans,
                                    const float* bias, const float* cvec, const float* rad, float eps, int norm_p,
                                    const float* b_u_in, const float* b_l_in, const float* h_scale, float* h_out,
                                    float* workspace, float* lb, float* ub, hipStream_t stream);
int64_t bf_crown_relu_linear_concretize_workspace(int64_t D, int64_t S, int64_t I);

/* bf_crown_relu_linear_concretize without the workspace argument: no counterpart in
 * the reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops or harnesses that forbid hipMalloc); it allocates
 * nothing.  Its workspace is a fixed 16 MiB device array per GPU (4M floats, held
 * until the process ends): returns 3 (size beyond the limit) when
 * bf_crown_relu_linear_concretize_workspace(D, S, I) exceeds 4194304 floats (e.g.
 * D * S > 233016 rows at I = 784).  norm_p as for bf_crown_relu_linear_concretize.  Calls that overlap on one GPU share that array
 * and race: serialise them.  Same results as bf_crown_relu_linear_concretize. */
int bf_crown_relu_linear_concretize_noalloc(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D,
                                            int64_t S, int64_t N, const float* relax, const float* add_l,
                                            int64_t add_ld, const float* W, int64_t I, int w_trans, const float* bias,
                                            const float* cvec, const float* rad, float eps, int norm_p, const float* b_u_in,
                                            const float* b_l_in, const float* h_scale, float* h_out, float* lb,
                                            float* ub, hipStream_t stream);

/* Two consecutive regions of the CROWN backward of an MLP in one launch: the
 * ReLU -> Linear region of bf_crown_relu_linear_fwd (prologue relaxation with
 * relax / add_l / bias; when all three are NULL, A is taken as already relaxed)
 * and the relaxation of the NEXT ReLU applied to the product before it is
 * stored:
 *   A_next = relax_next(A'' W^T) (+ add_next on the lower bound),
 *   b_out  = b_in [+ prologue sums] + sum_n (C * beta_sel + A_next * bias_next),
 *   c_out  = sum_n A_next * cvec_next   (only when cvec_next; row stride cvec_next_ld),
 * so the next region reads A_next as it is (relax, add_l and bias NULL) and the
 * input region can be concretized with bf_crown_linear_concretize.  A_pre_u /
 * A_pre_l (optional) receive the product before that relaxation (the
 * coefficient the alpha/beta gradient pass reads).  The same
 * steps as runtime/crown_ibp.py:1073-1090, 1211-1298 applied to two
 * consecutive layers (the reference's dense backward loop, crown_ibp.py:1371-1700).
 * W_t: the layer weight transposed, [P, N] row-major.  relax_next: table of
 * bf_relu_relax_table over the P columns ([D, P]).  Rows of one 128-row tile
 * spanning more than its LDS stage holds (10 domains with a relaxation prologue
 * and S >= 15, else 18) read the tables from global memory.  A short contraction
 * (N <= 16, e.g. the spec rows times the output layer) with no prologue table or
 * split term runs on the VALU instead of the tiled MFMA kernel (P % 4 == 0,
 * 16-byte aligned outputs).
 * workspace: bf_crown_relu_linear_relu_fwd_workspace(D, S, P) floats. */
int bf_crown_relu_linear_relu_fwd(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S,
                                  int64_t N, const float* relax, const float* add_l, int64_t add_ld,
                                  const float* W_t, int64_t P, const float* bias, const float* b_u_in,
                                  const float* b_l_in, const float* relax_next, const float* add_next,
                                  int64_t add_next_ld, const float* bias_next, const float* cvec_next,
                                  int64_t cvec_next_ld, float* workspace, float* A_next_u, float* A_next_l,
                                  float* A_pre_u, float* A_pre_l, float* b_u_out, float* b_l_out, float* c_u_out,
                                  float* c_l_out, hipStream_t stream);
int64_t bf_crown_relu_linear_relu_fwd_workspace(int64_t D, int64_t S, int64_t P);

/* Lp-ball / box concretization of an input layer whose coefficient is already
 * relaxed (the output of bf_crown_relu_linear_relu_fwd):
 *   lb = (cen_l - eps * sum_i |(A_l W^T)_i| * rad_i) + b_l, ub mirrored,
 * with the center and bias sums given per row; norm_p (0, 1, 2) swaps the
 * row sum for the ball's dual norm as in bf_crown_relu_linear_concretize.  concretize_affine
 * (runtime/perturbation.py:175-222, 327-359) as called at crown_ibp.py:2044-2051.
 * h_scale/h_out (optional, lower bound only): the gradient seed
 * h = h_scale[m] * sign(A_l W^T) * rad, as in bf_crown_relu_linear_concretize.
 * workspace: bf_crown_linear_concretize_workspace(D, S, I) floats. */
int bf_crown_linear_concretize(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S,
                               int64_t N, const float* W_t, int64_t I, const float* rad, float eps, int norm_p,
                               const float* cen_u, const float* cen_l, const float* b_u, const float* b_l,
                               const float* h_scale, float* h_out, float* workspace, float* lb, float* ub,
                               hipStream_t stream);
int64_t bf_crown_linear_concretize_workspace(int64_t D, int64_t S, int64_t I);

/* Standalone relaxation pass (bandwidth-bound form of kernel #3): writes A'
 * [D*S, K] and the bias/center row sums.  Replaces
 * _backprop_relu_step_dense_reference (runtime/crown_ibp.py:1211-1298); used
 * ahead of the conv transposed contraction, and to materialize per domain the
 * relaxation of a coefficient shared by all domains.  A rows: A + d*a_dstride +
 * s*K (a_dstride = S*K, or 0 when every domain shares the same S rows).  relax:
 * table of bf_relu_relax_table (NULL = identity); kbias: per-element bias of the
 * affine layer [K]; cvec: center projection [D, K] (optional). */
int bf_crown_relu_relax(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t K,
                        const float* relax, const float* add_l, int64_t add_ld, const float* kbias, const float* cvec,
                        const float* b_u_in, const float* b_l_in, float* A_u_out, float* A_l_out, float* b_u_out,
                        float* b_l_out, float* c_u_out, float* c_l_out, hipStream_t stream);

/* The same pass with the slopes and intercepts computed in place from the
 * pre-activation box (pre_lo, pre_hi [D,K]; both NULL = identity) and the
 * optional lower-slope override alpha ([D,K] with alpha_ld K, or shared with
 * alpha_ld 0), by the arithmetic of bf_relu_relax_table
 * (runtime/crown_ibp.py:722-758, 1176-1298): no table is built or read. */
int bf_crown_relu_relax_lu(const float* A_u, const float* A_l, int64_t a_dstride, int64_t D, int64_t S, int64_t K,
                           const float* pre_lo, const float* pre_hi, const float* alpha, int64_t alpha_ld,
                           const float* add_l, int64_t add_ld, const float* kbias, const float* cvec,
                           const float* b_u_in, const float* b_l_in, float* A_u_out, float* A_l_out, float* b_u_out,
                           float* b_l_out, float* c_u_out, float* c_l_out, hipStream_t stream);

/* Transposed convolution of coefficient rows (Conv2dLinearOperator.to_dense,
 * runtime/linear_operator.py:1067-1092; FusedCrownExecutor "fused_relu_conv2d"
 * after bf_crown_relu_relax).  With norm_u/norm_l instead of y_u/y_l the
 * output rows are reduced to sum |y| (* wvec[d, e]) -- the concretization norm
 * of the input layer (linear_operator.py:1378-1452 + perturbation.py:175-222).
 * norm_p 2 reduces to sum y^2 (L2 ball), 1 to max |y| (L1 ball; Conv2dLinearOperator
 * row_l2_norm / row_abs_max, linear_operator.py:991-997), both without wvec;
 * bf_concretize_finalize with the same norm_p turns them into bounds.  Their
 * gradient seed h_out (y_l NULL) is h_scale[r] * d norm / dy, as for
 * bf_crown_relu_linear_concretize. */
int bf_conv_transpose_rows(const float* A_u, const float* A_l, int64_t R, int Co, int Ho, int Wo, const float* W,
                           int Ci, int KH, int KW, int sh, int sw, int ph, int pw, int Hi, int Wi, float* y_u,
                           float* y_l, int64_t S, const float* wvec, int64_t w_ld, int norm_p, float* norm_u,
                           float* norm_l, const float* h_scale, float* h_out, hipStream_t stream);

/* 1 when bf_crown_relu_conv_transpose (and the channel-last path of
 * bf_conv_transpose_rows) takes this conv shape: KH % sh == KW % sw == 0, Co a
 * multiple of 16, the staged map and weights within 64 KB of LDS; else 0. */
int bf_conv_transpose_hwc_supported(int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw, int ph, int pw,
                                    int Hi, int Wi);

/* One ReLU -> Conv2d region of the CROWN backward in one pass: the ReLU
 * relaxation of the coefficient rows A [D*S, Co*Ho*Wo] (slopes from the
 * pre-activation box pre_lo/pre_hi [D, Co*Ho*Wo] and the optional lower-slope
 * override alpha, as bf_crown_relu_relax_lu; the split term add_l on the lower
 * bound) applied while each row's map is staged, never written unless
 * relaxed_u/relaxed_l are given, then the transposed convolution to
 * y [D*S, Ci*Hi*Wi], with b_out = (b_in + sum A * beta_sel) + sum A' * kbias.
 * Replaces bf_crown_relu_relax_lu followed by bf_conv_transpose_rows: the
 * sign-split transform of SignSplitLinearOperator (runtime/linear_operator.py:722-905)
 * taken lazily into the conv operator (Conv2dLinearOperator.to_dense,
 * linear_operator.py:1067-1092), with the dense ReLU backward's bias terms
 * (runtime/crown_ibp.py:1211-1298).  Returns 1 for a shape that
 * bf_conv_transpose_hwc_supported rejects.  w_packed (optional): the weights
 * packed by bf_conv_transpose_pack_weights. */
int bf_crown_relu_conv_transpose(const float* A_u, const float* A_l, int64_t D, int64_t S, int Co, int Ho, int Wo,
                                 const float* pre_lo, const float* pre_hi, const float* alpha, int64_t alpha_ld,
                                 const float* add_l, int64_t add_ld, const float* kbias, const float* b_u_in,
                                 const float* b_l_in, const float* W, const float* w_packed, int Ci, int KH, int KW,
                                 int sh, int sw, int ph, int pw, int Hi, int Wi, float* y_u, float* y_l,
                                 float* b_u_out, float* b_l_out, float* relaxed_u, float* relaxed_l,
                                 hipStream_t stream);

/* One "fused_relu_conv2d" region of FusedCrownExecutor.run
 * (runtime/fused_crown.py:97-123; the reference's fused TVM kernel,
 * backends/tvm/fused_crown_conv2d.py:161-350) in one pass: the relaxation is
 * the request's four tensors alpha_u, beta_u, alpha_l, beta_l [D, Co*Ho*Wo]
 * read directly (no box, no split term), applied while each row's map is
 * staged as in bf_crown_relu_conv_transpose, then the transposed convolution
 * and b_out = (b_in + sum A * beta_sel) + sum A' * kbias.  Shapes: those of
 * bf_conv_transpose_hwc_supported (else returns 1); an input-layer shape (at
 * most 16 map channels of at most 256 pixels, at most 3 output channels of at
 * most 1024 pixels, at most 2 x 2 taps per output pixel) runs the tap-product
 * kernel in its register form instead. */
int bf_crown_relu_planes_conv_transpose(const float* A_u, const float* A_l, int64_t D, int64_t S, int Co, int Ho,
                                        int Wo, const float* alpha_u, const float* beta_u, const float* alpha_l,
                                        const float* beta_l, const float* kbias, const float* b_u_in,
                                        const float* b_l_in, const float* W, const float* w_packed, int Ci, int KH,
                                        int KW, int sh, int sw, int ph, int pw, int Hi, int Wi, float* y_u,
                                        float* y_l, float* b_u_out, float* b_l_out, hipStream_t stream);

/* The input layer of a conv network in one pass: the ReLU relaxation of
 * bf_crown_relu_relax_lu applied to each coefficient row as it is staged (with
 * b_out = (b_in + sum A * beta_sel) + sum A' * kbias and c_out = sum A' * cvec[d]),
 * then the transposed convolution reduced to the concretization norm
 * norm[r] = sum |y| (* wvec[d, e]) and, with h_scale, the lower bound's gradient
 * seed h_out = h_scale[r] * sign(y) (* wvec) -- bf_conv_transpose_rows with norm
 * outputs on the relaxed rows, never writing them unless relaxed_u/relaxed_l are
 * given.  Replaces bf_crown_relu_relax_lu followed by bf_conv_transpose_rows for
 * the input region (runtime/crown_ibp.py:1211-1298 then the input-layer
 * concretization of Conv2dLinearOperator, runtime/linear_operator.py:1378-1452
 * and runtime/perturbation.py:175-222).  norm_p as for bf_conv_transpose_rows.
 * Shapes: those bf_conv_transpose_small_supported accepts (<= 4 input channels,
 * <= 16 taps).  lb / ub (optional, [D*S]; each needs its coefficient and its
 * norm, bias and center outputs): the bounds (c -/+ eps * norm) + b of
 * bf_concretize_finalize with one partial norm, written by the launch itself
 * where the register form runs (else by one finalize launch). */
int bf_conv_transpose_small_supported(int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw, int ph,
                                      int pw, int Hi, int Wi);
int bf_crown_relu_conv_transpose_concretize(const float* A_u, const float* A_l, int64_t D, int64_t S, int Co, int Ho,
                                            int Wo, const float* pre_lo, const float* pre_hi, const float* alpha,
                                            int64_t alpha_ld, const float* add_l, int64_t add_ld, const float* kbias,
                                            const float* cvec, const float* b_u_in, const float* b_l_in,
                                            const float* W, int Ci, int KH, int KW, int sh, int sw, int ph, int pw,
                                            int Hi, int Wi, const float* wvec, int64_t w_ld, int norm_p,
                                            const float* h_scale, float* h_out, float* norm_u, float* norm_l,
                                            float* b_u_out, float* b_l_out, float* c_u_out, float* c_l_out,
                                            float* relaxed_u, float* relaxed_l, float eps, float* lb, float* ub,
                                            hipStream_t stream);

/* The weights of that pass in the order its workgroups stage them
 * (bf_conv_transpose_packed_floats floats, 16-byte aligned; 0 = shape not
 * taken), so that a caller who keeps them per weight tensor passes them as
 * w_packed and each workgroup copies them instead of gathering from W. */
int64_t bf_conv_transpose_packed_floats(int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw, int ph,
                                        int pw, int Hi, int Wi);
int bf_conv_transpose_pack_weights(const float* W, int Co, int Ho, int Wo, int Ci, int KH, int KW, int sh, int sw,
                                   int ph, int pw, int Hi, int Wi, float* out, hipStream_t stream);

/* Convolution of rows (IBP center/radius, center projection x0 conv W, and the
 * gradient of a transposed convolution), plus optional rank-1 term
 * y[r] += row_scale[r] * vec[(r / vec_div) * vec_ld + e]. */
int bf_conv2d_rows(const float* x, int64_t in_div, int64_t R, int Ci, int Hi, int Wi, const float* W, int abs_w,
                   int Co, int KH, int KW, int sh, int sw, int ph, int pw, int Ho, int Wo, float* y,
                   const float* row_scale, const float* vec, int64_t vec_div, int64_t vec_ld, hipStream_t stream);

/* Plain fp32 MFMA contraction C = A @ op(B) (op = transpose when trans_b,
 * |.| when abs_b): the lazy A @ W of RightMatmulLinearOperator.to_dense
 * (runtime/linear_operator.py:585-586). */
int bf_gemm(const float* A, int64_t lda, const float* B, int64_t ldb, int trans_b, int abs_b, float* C, int64_t ldc,
            int64_t M, int64_t N, int64_t K, hipStream_t stream);

/* Contraction with a rank-1 epilogue C[m,n] = (A @ op(B))[m,n] + r_row[m] * v_col[(m/S)*v_ld + n]:
 * the transposed contraction of the gradient pass with the bias terms.  When
 * the output is too small to fill the device, K is split into chunks whose
 * partial products go to the workspace (bf_gemm_rank1_workspace floats; 0 =
 * no split for this shape) and are summed in chunk order; with a NULL or too
 * small workspace the contraction runs unsplit. */
int bf_gemm_rank1(const float* A, int64_t lda, const float* B, int64_t ldb, int trans_b, float* C, int64_t ldc,
                  int64_t M, int64_t N, int64_t K, int64_t S, const float* r_row, const float* v_col, int64_t v_ld,
                  float* workspace, int64_t workspace_floats, hipStream_t stream);
int64_t bf_gemm_rank1_workspace(int64_t M, int64_t N, int64_t K);

/* ---- kernel #4: concretization -------------------------------------------- */

/* Dense coefficient rows A [M, I] against the input set:
 * out = A . center[d] -/+ eps * sum |A| (Linf, rad NULL) or -/+ sum |A| * rad[d] (box), + b;
 * norm_p 2 / 1 (rad NULL): eps times the row's L2 norm / max |A| (L2 / L1 ball).
 * Replaces LpBallPerturbation/BoxPerturbation.concretize_affine on a
 * DenseLinearOperator (runtime/perturbation.py:175-222, 327-359;
 * runtime/linear_operator.py:354-372).  is_lower selects the sign. */
int bf_concretize_dense(const float* A, int64_t D, int64_t S, int64_t I, const float* center, const float* rad,
                        float eps, int norm_p, const float* b, int is_lower, float* out, hipStream_t stream);

/* lb = (cen_l - eps * sum_q partial_l[q]) + b_l (ub mirrored), fixed-order sum over nparts;
 * norm_p 1: max over the parts (partials of max |.|), 2: sqrt of their sum
 * (partials of sum of squares), 0: their sum. */
int bf_concretize_finalize(const float* partial_u, const float* partial_l, int nparts, int64_t M,
                           const float* cen_u, const float* cen_l, const float* b_u, const float* b_l, float eps, int norm_p,
                           float* lb, float* ub, hipStream_t stream);

/* ---- kernel #5: alpha / beta gradients and the optimiser ------------------ */

/* Reverse pass through one ReLU relaxation of the lower bound: g_in = dL/dA,
 * g_alpha = dL/dalpha [D,N], g_beta = dL/dbeta [D,N] (see bf_grad.hip).
 * Replaces the autograd backward of runtime/crown_ibp.py:1211-1298 driven by
 * runtime/alpha_beta_crown.py:913-923 / runtime/alpha_crown.py:236-246. */
int bf_relu_grad(const float* g_out, const float* A, int64_t a_dstride, int64_t D, int64_t S, int64_t N,
                 const float* pre_lo, const float* pre_hi, const float* alpha, int64_t alpha_ld, const float* G,
                 const int8_t* split, int64_t split_ld, float* g_in, float* g_alpha, float* g_beta,
                 hipStream_t stream);

/* out[d, n] = max over the S rows of domain d of max(|A_u[d*S+s, n]|, |A_l[d*S+s, n]|)
 * for the dense coefficient rows [D*S, N] of the two bounds (either may be NULL):
 * the per-ReLU objective influence of
 * run_crown_ibp_mlp_with_relu_influence_from_forward_trace (runtime/crown_ibp.py:1810-1833,
 * 2201-2241). */
int bf_rows_abs_max(const float* A_u, const float* A_l, int64_t D, int64_t S, int64_t N, float* out,
                    hipStream_t stream);

/* dL/dA of the dense concretization of the lower bound (bf_concretize_dense, is_lower = 1):
 * g[m, j] = G[m] * center[d, j] + (G[m] * -w[d, j]) * sign(A[m, j]), w = eps (rad NULL) or rad [D, I];
 * norm_p 2 / 1 (rad NULL): G[m] * center[d, j] - eps * G[m] * d|A[m]|_q / dA[m, j] with the L2 norm's
 * A / |A|_2 (0 for a zero row) or max |A|'s sign(A) / ties on the maxima, as autograd forms them;
 * the autograd backward of concretize_affine (runtime/perturbation.py:175-222, 327-359) at the input of a
 * DAG task, driven by runtime/alpha_beta_crown.py:913-923. */
int bf_concretize_dense_grad(const float* A, int64_t D, int64_t S, int64_t I, const float* center, const float* rad,
                             float eps, int norm_p, const float* G, float* g, hipStream_t stream);

/* out[m, n] = (a[m, n] + b[m, n]) + r_row[m] * vec[(m / S) * v_ld + n], every term optional (NULL), out may
 * alias a or b: the fan-in accumulation of backward states (runtime/crown_ibp.py:892-909, A_cur.add(A_upd))
 * and, in the reverse pass of a DAG task, the sum of an add's operand gradients with the rank-1 term of a
 * constant operand (runtime/crown_ibp.py:1928-1970). */
int bf_rows_add(const float* a, const float* b, int64_t M, int64_t N, int64_t S, const float* r_row, const float* vec,
                int64_t v_ld, float* out, hipStream_t stream);

/* beta split coefficient add = -beta * s * 1(s != 0) (runtime/alpha_beta_crown.py:615-640). */
int bf_beta_coeff(const float* beta, int64_t beta_ld, const int8_t* split, int64_t split_ld, int64_t D, int64_t N,
                  float* out, hipStream_t stream);
/* The same for `count` ReLUs in one launch (host arrays of device pointers and sizes; D rows each). */
int bf_beta_coeff_multi(int count, const float* const* beta, const int64_t* beta_ld, const int8_t* const* split,
                        const int64_t* split_ld, const int64_t* ncol, int64_t D, float* const* out,
                        hipStream_t stream);

/* torch.optim.Adam step (no weight decay / amsgrad) then clamp to [lo, hi]
 * (hi only when has_clamp_hi), in place (runtime/alpha_beta_crown.py:747, 918-923).
 * At step 1 the moments start at zero, as torch.optim.Adam's fresh state does: m and v
 * are written, not read (they need no clearing before the first step). */
int bf_adam_clamp_step(float* p, float* m, float* v, const float* g, int64_t n, double lr, double beta1,
                       double beta2, float eps, int step, float clamp_lo, float clamp_hi, int has_clamp_hi,
                       hipStream_t stream);
/* The same step for `count` parameter tensors in one launch (one optimizer over all of them, as the
 * reference's single torch.optim.Adam over every alpha and beta; host arrays of device pointers, sizes
 * and per-tensor clamps).  best (optional host array of device pointers): each tensor, taken as `rows`
 * rows, is first copied to best[k] on the rows where improved[row] != 0 -- the best-of copy of
 * bf_masked_copy_rows_multi (alpha_beta_crown.py:840-876) taken from the values the step then updates. */
int bf_adam_clamp_multi(int count, float* const* p, float* const* m, float* const* v, const float* const* g,
                        const int64_t* n, const float* clamp_lo, const float* clamp_hi, const int* has_clamp_hi,
                        double lr, double beta1, double beta2, float eps, int step, float* const* best,
                        const int* improved, int64_t rows, hipStream_t stream);

/* Per-domain best-of tracking on mean_s lb (runtime/alpha_beta_crown.py:840-876).  ub and best_ub may
 * both be NULL: the lower bounds alone are tracked (the caller then evaluates the upper bound once, with
 * the best parameters). */
int bf_best_update(const float* lb, const float* ub, int64_t D, int64_t S, float* best_metric, float* best_lb,
                   float* best_ub, int* improved, int first, hipStream_t stream);
int bf_masked_copy_rows(float* dst, const float* src, int64_t D, int64_t N, const int* mask, hipStream_t stream);
/* The best-of copy for `count` parameter tensors of D rows in one launch (host arrays). */
int bf_masked_copy_rows_multi(int count, float* const* dst, const float* const* src, const int64_t* ncol, int64_t D,
                              const int* mask, hipStream_t stream);

/* out[n] = sum_d x[d, n] (gradient of a parameter shared by all domains). */
int bf_sum_rows(const float* x, int64_t D, int64_t N, float* out, hipStream_t stream);

/* "alpha from CROWN" init (runtime/native_alpha_beta_optimizer_schedule.py:635-653). */
int bf_alpha_from_crown(const float* lo, const float* hi, int64_t n, float* out, hipStream_t stream);

/* The ADAPTIVE lower slope of the native plain-CROWN relaxation
 * (runtime/bound_ir_interpreter.py:1380-1397), the node bound of the native
 * ReLU-split queue: 1 on an ambiguous neuron whose upper chord slope
 * u / max(u - l, eps) exceeds 0.5, 1 on stable-active, else 0. */
int bf_alpha_adaptive(const float* lo, const float* hi, int64_t n, float* out, hipStream_t stream);

/* Optimisation objective of one step (runtime/alpha_beta_crown.py:787-815): per domain
 * the metric of `objective` (0 lower: R_min(lb); 1 upper: -R_max(ub); 2 gap:
 * -R_max(ub - lb); 3 both: w_lb R_min(lb) - w_ub R_max(ub)) with the spec reduction
 * `reduce` (0 mean, 1 min/max, 2 softmin/softmax with temperature tau), from lb [D, S]
 * (lower bound of C) and nub [D, S] (lower bound of -C, i.e. -ub); G_l = dL/dlb and
 * G_nu = dL/dnub (optional) for L = g_scale * sum_d metric_d; and with best_metric the
 * per-domain best-of update of the metric, best_lb and best_ub (optional) with the
 * improved flags.  S <= 64. */
int bf_objective_step(const float* lb, const float* nub, int64_t D, int64_t S, int objective, int reduce, float tau,
                      float w_lb, float w_ub, float g_scale, float* metric, float* G_l, float* G_nu,
                      float* best_metric, float* best_lb, float* best_ub, int* improved, int first,
                      hipStream_t stream);

/* x[m, :] *= scale[m], in place (row weights applied to a gradient seed). */
int bf_scale_rows(float* x, int64_t M, int64_t N, const float* scale, hipStream_t stream);

/* ---- BaB decisions ----------------------------------------------------------- */

/* Branching rule update for one ReLU layer (runtime/alpha_beta_crown.py:145-182):
 * widest ambiguous neuron, first index on ties, strictly wider to replace. */
int bf_branch_update(const float* lo, const float* hi, int64_t D, int64_t N, int layer, float* best_gap,
                     int* best_layer, int* best_idx, hipStream_t stream);

/* Branching rule of the native ReLU-split queue for one layer
 * (_select_branch, runtime/native_relu_split_bab_runtime.py:1015-1049): per domain the
 * widest unsplit (split == 0) ambiguous neuron, width u - l in double, first index on
 * ties; replaces best_* (width, layer, index, its l and u) only when strictly wider.
 * Call per layer in sorted-name order, best_width starting at -1. */
int bf_branch_update_native(const float* lo, const float* hi, const int8_t* split, int64_t split_ld, int64_t D,
                            int64_t N, int layer, double* best_width, int* best_layer, int* best_idx, float* best_lo,
                            float* best_hi, hipStream_t stream);

/* First-layer split infeasibility certificate, one node per workgroup
 * (_is_infeasible_split_first_layer_convex_combo, runtime/alpha_beta_crown.py:391-532;
 * halfspaces as _collect_first_layer_split_halfspaces, :259-389).  Node g's halfspaces
 * are s * (rows[i] . x + bias[i]) >= 0 for its nonzero split[g * split_ld + i] (in i
 * order); the input set is the Lp ball (center row g, eps; norm_p 0 Linf, 2 L2,
 * 1 L1) or, with rad, the box center +- rad (norm_p 0).  Searches a convex combination w = softmax(z) by Adam on z (lr,
 * betas 0.9/0.999, eps 1e-8, `steps` steps from z = 0) and sets out[g] = 1 at the
 * first step whose maximum over the set is below -tol, else 0; -1 when a node has
 * more than 1024 splits.  max_out (optional, [nodes]) receives the smallest maximum
 * the search saw (the certificate's value when out is 1; 0 for a node with no split
 * or too many).  in_dim <= 16384, steps <= 256. */
int bf_split_certificate(const float* rows, int64_t row_ld, const float* bias, const int8_t* split, int64_t split_ld,
                         const float* center, int64_t center_ld, const float* rad, int64_t rad_ld, float eps,
                         int norm_p, int64_t nodes, int64_t n0, int64_t in_dim, int steps, double lr, double tol,
                         int32_t* out, float* max_out, hipStream_t stream);

/* Node verdict (runtime/bab.py:870-895): 1 certified (min_s lb >= threshold - tol),
 * 2 infeasible split, 0 open. */
int bf_domain_status(const float* lb, int64_t D, int64_t S, const int* infeasible, float threshold, float tol,
                     int* status, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BOUNDFLOW_HIP_H */
