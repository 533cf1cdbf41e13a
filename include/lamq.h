/*
 * lamq.h -- C ABI of the MI355X (gfx950) per-matrix quantization hot path.
 *
 * Every entry point takes caller-owned device pointers with explicit leading dimensions
 * (in elements) and a hipStream_t (passed as void*), enqueues its kernels on that stream and
 * returns an int status:
 *     0                 success
 *     LAMQ_EINVAL (-1)  an argument is out of range or a pointer is NULL (nothing was launched)
 *     LAMQ_EUNSUP (-2)  a shape or parameter this build does not support (nothing was launched)
 *     > 0               the hipError_t of a failed launch
 * Results that depend on the data (a pivot that is not positive, an invalid trellis path) are
 * reported through device-side outputs named in each declaration. Nothing here allocates device
 * memory; entry points that need scratch take a workspace whose size a *_workspace_size query
 * returns. No entry point keeps state between calls, and calls on distinct streams with
 * distinct buffers are independent.
 *
 * Data types: bf16 is passed as uint16_t bit patterns; fp64 as double; fp32 as float.
 * Matrices are row-major.
 */
#ifndef LAMQ_H
#define LAMQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LAMQ_OK 0
#define LAMQ_EINVAL (-1)
#define LAMQ_EUNSUP (-2)

/* Version of this ABI (major * 100 + minor). */
int lamq_abi_version(void);

/* ------------------------------------------------------------------------------------------------
 * Viterbi over a bitshift trellis, one path per row.
 * Replaces opgraph/codes.py:151-181 viterbi(X, values, L, k, chunk=None, start=None).
 *   x       [B, T] float32 targets (row stride ldx); the reference casts its float64 inputs to float32
 *   C       [2^L] float32 state values
 *   start   NULL (first state free) or [B] int32 previous states (codes.py:165-167)
 *   states  [B, T] int32 output (row stride lds)
 * Ties: the lowest predecessor h and the lowest final state win, as torch's min/argmin do.
 * Supported: 2 <= L <= 12 with 1 <= k <= min(4, L-1), where paths longer than 32 steps keep their
 * back-pointers in the workspace; and every other 1 <= k <= min(8, L) with L <= 14 (the reference's
 * uint8 back-pointers allow k <= 8) on a wide search that always keeps them there, a byte per group of
 * 2^k predecessors and position. Workspace: lamq_viterbi_workspace_size(B, T, L, k) bytes (0: none).
 * ---------------------------------------------------------------------------------------------- */
size_t lamq_viterbi_workspace_size(int64_t B, int T, int L, int k);
int lamq_viterbi_rows(const float* x, int64_t B, int T, int64_t ldx, const float* C, int L, int k,
                      const int32_t* start, int32_t* states, int64_t lds, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------
 * One lazy block [b0, b1) of the row-trellis block-LDLQ sweep, for every row.
 * Replaces the inner loop of opgraph/syntax.py:106-121 (sweep) driven by the project closure of
 * opgraph/codes.py:442-450 and RowTrellisCode.step (codes.py:397-404).
 *   T        [m, n] float64 running target (row stride ldT), rows in the rotated basis, not divided
 *            by S; columns [b0, b1) are settled and receive the in-block refit; columns >= b1 are
 *            read (look-ahead) but not written
 *   U        [n, n] float64 upper Cholesky factor of H^-1 (row stride ldU)
 *   S        [m] float64 row scales
 *   table64  [2^L] float64 state values; table32 the same values cast to float32
 *   state    [m] int32, the state before column b0 on entry (0 at b0 = 0), after b1-1 on return
 *   states   [m, n] int32 output for columns [b0, b1) (row stride lds)
 *   Z        [m, b1-b0] float64 output: the block's refit coefficients z = E U_BB^-1 (row stride ldZ),
 *            the left operand of the trailing update
 *   pre      0 <= pre <= min(b0, 1024): the look-ahead columns past b1 lack the trailing updates (syntax.py:123)
 *            of the pre columns before b0, earlier blocks of the caller's run (the caller updates the columns past
 *            the run in one product after the run); the block reads them as T[:, c] - Z[:, -pre:0] U[b0-pre:b0, c],
 *            Z's pre columns before the block holding those blocks' coefficients (ldZ >= pre + b1 - b0).
 *            pre = 0: T already holds every earlier update.
 * width divides lazy = b1-b0 except in the last block; width <= 16, width + look <= 24; b1 - b0 <= 128
 * (the reference runs 16, 8 and 128). Supported: 2 <= L <= 12 with 1 <= k <= min(4, L-1).
 * ---------------------------------------------------------------------------------------------- */
int lamq_ldlq_trellis_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                            const double* S, const double* table64, const float* table32, int L, int k,
                            int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                            int64_t lds, double* Z, int64_t ldZ, int64_t pre, void* stream);

/* ------------------------------------------------------------------------------------------------
 * One lazy block [b0, b1) of the width-1 LDLQ sweep onto a scalar set of K levels.
 * Replaces opgraph/syntax.py:106-121 with the project of opgraph/nested.py:127-140 (mode 0: T is
 * already X/S, index = first argmin_i (t - lv_i)^2, q = lv[index]) or of opgraph/codes.py:322-332,
 * 442-450 (mode 1: T is X, index = bucketize(t/S, midpoints) with halfway ties to the lower level,
 * q = lv[index]*S; S must be given). idx [m, n] int32 output for [b0, b1) (row stride ldi); Z as
 * above. K <= 256, b1 - b0 <= 128.
 * ---------------------------------------------------------------------------------------------- */
int lamq_ldlq_scalar_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                           const double* S, const double* levels, int K, int mode, int64_t b0, int64_t b1,
                           int32_t* idx, int64_t ldi, double* Z, int64_t ldZ, void* stream);

/* The same width-1 block for R rates at once. Replaces opgraph/nested.py:104-147 (multirate_sweep without output
 * shaping): T and Z hold the rates' copies of the m rows stacked rate-major ([R*m, n] and [R*m, b1-b0]: copy r of row i
 * is row r*m + i, X.repeat(R, 1)); one index per entry, idx[i][j] = first argmin_k sum_r w_r (t_r - tables[r*K + k])^2
 * (each term the weight times the rounded square, summed in rate order); copy r settles on tables[r*K + idx] and is
 * refit for its own error. U == NULL: no refit, every column alone (the sweep without H; Z unused).
 * 1 <= R <= 4, K <= 256, b1 - b0 <= 128. */
int lamq_ldlq_multirate_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                              const double* tables, int R, int K, const double* weights, int64_t b0, int64_t b1,
                              int32_t* idx, int64_t ldi, double* Z, int64_t ldZ, void* stream);

/* ------------------------------------------------------------------------------------------------
 * The 16-bit-state trellis (13 <= L <= 16, 1 <= k <= min(4, L-12)): the same two operations as
 * lamq_viterbi_rows and lamq_ldlq_trellis_block (the same references, the same arithmetic and tie rules)
 * for tables whose values are exactly representable in fp16, passed as their fp16 bit patterns
 * (table16, 4-byte aligned; table64 holds the same values in float64 for the settled values).
 * One 1024-thread workgroup per row. The fused block needs width <= 16, width + look <= 24 and
 * b1 - b0 <= 128; the
 * standalone search keeps back-pointers of paths longer than 24 steps in the workspace:
 * lamq_viterbi16_workspace_size(B, T, L, k) bytes.
 * ---------------------------------------------------------------------------------------------- */
size_t lamq_viterbi16_workspace_size(int64_t B, int T, int L, int k);
int lamq_viterbi16_rows(const float* x, int64_t B, int T, int64_t ldx, const uint16_t* table16, int L, int k,
                        const int32_t* start, int32_t* states, int64_t lds, void* workspace,
                        size_t workspace_bytes, void* stream);
int lamq_ldlq_trellis16_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                              const double* S, const double* table64, const uint16_t* table16, int L, int k,
                              int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                              int64_t lds, double* Z, int64_t ldZ, int64_t pre, void* stream);

/* The same fused block with the back-pointers in a caller's workspace: lamq_ldlq_trellis16_block's results, bit for
 * bit. With 2^15 groups (L = 16, k = 1) the minima-exchange search's 128 KB of group minima leave no LDS for the
 * back-pointers; given this workspace, that case runs the minima-exchange kernel (two barriers per step) instead of
 * the quarter-window one (eight). With 2^14 groups (L = 16, k = 2; L = 15, k = 1) the back-pointers (94 KB) fit in
 * LDS beside one 64 KB buffer of group minima; in the workspace they leave room for a second (one barrier per step
 * instead of two). Other (L, k) need none and ignore it.
 * workspace: lamq_ldlq_trellis16_block_workspace_size(m, L, k) bytes (0: not needed), 4-byte aligned. */
size_t lamq_ldlq_trellis16_block_workspace_size(int64_t m, int L, int k);
int lamq_ldlq_trellis16_block_ws(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                 const double* S, const double* table64, const uint16_t* table16, int L, int k,
                                 int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                                 int64_t lds, double* Z, int64_t ldZ, int64_t pre, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* The fused block of every row group of a stage in one launch (the per-group sweeps of quantize.py:502-565 over a
 * stage's row groups, quantize_row_groups, as one batched sweep): group g is the rows [r0, r0 + rows) of T, S, state,
 * states and Z, swept at its k with its tables, and its workspace (lamq_ldlq_trellis16_block_workspace_size(rows, L,
 * k) bytes) where that is not 0. The states, Z and T are lamq_ldlq_trellis16_block_ws's for each group, bit for bit;
 * one launch over all the rows leaves no idle tail between the groups' launches. At most
 * LAMQ_TRELLIS_MAX_GROUPS groups; their row ranges lie in [0, m) and do not overlap. */
#define LAMQ_TRELLIS_MAX_GROUPS 8
typedef struct {
    int64_t r0;
    int64_t rows;
    int k;
    const double* table64;
    const uint16_t* table16;
    void* workspace;
    size_t workspace_bytes;
} lamq_trellis_group;
int lamq_ldlq_trellis16_block_groups(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                     const double* S, int L, const lamq_trellis_group* groups, int ngroups,
                                     int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                                     int64_t lds, double* Z, int64_t ldZ, int64_t pre, void* stream);

/* The same batched block for the 12-bit-state trellis (L = 12, the reference's fitted tables; 1 <= k <= 4): group g
 * is the rows [r0, r0 + rows) of T, S, state, states and Z, swept at its k with its float64 and float32 tables (each
 * 4,096 entries), exactly as lamq_ldlq_trellis_block sweeps that group alone (the same states, Z and T, bit for bit);
 * one launch over all the rows leaves no idle tail between the groups' launches. At most LAMQ_TRELLIS_MAX_GROUPS
 * groups; their row ranges lie in [0, m) and do not overlap. L other than 12: LAMQ_EUNSUP. */
typedef struct {
    int64_t r0;
    int64_t rows;
    int k;
    const double* table64;
    const float* table32;
} lamq_trellis_group32;
int lamq_ldlq_trellis_block_groups(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                   const double* S, int L, const lamq_trellis_group32* groups, int ngroups,
                                   int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                                   int64_t lds, double* Z, int64_t ldZ, int64_t pre, void* stream);

/* ------------------------------------------------------------------------------------------------
 * The lazy trailing update T[:, b1:n] -= Z @ U[b0:b1, b1:n] on fp64 MFMA.
 * Replaces opgraph/syntax.py:122-123 (and opgraph/ldlq_gpu.py:48).
 *   Z [m, b1-b0] (row stride ldZ), b1 - b0 <= 1024.
 * ---------------------------------------------------------------------------------------------- */
int lamq_trailing_update_f64(double* T, int64_t m, int64_t n, int64_t ldT, const double* Z, int64_t ldZ,
                             const double* U, int64_t ldU, int64_t b0, int64_t b1, void* stream);

/* C [M, N] -= A [M, K] @ op(B) in fp64 (op(B) = B [K, N], or B^T for B [N, K] when transb), with op(B) optionally
 * triangular: tri = 1 when op(B)[k][j] = 0 for k < j, tri = 2 when op(B)[k][j] = 0 for k > j (the zero part is then
 * skipped, not read). The products of the QEP targets with the inverse factor, (H + lambda I)^-1 = U^T U
 * (quantize.py:1330-1335, 1503): W D U^T U as two triangular products. Also the noise of compiler.py:124
 * (ldlq_noise's triangular solve E A = eta diag(A), as the product (eta diag(A)) U with U = A^-1). */
int lamq_gemm_sub_f64(double* C, int64_t ldc, const double* A, int64_t lda, const double* B, int64_t ldb, int64_t M,
                      int64_t N, int64_t K, int transb, int tri, void* stream);

/* One step of the generic sweep for a projection Q [m, w] computed by the caller (opgraph/syntax.py:117-121):
 * E = T[:, j:j+w] - Q, z = E U_BB^-1, T[:, j+w:b1] -= z @ U[j:j+w, j+w:b1], Z[:, j-b0 : j-b0+w] = z.
 * The same arithmetic as the fused block kernels; w <= 64. */
int lamq_refit_step(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU, const double* Q,
                    int64_t ldq, int64_t j, int w, int64_t b0, int64_t b1, double* Z, int64_t ldZ, void* stream);

/* T[:, dead] = 0 before a sweep (opgraph/syntax.py:101); dead [n] uint8. */
int lamq_zero_columns(double* T, int64_t m, int64_t n, int64_t ldT, const uint8_t* dead, void* stream);

/* Output shaping: the projection of multirate_sweep with G, one rate (opgraph/nested.py:104-147). Within a column
 * the rows are settled `block` at a time: each entry of rows [a, b) on its nearest level (the first least |u - level|,
 * nested.py:131), then the later rows re-solved, u[b:] -= (u[a:b] - q[a:b]) M_q (nested.py:132-133), with
 * M_q = V[a:b, a:b]^-1 V[a:b, b:] (nested.py:126-127) and V the upper factor of the damped output sensitivity
 * (frame.Environment(G, damp=0.03).U, an lamq_chol_inv_upper factor).
 *   lamq_shaping_feedback: every block's M_q but the last's (empty), packed in block order, each row-major
 *     [(b - a) x (m - b)]: lamq_shaping_feedback_size(m, block) bytes. V [m, m] upper (row stride ldV).
 *   lamq_ldlq_shaped_column: column j of T [m, n] settled so (T is only read): idx[:, j] (int32, row stride ldi >= n)
 *     and the settled levels Q [m] (the projection the caller's refit step subtracts). levels [K], K <= 256.
 * m <= LAMQ_SHAPE_MAX_M (the column lives in LDS), block <= LAMQ_SHAPE_MAX_BLOCK. */
#define LAMQ_SHAPE_MAX_M 16384
#define LAMQ_SHAPE_MAX_BLOCK 64
size_t lamq_shaping_feedback_size(int64_t m, int block);
int lamq_shaping_feedback(const double* V, int64_t m, int64_t ldV, int block, double* M, void* stream);
int lamq_ldlq_shaped_column(const double* T, int64_t m, int64_t n, int64_t ldT, int64_t j, const double* M, int block,
                            const double* levels, int K, int32_t* idx, int64_t ldi, double* Q, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Damped Hessian and the upper Cholesky factor of its inverse.
 * Replaces opgraph/frame.py:515-522 (Environment.__init__):
 *   dead = diag(H) == 0;  H[dead, dead] = 1;  H += damp * mean(diag H) * I;
 *   U = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(H)), upper=True)
 * computed as U = J inv(chol(J H J)) J (J the order reversal), the same unique factor.
 *   H     [n, n] float64 input (row stride ldH; the lower triangle is read)
 *   Hd    NULL or [n, n] float64 output of the damped H (row stride ldHd)
 *   U     [n, n] float64 output (row stride ldU), zero below the diagonal
 *   dead  NULL or [n] uint8 output
 *   info  [1] int32 device output: 0, or j+1 when the leading minor of order j+1 of J H J is not
 *         positive definite (torch.linalg.LinAlgError in the reference)
 *   workspace: lamq_chol_inv_upper_workspace_size(n) bytes
 * lamq_chol_inv_upper enqueues everything on `stream`. lamq_chol_inv_upper_ex may be given a second stream of the
 * caller's, `side_stream` (NULL: none), on which the inverse half of the steps runs, ordered after the work already
 * on `stream` and joined back into `stream` before the call returns (events made and released by the call), so the
 * results are ordered on `stream` either way; the library keeps no streams or other state of its own. Concurrent
 * calls must not share a side stream unless their inverses may run one after the other (the results are the same).
 * ---------------------------------------------------------------------------------------------- */
size_t lamq_chol_inv_upper_workspace_size(int64_t n);
/* flags of lamq_chol_inv_upper_ex: LAMQ_CHOL_KEEP_DEAD leaves a zero diagonal as it is (no unit diagonal at dead
 * columns; the damping mean counts it as zero), as opgraph/ldlq_gpu.py:15-25 (ldlq_factor) damps. */
#define LAMQ_CHOL_KEEP_DEAD 1
int lamq_chol_inv_upper_ex(const double* H, int64_t n, int64_t ldH, double damp, int flags, double* Hd,
                           int64_t ldHd, double* U, int64_t ldU, uint8_t* dead, int32_t* info, void* workspace,
                           size_t workspace_bytes, void* stream, void* side_stream);
int lamq_chol_inv_upper(const double* H, int64_t n, int64_t ldH, double damp, double* Hd, int64_t ldHd,
                        double* U, int64_t ldU, uint8_t* dead, int32_t* info, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Randomized Hadamard transform of rows: out[r, :] = in[r, :] @ R^T with R = (A (x) B)/sqrt(n) diag(s).
 * Replaces the dense products W @ R_in.T and R_in @ H @ R_in.T of opgraph/codes.py:129-132, 430,
 * 439 (rht, incoherence_in) with the Kronecker-factored form of hadamard_factors (codes.py:104-119).
 *   A [a, a], B [b, b] int8 (+1/-1), a*b = n <= 16384; signs [n] int8 (+1/-1)
 *   in/out may alias. rms: NULL or [rows] float64 output max(sqrt(mean_j out[r, j]^2), 1e-12)
 *   (codes.py:436).
 * inverse != 0 applies R instead of R^T: out = in @ R (the reconstruction diag(S) Q R_in of a Net).
 * R H R^T is two row passes with a transpose between them (lamq_transpose_f64, out = in^T, no aliasing).
 * ---------------------------------------------------------------------------------------------- */
int lamq_rht_rows(const double* in, int64_t rows, int64_t n, int64_t ldi, double* out, int64_t ldo,
                  const int8_t* signs, const int8_t* A, int a, const int8_t* B, int b, int inverse, double* rms,
                  void* stream);
int lamq_transpose_f64(const double* in, int64_t rows, int64_t cols, int64_t ldi, double* out, int64_t ldo,
                       void* stream);
/* Row scales S_r = max(sqrt(mean_j X[r, j]^2), 1e-12) (opgraph/codes.py:436, nested.py:168). */
int lamq_row_rms(const double* X, int64_t rows, int64_t n, int64_t ldx, double* S, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Token-weighted Gram matrix on bf16 MFMA with fp32 accumulation:
 *   H[i, j] += scale * sum_t w_t X[t, i] X[t, j]     (lower triangle i >= j written; upper untouched)
 * Replaces the capture accumulation of quantize.py:1465 (H += X^T (w * X)), compiler.py:244 and
 * opgraph/frame.py:498-505.
 *   X [N, n] bf16 (row stride ldx; n and ldx even, X 4-byte aligned);  w NULL (every w_t = 1) or
 *   [N] float32;  H [n, n] float32 (row stride ldH).
 * Without w, and with n and ldx multiples of 8 and X 16-byte aligned, the 256x256-tile kernel runs.
 * With w the weighted operand is split into two bf16 parts (hi + lo) so the products keep float32
 * precision (twice the MFMA work; lamq_hessian_accum_rows below is exact and costs one product when
 * the weights take few values). Small n splits the tokens over workgroups; the partial sums then go
 * through the workspace (lamq_gram_workspace_size(N, n, 1) bytes, possibly 0) and are added in a
 * fixed order.
 * lamq_hessian_finalize mirrors the lower triangle, divides by ntok (quantize.py:1470) and, if H64
 * is given, writes the float64 copy the sweep consumes.
 * ---------------------------------------------------------------------------------------------- */
size_t lamq_gram_workspace_size(int64_t N, int64_t n, int sym);
int lamq_hessian_accum(const uint16_t* X, int64_t N, int64_t n, int64_t ldx, const float* w, float scale,
                       float* H, int64_t ldH, void* workspace, size_t workspace_bytes, void* stream);
int lamq_hessian_finalize(float* H, int64_t n, int64_t ldH, float ntok, double* H64, int64_t ldH64,
                          void* stream);

/* QEP cross-Gram D[i, j] += scale * sum_t w_t Xr[t, i] Xq[t, j] (all of D), quantize.py:1457.
 * Workspace: lamq_gram_workspace_size(N, n, 0) bytes. */
int lamq_cross_gram(const uint16_t* Xr, const uint16_t* Xq, int64_t N, int64_t n, int64_t ldx, const float* w,
                    float scale, float* D, int64_t ldD, void* workspace, size_t workspace_bytes, void* stream);

/* The same sums over a list of token rows, unweighted, on the 256x256-tile kernel:
 *   H[i, j] += scale * sum_{r in rows} X[r, i] X[r, j]   (lower triangle)
 *   D[i, j] += scale * sum_{r in rows} Xr[r, i] Xq[r, j]
 * A token weight shared by a set of rows is the scale of that set's call: quantize.py:1389-1391 weights
 * tokens by their kind (token_weights with the digits specs, quantize.py:593-607, gives at most three
 * distinct weights), so H = sum over the distinct weights c of w_c * X_c^T X_c, with exact bf16
 * products and float32 sums. rows: nrows int32 indices into X (each < the rows of X);
 * n and ldx multiples of 8, X 16-byte aligned (else LAMQ_EUNSUP). Workspace:
 * lamq_gram_workspace_size(nrows, n, 1 or 0) bytes. */
int lamq_hessian_accum_rows(const uint16_t* X, const int32_t* rows, int64_t nrows, int64_t n, int64_t ldx, float scale,
                            float* H, int64_t ldH, void* workspace, size_t workspace_bytes, void* stream);
int lamq_cross_gram_rows(const uint16_t* Xr, const uint16_t* Xq, const int32_t* rows, int64_t nrows, int64_t n,
                         int64_t ldx, float scale, float* D, int64_t ldD, void* workspace, size_t workspace_bytes,
                         void* stream);

/* ------------------------------------------------------------------------------------------------
 * Per-token KL(p_ref || p_q) of two bf16 logit matrices in one streaming pass.
 * Replaces compiler.py:177-188 (kl()), quantize.py:904-920 and text_kl.py:57-61:
 *   kl_t = sum_v softmax(ref_t)_v (log_softmax(ref_t)_v - log_softmax(q_t)_v)
 *   ref, q  [T, V] bf16 (row strides ldr, ldq);  w NULL or [T] float32 token weights
 *   kl      [T] float32 output;  sums [2] float64 output: sum_t w_t kl_t and sum_t w_t
 * workspace: lamq_kl_workspace_size(T) bytes.
 * ---------------------------------------------------------------------------------------------- */
size_t lamq_kl_workspace_size(int64_t T);
int lamq_kl_rows(const uint16_t* ref, const uint16_t* q, int64_t T, int64_t V, int64_t ldr, int64_t ldq,
                 const float* w, float* kl, double* sums, void* workspace, size_t workspace_bytes, void* stream);

/* The same on float32 logits: the reference takes the model's logits as .logits.float() (compiler.py:180,185), so a
 * float32 model's logits enter unrounded. Same arguments, workspace and results; on logits bf16 holds exactly the
 * results equal lamq_kl_rows' bit for bit (the same float32 arithmetic in the same order). */
int lamq_kl_rows_f32(const float* ref, const float* q, int64_t T, int64_t V, int64_t ldr, int64_t ldq,
                     const float* w, float* kl, double* sums, void* workspace, size_t workspace_bytes, void* stream);

/* lamq_kl_rows without a workspace and without any allocation: no counterpart in the reference. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving or measurement loops, harnesses that
 * forbid hipMalloc). The per-token partials live in a static device array of LAMQ_KL_NOALLOC_MAX_T * 2 float64
 * (1 MiB) that each GPU holds until the process ends; its address is looked up once per device on the first call
 * (the stream's device must be current). T > LAMQ_KL_NOALLOC_MAX_T returns LAMQ_EINVAL before any launch. Every
 * entry of the array a call reads it has written first, so nothing needs clearing; calls that overlap on one GPU
 * (two streams at once) share the array and race. Same arguments and results as lamq_kl_rows otherwise. */
#define LAMQ_KL_NOALLOC_MAX_T 65536
int lamq_kl_rows_noalloc(const uint16_t* ref, const uint16_t* q, int64_t T, int64_t V, int64_t ldr, int64_t ldq,
                         const float* w, float* kl, double* sums, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Pack row-trellis states into the opgraph-packed-1 bitstream.
 * Replaces compiler_artifact.py:225-240 (pack_symbols) and :261-284 (valid_path, pack_trellis):
 *   symbols = state & (2^k - 1), each row padded forward to a multiple of 32, reversed, then
 *   packed little-endian, k uint32 words per 32 symbols.
 *   states [m, n] int32 (row stride lds);  codes [m, ceil(n/32)*k] uint32 (row stride ldc)
 *   bad    [1] int32 device output, set to 1 if any row is not a trellis path from state 0
 *          (the reference raises ValueError); must be zero on entry. 1 <= k <= 8, k < L <= 16.
 * ---------------------------------------------------------------------------------------------- */
int lamq_pack_trellis(const int32_t* states, int64_t m, int64_t n, int64_t lds, int k, int L, uint32_t* codes,
                      int64_t ldc, int32_t* bad, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Pack one row group of a matrix's code array into the opgraph-packed-1 bitstream, reading the group's rows in
 * place. Replaces compiler_artifact.py:225-240 (pack_symbols), :261-284 (valid_path, pack_trellis) and the
 * per-group slicing and checks of encode_entry (:328-353: encoded[rows] - table_index * 4096, "a row crosses
 * table identities", "scalar index outside table").
 *   src    [src_rows, n] int32 (row stride ld >= n): the matrix's codes (trellis states or scalar symbols)
 *   rows   [m] int64 indices into src (NULL: rows 0..m-1); a row outside [0, src_rows) sets bad bit 2 and
 *          its code words to zero, nothing is read for it
 *   base   subtracted from every entry (the group's table offset, table_index * 2^L)
 *   trellis = 1: entries are row-trellis states; symbols state & (2^k - 1), each row padded forward to a
 *          multiple of 32 and reversed; bad bit 1 if a row, after base, is not a path from state 0 in
 *          [0, 2^L). 1 <= k < L <= 16.
 *   trellis = 0: entries are scalar symbols packed in column order; bad bit 1 if one is outside [0, 2^k).
 *   codes  [m, ceil(n/32)*k] uint32 (row stride ldc);  1 <= k <= 8
 *   bad    [1] int32 device flags (must be zero on entry; the reference raises ValueError)
 * lamq_pack_trellis(states, m, n, lds, k, L, ...) is lamq_pack_codes(states, lds, m, NULL, m, n, 0, k, L, 1, ...).
 * ---------------------------------------------------------------------------------------------- */
int lamq_pack_codes(const int32_t* src, int64_t ld, int64_t src_rows, const int64_t* rows, int64_t m, int64_t n,
                    int32_t base, int k, int L, int trellis, uint32_t* codes, int64_t ldc, int32_t* bad, void* stream);

/* ------------------------------------------------------------------------------------------------
 * lamq_pack_codes for many row groups in one launch (per 32 groups): every group of a stage's matrices, where a launch
 * per group (a few hundred rows each) costs more in fixed launch time than its HBM traffic. Replaces the per-group
 * loop of compiler_artifact.py:328-353 (encode_entry over a matrix's groups) around pack_symbols and pack_trellis
 * (:225-240, :261-284). Each entry carries one lamq_pack_codes call's src, ld, src_rows, rows, m, base, k, codes and
 * ldc; n, L and trellis are shared. Every group's code words and bad flags are those lamq_pack_codes gives for it
 * alone (the same arithmetic); groups must not share code words. Every entry is checked, as lamq_pack_codes checks
 * its arguments, before anything is launched.
 * ---------------------------------------------------------------------------------------------- */
typedef struct {
    const int32_t* src;
    int64_t ld;
    int64_t src_rows;
    const int64_t* rows;
    int64_t m;
    int32_t base;
    int k;
    uint32_t* codes;
    int64_t ldc;
} lamq_pack_group;
int lamq_pack_codes_groups(const lamq_pack_group* groups, int ngroups, int64_t n, int L, int trellis, int32_t* bad,
                           void* stream);

/* ------------------------------------------------------------------------------------------------
 * The causal softmax of the calibration forwards' attention (the forward of the model the reference's capture runs,
 * quantize.py:1029, 1626-1694: transformers' causal attention, scores times scaling, the causal mask, softmax in
 * float32, cast back to bf16), fused into one pass over bf16 scores:
 *   P[r, c] = bf16( exp(s[r, c] - m_r) / sum_c' exp(s[r, c'] - m_r) ),  s = float(S[r, c]) * scale for c <= r % T,
 *   -inf past it;  m_r = max_c s[r, c].
 *   S, P   [rows, T] bf16 bits (row strides lds, ldp; 16-byte aligned, strides multiples of 8); rows run over
 *          (sequence, head, query), query r % T. P may be S (same stride); otherwise they may not overlap.
 *   T % 8 == 0, T <= 4096; scale > 0.
 * ---------------------------------------------------------------------------------------------- */
int lamq_causal_softmax_bf16(const uint16_t* S, uint16_t* P, int64_t rows, int T, int64_t lds, int64_t ldp,
                             float scale, void* stream);

/* RMSNorm of the forwards (the calibration model's RMSNorm, quantize.py:1029, in float32 and back to bf16):
 *   Y[r, :] = bf16( float(bf16(x * rsqrt(mean(x^2) + eps))) * float(g) ),  x = float(X[r, :])
 *   X [rows, n] (row stride ldx), Y [rows, n] (ldy), g [n], bf16 bits; n, ldx, ldy multiples of 8, X, Y, g 16-byte
 *   aligned; n <= 10,240 (LAMQ_EUNSUP above). Replaces the pow / mean / rsqrt / mul chain of the forwards. */
int lamq_rms_norm_bf16(const uint16_t* X, int64_t rows, int64_t n, int64_t ldx, const uint16_t* g, uint16_t* Y,
                       int64_t ldy, float eps, void* stream);

/* The per-head RMSNorm of q and k and the rotary embedding after it, fused (the calibration model's q_norm / k_norm
 * and apply_rotary_pos_emb, quantize.py:1029, in the roundings of the unfused bf16 chain):
 *   y = bf16( float(bf16(x * rsqrt(mean(x^2) + eps))) * float(g) )        (a row of lamq_rms_norm_bf16)
 *   Y[r, i] = bf16( float(bf16(y[i] * cos[t, i])) + float(bf16(rot[i] * sin[t, i])) ),
 *   rot[i] = -y[i + 64] (i < 64), y[i - 64] (i >= 64),  t = (r / heads) % T
 *   X [rows, n] (row stride ldx), Y [rows, n] (ldy), g [n], cos and sin [T, n] (row stride ldcs), bf16 bits, rows
 *   ordered (sequence, token, head), rows a multiple of heads * T; n = 128 (LAMQ_EUNSUP otherwise); strides
 *   multiples of 8, pointers 16-byte aligned. Replaces q_norm / k_norm followed by q * cos + rotate_half(q) * sin
 *   (a negation, a concatenation, two products and a sum over q and over k) in the forwards. */
int lamq_rms_norm_rope_bf16(const uint16_t* X, int64_t rows, int64_t n, int64_t ldx, const uint16_t* g,
                            const uint16_t* cosT, const uint16_t* sinT, int64_t ldcs, int64_t heads, int64_t T,
                            uint16_t* Y, int64_t ldy, float eps, void* stream);

/* The MLP gate of the forwards (silu(gate) * up, in float32 with the bf16 rounding after each of the two as the
 * unfused chain rounds): y = bf16(float(bf16(a / (1 + exp(-a)))) * float(b)), n elements (a multiple of 8) of
 * 16-byte aligned contiguous bf16 a, b, y. */
int lamq_swiglu_bf16(const uint16_t* a, const uint16_t* b, uint16_t* y, int64_t n, void* stream);

/* ----------------------------------------------------------------------------------------------
 * Causal grouped-query attention of the forwards, fused (the attention lamq_causal_softmax_bf16 serves, quantize.py:1029 and the
 * layer loop 1626-1694, with the scores kept in registers: an online softmax over key blocks of 32, exp2 with the
 * scale folded in, probabilities rounded to bf16 for the product with v, float32 sums):
 *   out[b, t, h, :] = sum_{u <= t} softmax_u(q[b, h, t, :] . k[b, h / (H / Hkv), u, :] * scale) v[b, h / (H / Hkv), u, :]
 *   q [B, H, T, 128], k, v [B, Hkv, T, 128], out [B, H, T, 128] bf16 bits, each given by its (batch, head, token)
 *   strides in elements with the head dim contiguous; strides multiples of 8, q, k, v 16-byte and out 8-byte
 *   aligned. H % Hkv == 0; head dim 128 (LAMQ_EUNSUP otherwise); scale > 0.
 * Replaces the bf16 q k^T product, lamq_causal_softmax_bf16 and the product with v in the forwards.
 * T from 1 to 8,388,607; B, H at most 65,535 (LAMQ_EUNSUP above).
 * ---------------------------------------------------------------------------------------------- */
int lamq_attention_causal_bf16(const uint16_t* q, int64_t sqb, int64_t sqh, int64_t sqt, const uint16_t* k,
                               int64_t skb, int64_t skh, int64_t skt, const uint16_t* v, int64_t svb, int64_t svh,
                               int64_t svt, uint16_t* out, int64_t sob, int64_t soh, int64_t sot, int64_t B, int64_t H,
                               int64_t Hkv, int64_t T, int64_t D, float scale, void* stream);

/* ----------------------------------------------------------------------------------------------
 * Measurement only; no counterpart in the reference. The L2-to-CU delivery ceiling of the direct global->LDS load path
 * the Gram kernels feed their MFMAs through: `workgroups` workgroups (one a CU: 160 KB of LDS each) stream `stages`
 * stages of 32 KB each (1 KB loads of 16 bytes a lane, a five-buffer LDS ring, one barrier a stage) from the
 * region_bytes-long region (region_bytes a multiple of 1,024, at least 65,536) of buf that belongs to their XCD:
 * workgroup b reads region b % 8, so buf holds 8 regions. Bytes delivered: workgroups * stages * 32,768.
 * ---------------------------------------------------------------------------------------------- */
int lamq_probe_l2_delivery(const void* buf, int64_t region_bytes, int stages, int workgroups, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* LAMQ_H */
