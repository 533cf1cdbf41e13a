// Damped Hessian and U = the upper Cholesky factor of its inverse (opgraph/frame.py:515-522).
//
// With J the order reversal, J Hd J = L L^T (L lower) gives Hd = V V^T with V = J L J upper, so
// Hd^-1 = V^-T V^-1 and U = V^-1 = J L^-1 J is upper with a positive diagonal: the factor
// torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(Hd)), upper=True) returns.
// One Cholesky (n^3/3 flops) and one triangular inverse (n^3/3) replace the reference's three
// factorizations (4n^3/3). Both are blocked right-looking with 64-wide panels. One wave factors each
// diagonal block in LDS and inverts it (Lkk^-1 kept in the workspace); the panel below, the block rows
// of the inverse and all trailing updates are then fp64 MFMA products: panel = A_panel Lkk^-T,
// X_k = Lkk^-1 B_k.
#include "gemm_f64.h"

#define NBK 64
#define NB2 256  // panel width of the two-level blocking (a multiple of NBK)

// dead = diag(H) == 0; the damping delta = damp * mean(diag H') where H' has unit diagonal at dead (with
// keep_dead, H' = H: the dead diagonal stays zero and counts as zero).
__global__ __launch_bounds__(256) void diag_stats_kernel(const double* __restrict__ H, int64_t n, int64_t ldH, double damp,
                                                         int keep_dead, uint8_t* __restrict__ dead,
                                                         double* __restrict__ delta, int32_t* __restrict__ info)
{
    __shared__ double part[256];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const double d = H[i * ldH + i];
        const bool z = d == 0.0;
        if (dead) dead[i] = z ? 1 : 0;
        s += (z && !keep_dead) ? 1.0 : d;
    }
    part[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const double mean = part[0] / (double)n;
        *delta = damp * mean;
        *info = 0;
    }
}

// A = J Hd J (lower triangle), Hd = H with unit diagonal at dead columns (unless keep_dead) plus delta on the
// diagonal.
__global__ void prep_kernel(const double* __restrict__ H, int64_t n, int64_t ldH, const double* __restrict__ delta,
                            int keep_dead, double* __restrict__ A, double* __restrict__ Hd, int64_t ldHd)
{
    const int64_t i = (int64_t)blockIdx.y * 16 + threadIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i >= n || j >= n) return;
    double v = H[i * ldH + j];
    if (i == j) v = ((v == 0.0 && !keep_dead) ? 1.0 : v) + *delta;
    // the factorization reads the lower triangle of H, as LAPACK's lower Cholesky does: H[i][j]
    // with i >= j lands on A[n-1-j][n-1-i], in the lower triangle of A
    if (i >= j) A[(n - 1 - j) * n + (n - 1 - i)] = v;
    if (Hd) Hd[i * ldHd + j] = v;
}

// The nb x nb diagonal block at (k0, k0) of A (lower): its Cholesky factor Lkk, written back into A, and
// Lkk^-1 (lower), written to Linv (ld NBK). One wave, everything in registers and fully unrolled (register
// arrays need compile-time indices); a block shorter than NBK is padded with the identity.
// Factorization: lane i holds row i, r[j] = a[i][j]. Column c: d = a[c][c]; l[i][c] = a[i][c] / sqrt(d)
// (l[c][c] = sqrt(d)); a[i][j] -= l[i][c] l[j][c] for j > c. Column c of L is published through LDS
// (lt[c][i] = l[i][c]) and read back as broadcasts.
// Inverse: lane c holds column c of X = L^-1, x = e_c initially; for l = 0..: x[l] /= l[l][l];
// x[i] -= l[i][l] x[l] for i > l (the l[i][l] broadcast from lt).
__global__ __launch_bounds__(64) void diag_block_kernel(double* __restrict__ A, int64_t n, int64_t k0, int nb,
                                                        double* __restrict__ Linv, int32_t* __restrict__ info)
{
    __shared__ __align__(16) double lt[NBK][NBK];  // lt[c][i] = L[i][c]
    if (*info != 0) return;
    const int lane = threadIdx.x;
    const bool live = lane < nb;
    double r[NBK];
    // branch-free loads: rows and columns clamped into the block, padding selected afterwards
    const double* Ar = A + (k0 + (live ? lane : 0)) * n + k0;
#pragma unroll
    for (int j = 0; j < NBK; ++j) {
        const double v = Ar[j < nb ? j : nb - 1];
        r[j] = (live && j < nb) ? (j <= lane ? v : 0.0) : (j == lane ? 1.0 : 0.0);
    }
    int fail = 0;  // the first non-positive pivot; the loop runs on without branching, its output unused
#pragma unroll
    for (int c = 0; c < NBK; ++c) {
        lt[c][lane] = r[c];
        const double d = lt[c][c];
        fail = (fail == 0 && !(d > 0.0)) ? (int)(k0 + c + 1) : fail;
        const double sd = sqrt(d);
        const double lic = lane > c ? r[c] / sd : (lane == c ? sd : 0.0);
        r[c] = lic;
        lt[c][lane] = lic;
#pragma unroll
        for (int j = c + 1; j < NBK; ++j) r[j] = fma(-lic, lt[c][j], r[j]);
        // the empty asm pins this step's updates here: without it the compiler sinks them into per-column dot
        // products (a left-looking order) that keep every broadcast value live. One group per step, after all of
        // the step's loads, so the loads still issue back to back.
#pragma unroll
        for (int j = c + 1; j < NBK; ++j) asm volatile("" : "+v"(r[j]));
    }
    if (fail != 0) {  // uniform
        if (lane == 0) *info = fail;
        return;
    }
    if (live) {
        double* Aw = A + (k0 + lane) * n + k0;
#pragma unroll
        for (int j = 0; j < NBK; ++j)
            if (j < nb && j <= lane) Aw[j] = r[j];
    }
    double x[NBK];
#pragma unroll
    for (int i = 0; i < NBK; ++i) x[i] = i == lane ? 1.0 : 0.0;
#pragma unroll
    for (int l = 0; l < NBK; ++l) {
        x[l] = x[l] / lt[l][l];
#pragma unroll
        for (int i = l + 1; i < NBK; ++i) x[i] = fma(-lt[l][i], x[l], x[i]);
#pragma unroll
        for (int i = l + 1; i < NBK; ++i) asm volatile("" : "+v"(x[i]));
    }
#pragma unroll
    for (int i = 0; i < NBK; ++i) Linv[i * NBK + lane] = x[i];
}

__global__ void identity_kernel(double* __restrict__ X, int64_t n, int64_t ldX)
{
    const int64_t i = (int64_t)blockIdx.y * 16 + threadIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i < n && j < n) X[i * ldX + j] = i == j ? 1.0 : 0.0;
}

// U = J X J (upper), in place: entries (i, j) and (n-1-i, n-1-j) swap, then the strict lower part is
// cleared. X is lower triangular on entry.
__global__ void reverse_kernel(double* __restrict__ U, int64_t n, int64_t ldU, const int32_t* __restrict__ info)
{
    const int64_t i = (int64_t)blockIdx.y * 16 + threadIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i >= n || j >= n) return;
    const int64_t pi = n - 1 - i, pj = n - 1 - j;
    if (*info != 0) {
        U[i * ldU + j] = 0.0;
        return;
    }
    if (j > i) return;  // strict upper entries of X are zero; their partner thread writes them
    if (i == j) {
        // diagonal pairs (i, i) <-> (pi, pi): swapped by the member with i < pi
        if (i < pi) {
            const double a = U[i * ldU + i], b = U[pi * ldU + pi];
            U[i * ldU + i] = b;
            U[pi * ldU + pi] = a;
        }
        return;
    }
    // j < i: the partner (pi, pj) has pj > pi, a strict upper entry that holds zero and that no
    // other thread reads or writes
    U[pi * ldU + pj] = U[i * ldU + j];
    U[i * ldU + j] = 0.0;
}

extern "C" size_t lamq_chol_inv_upper_workspace_size(int64_t n)
{
    if (n < 1) return 0;
    // J Hd J and its factor, the inverses of the diagonal blocks, the damping scalar
    return (size_t)n * (size_t)n * sizeof(double) + (size_t)cdiv(n, NBK) * NBK * NBK * sizeof(double) + 256;
}

extern "C" int lamq_chol_inv_upper_ex(const double* H, int64_t n, int64_t ldH, double damp, int flags, double* Hd,
                                      int64_t ldHd, double* U, int64_t ldU, uint8_t* dead, int32_t* info, void* workspace,
                                      size_t workspace_bytes, void* stream)
{
    if (!H || !U || !info || !workspace || n < 1 || ldH < n || ldU < n || (Hd && ldHd < n)) return LAMQ_EINVAL;
    if (flags & ~LAMQ_CHOL_KEEP_DEAD) return LAMQ_EINVAL;
    const int keep_dead = (flags & LAMQ_CHOL_KEEP_DEAD) ? 1 : 0;
    if (workspace_bytes < lamq_chol_inv_upper_workspace_size(n)) return LAMQ_EINVAL;
    if (n > (int64_t)1 << 20) return LAMQ_EUNSUP;
    hipStream_t s = as_stream(stream);
    double* A = reinterpret_cast<double*>(workspace);
    double* Linv = A + n * n;  // cdiv(n, NBK) blocks of NBK x NBK
    double* delta = Linv + cdiv(n, NBK) * NBK * NBK;
    hipLaunchKernelGGL(diag_stats_kernel, dim3(1), dim3(256), 0, s, H, n, ldH, damp, keep_dead, dead, delta, info);
    LAMQ_LAUNCH_CHECK();
    const dim3 g2((unsigned)cdiv(n, 64), (unsigned)cdiv(n, 16)), b2(64, 16);
    hipLaunchKernelGGL(prep_kernel, g2, b2, 0, s, H, n, ldH, delta, keep_dead, A, Hd, ldHd);
    LAMQ_LAUNCH_CHECK();
    // Cholesky of A = J Hd J, lower, in panels of NB2 columns: inside a panel, 64-wide steps update only the panel's
    // own columns; the columns after it get one product of depth NB2 per panel (a quarter of the traffic of 64-deep
    // updates of the whole trailing matrix)
    for (int64_t K0 = 0; K0 < n; K0 += NB2) {
        const int64_t pe = (K0 + NB2 < n) ? K0 + NB2 : n;
        for (int64_t k0 = K0; k0 < pe; k0 += NBK) {
            const int nb = (int)(n - k0 < NBK ? n - k0 : NBK);
            double* Lk = Linv + (k0 / NBK) * NBK * NBK;
            hipLaunchKernelGGL(diag_block_kernel, dim3(1), dim3(64), 0, s, A, n, k0, nb, Lk, info);
            LAMQ_LAUNCH_CHECK();
            const int64_t rest = n - k0 - nb;
            if (rest > 0) {
                double* P = A + (k0 + nb) * n + k0;
                // P = P Lkk^-T (the row-wise triangular solve as one product, in place: one tile column)
                int rc = gemm_sub_f64<true, false, true>(P, n, P, n, Lk, NBK, rest, nb, nb, info, s);
                if (rc) return rc;
                const int64_t pc = pe - (k0 + nb);
                if (pc > 0) {
                    rc = gemm_sub_f64<true, true>(A + (k0 + nb) * n + k0 + nb, n, P, n, P, n, rest, pc, nb, info, s);
                    if (rc) return rc;
                }
            }
        }
        const int64_t rest = n - pe;
        if (rest > 0) {
            const double* P = A + pe * n + K0;
            int rc = gemm_sub_f64<true, true>(A + pe * n + pe, n, P, n, P, n, rest, rest, pe - K0, info, s);
            if (rc) return rc;
        }
    }
    // X = L^-1 into U (right-looking solve of L X = I): X_k = Lkk^-1 B_k, then B_i -= L_ik X_k below, inside the
    // panel at once and below it once per panel (X is lower triangular, so the panel's rows are zero right of
    // their diagonal and one product of depth NB2 carries the panel's steps)
    hipLaunchKernelGGL(identity_kernel, g2, b2, 0, s, U, n, ldU);
    LAMQ_LAUNCH_CHECK();
    for (int64_t K0 = 0; K0 < n; K0 += NB2) {
        const int64_t pe = (K0 + NB2 < n) ? K0 + NB2 : n;
        for (int64_t k0 = K0; k0 < pe; k0 += NBK) {
            const int nb = (int)(n - k0 < NBK ? n - k0 : NBK);
            const double* Lk = Linv + (k0 / NBK) * NBK * NBK;
            int rc = gemm_sub_f64<false, false, true>(U + k0 * ldU, ldU, Lk, NBK, U + k0 * ldU, ldU, nb, k0 + nb, nb, info,
                                                      s);
            if (rc) return rc;
            const int64_t rin = pe - (k0 + nb);
            if (rin > 0) {
                rc = gemm_sub_f64<false, false>(U + (k0 + nb) * ldU, ldU, A + (k0 + nb) * n + k0, n, U + k0 * ldU, ldU, rin,
                                                k0 + nb, nb, info, s);
                if (rc) return rc;
            }
        }
        const int64_t rest = n - pe;
        if (rest > 0) {
            int rc = gemm_sub_f64<false, false>(U + pe * ldU, ldU, A + pe * n + K0, n, U + K0 * ldU, ldU, rest, pe, pe - K0,
                                                info, s);
            if (rc) return rc;
        }
    }
    hipLaunchKernelGGL(reverse_kernel, g2, b2, 0, s, U, n, ldU, info);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

extern "C" int lamq_chol_inv_upper(const double* H, int64_t n, int64_t ldH, double damp, double* Hd, int64_t ldHd,
                                   double* U, int64_t ldU, uint8_t* dead, int32_t* info, void* workspace,
                                   size_t workspace_bytes, void* stream)
{
    return lamq_chol_inv_upper_ex(H, n, ldH, damp, 0, Hd, ldHd, U, ldU, dead, info, workspace, workspace_bytes, stream);
}
