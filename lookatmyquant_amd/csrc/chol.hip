// Damped Hessian and U = the upper Cholesky factor of its inverse (opgraph/frame.py:515-522).
//
// With J the order reversal, J Hd J = L L^T (L lower) gives Hd = V V^T with V = J L J upper, so
// Hd^-1 = V^-T V^-1 and U = V^-1 = J L^-1 J is upper with a positive diagonal: the factor
// torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(Hd)), upper=True) returns.
// One Cholesky (n^3/3 flops) and one triangular inverse (n^3/3) replace the reference's three
// factorizations (4n^3/3). Both are blocked right-looking with 64-wide panels: the diagonal block
// is factored in LDS by one workgroup, the panel below by a row-parallel triangular solve, and the
// trailing updates run on fp64 MFMA.
#include "gemm_f64.h"

#define NBK 64

// dead = diag(H) == 0; the damping delta = damp * mean(diag H') where H' has unit diagonal at dead.
__global__ __launch_bounds__(256) void diag_stats_kernel(const double* __restrict__ H, int64_t n, int64_t ldH, double damp,
                                                         uint8_t* __restrict__ dead, double* __restrict__ delta,
                                                         int32_t* __restrict__ info)
{
    __shared__ double part[256];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const double d = H[i * ldH + i];
        const bool z = d == 0.0;
        if (dead) dead[i] = z ? 1 : 0;
        s += z ? 1.0 : d;
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

// A = J Hd J (lower triangle), Hd = H with unit diagonal at dead columns plus delta on the diagonal.
__global__ void prep_kernel(const double* __restrict__ H, int64_t n, int64_t ldH, const double* __restrict__ delta,
                            double* __restrict__ A, double* __restrict__ Hd, int64_t ldHd)
{
    const int64_t i = (int64_t)blockIdx.y * 16 + threadIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i >= n || j >= n) return;
    double v = H[i * ldH + j];
    if (i == j) v = (v == 0.0 ? 1.0 : v) + *delta;
    // the factorization reads the lower triangle of H, as LAPACK's lower Cholesky does: H[i][j]
    // with i >= j lands on A[n-1-j][n-1-i], in the lower triangle of A
    if (i >= j) A[(n - 1 - j) * n + (n - 1 - i)] = v;
    if (Hd) Hd[i * ldHd + j] = v;
}

// Unblocked Cholesky of the nb x nb diagonal block at (k0, k0) of A (lower), in LDS.
__global__ __launch_bounds__(256) void potf2_kernel(double* __restrict__ A, int64_t n, int64_t k0, int nb,
                                                    int32_t* __restrict__ info)
{
    __shared__ double a[NBK][NBK + 1];
    __shared__ int fail;
    if (*info != 0) return;
    for (int e = threadIdx.x; e < nb * nb; e += 256) {
        const int i = e / nb, j = e - i * nb;
        a[i][j] = j <= i ? A[(k0 + i) * n + k0 + j] : 0.0;
    }
    if (threadIdx.x == 0) fail = 0;
    __syncthreads();
    for (int c = 0; c < nb; ++c) {
        if (threadIdx.x == 0) {
            const double d = a[c][c];
            if (!(d > 0.0)) {
                fail = 1;
                *info = (int32_t)(k0 + c + 1);
            } else {
                a[c][c] = sqrt(d);
            }
        }
        __syncthreads();
        if (fail) return;
        const double l = a[c][c];
        for (int i = c + 1 + threadIdx.x; i < nb; i += 256) a[i][c] = a[i][c] / l;
        __syncthreads();
        const int m = nb - c - 1;
        for (int e = threadIdx.x; e < m * m; e += 256) {
            const int i = c + 1 + e / m, j = c + 1 + e % m;
            if (j <= i) a[i][j] = fma(-a[i][c], a[j][c], a[i][j]);
        }
        __syncthreads();
    }
    for (int e = threadIdx.x; e < nb * nb; e += 256) {
        const int i = e / nb, j = e - i * nb;
        if (j <= i) A[(k0 + i) * n + k0 + j] = a[i][j];
    }
}

// Panel below the diagonal block: rows i >= k0+nb, X = A[i, k0:k0+nb] L_kk^-T, by forward
// substitution per row: x[c] = (a[c] - sum_{l<c} x[l] L[c][l]) / L[c][c]. 64 rows per workgroup.
__global__ __launch_bounds__(64) void trsm_panel_kernel(double* __restrict__ A, int64_t n, int64_t k0, int nb,
                                                        const int32_t* __restrict__ info)
{
    __shared__ double Lk[NBK][NBK + 1];
    __shared__ double x[64][NBK + 1];
    if (*info != 0) return;
    for (int e = threadIdx.x; e < nb * nb; e += 64) {
        const int i = e / nb, j = e - i * nb;
        Lk[i][j] = j <= i ? A[(k0 + i) * n + k0 + j] : 0.0;
    }
    const int64_t rbase = k0 + nb + (int64_t)blockIdx.x * 64;
    for (int e = threadIdx.x; e < 64 * nb; e += 64) {
        const int r = e / nb, c = e - r * nb;
        x[r][c] = (rbase + r < n) ? A[(rbase + r) * n + k0 + c] : 0.0;
    }
    __syncthreads();
    const int r = threadIdx.x;
    for (int c = 0; c < nb; ++c) {
        double acc = x[r][c];
        for (int l = 0; l < c; ++l) acc = fma(-x[r][l], Lk[c][l], acc);
        x[r][c] = acc / Lk[c][c];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * nb; e += 64) {
        const int rr = e / nb, c = e - rr * nb;
        if (rbase + rr < n) A[(rbase + rr) * n + k0 + c] = x[rr][c];
    }
}

__global__ void identity_kernel(double* __restrict__ X, int64_t n, int64_t ldX)
{
    const int64_t i = (int64_t)blockIdx.y * 16 + threadIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i < n && j < n) X[i * ldX + j] = i == j ? 1.0 : 0.0;
}

// Block row k of L X = I: X[k0:k0+nb, c] = L_kk^-1 B[k0:k0+nb, c] for the columns c < k0+nb,
// by forward substitution per column; 64 columns per workgroup.
__global__ __launch_bounds__(64) void trsm_left_kernel(const double* __restrict__ A, int64_t n, double* __restrict__ X,
                                                       int64_t ldX, int64_t k0, int nb, const int32_t* __restrict__ info)
{
    __shared__ double Lk[NBK][NBK + 1];
    __shared__ double y[NBK][64 + 1];
    if (*info != 0) return;
    for (int e = threadIdx.x; e < nb * nb; e += 64) {
        const int i = e / nb, j = e - i * nb;
        Lk[i][j] = j <= i ? A[(k0 + i) * n + k0 + j] : 0.0;
    }
    const int64_t cbase = (int64_t)blockIdx.x * 64;
    const int64_t ncols = k0 + nb;
    for (int e = threadIdx.x; e < nb * 64; e += 64) {
        const int i = e / 64, c = e - i * 64;
        y[i][c] = (cbase + c < ncols) ? X[(k0 + i) * ldX + cbase + c] : 0.0;
    }
    __syncthreads();
    const int c = threadIdx.x;
    for (int i = 0; i < nb; ++i) {
        double acc = y[i][c];
        for (int l = 0; l < i; ++l) acc = fma(-Lk[i][l], y[l][c], acc);
        y[i][c] = acc / Lk[i][i];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nb * 64; e += 64) {
        const int i = e / 64, cc = e - i * 64;
        if (cbase + cc < ncols) X[(k0 + i) * ldX + cbase + cc] = y[i][cc];
    }
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
    return (size_t)n * (size_t)n * sizeof(double) + 256;
}

extern "C" int lamq_chol_inv_upper(const double* H, int64_t n, int64_t ldH, double damp, double* Hd, int64_t ldHd,
                                   double* U, int64_t ldU, uint8_t* dead, int32_t* info, void* workspace,
                                   size_t workspace_bytes, void* stream)
{
    if (!H || !U || !info || !workspace || n < 1 || ldH < n || ldU < n || (Hd && ldHd < n)) return LAMQ_EINVAL;
    if (workspace_bytes < lamq_chol_inv_upper_workspace_size(n)) return LAMQ_EINVAL;
    if (n > (int64_t)1 << 20) return LAMQ_EUNSUP;
    hipStream_t s = as_stream(stream);
    double* A = reinterpret_cast<double*>(workspace);
    double* delta = reinterpret_cast<double*>(reinterpret_cast<char*>(workspace) + (size_t)n * (size_t)n * sizeof(double));
    hipLaunchKernelGGL(diag_stats_kernel, dim3(1), dim3(256), 0, s, H, n, ldH, damp, dead, delta, info);
    LAMQ_LAUNCH_CHECK();
    const dim3 g2((unsigned)cdiv(n, 64), (unsigned)cdiv(n, 16)), b2(64, 16);
    hipLaunchKernelGGL(prep_kernel, g2, b2, 0, s, H, n, ldH, delta, A, Hd, ldHd);
    LAMQ_LAUNCH_CHECK();
    // Cholesky of A = J Hd J, lower
    for (int64_t k0 = 0; k0 < n; k0 += NBK) {
        const int nb = (int)(n - k0 < NBK ? n - k0 : NBK);
        hipLaunchKernelGGL(potf2_kernel, dim3(1), dim3(256), 0, s, A, n, k0, nb, info);
        LAMQ_LAUNCH_CHECK();
        const int64_t rest = n - k0 - nb;
        if (rest > 0) {
            hipLaunchKernelGGL(trsm_panel_kernel, dim3((unsigned)cdiv(rest, 64)), dim3(64), 0, s, A, n, k0, nb, info);
            LAMQ_LAUNCH_CHECK();
            const double* P = A + (k0 + nb) * n + k0;
            int rc = gemm_sub_f64<true, true>(A + (k0 + nb) * n + k0 + nb, n, P, n, P, n, rest, rest, nb, info, s);
            if (rc) return rc;
        }
    }
    // X = L^-1 into U (right-looking solve of L X = I)
    hipLaunchKernelGGL(identity_kernel, g2, b2, 0, s, U, n, ldU);
    LAMQ_LAUNCH_CHECK();
    for (int64_t k0 = 0; k0 < n; k0 += NBK) {
        const int nb = (int)(n - k0 < NBK ? n - k0 : NBK);
        hipLaunchKernelGGL(trsm_left_kernel, dim3((unsigned)cdiv(k0 + nb, 64)), dim3(64), 0, s, A, n, U, ldU, k0, nb, info);
        LAMQ_LAUNCH_CHECK();
        const int64_t rest = n - k0 - nb;
        if (rest > 0) {
            int rc = gemm_sub_f64<false, false>(U + (k0 + nb) * ldU, ldU, A + (k0 + nb) * n + k0, n, U + k0 * ldU, ldU, rest,
                                                k0 + nb, nb, info, s);
            if (rc) return rc;
        }
    }
    hipLaunchKernelGGL(reverse_kernel, g2, b2, 0, s, U, n, ldU, info);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
