// C -= A @ op(B) on fp64 MFMA (v_mfma_f64_16x16x4f64), the update shape shared by the lazy trailing
// refit of the sweep and by the blocked factorizations.
#pragma once
#include "common.h"

typedef double lamq_d4 __attribute__((ext_vector_type(4)));

// Workgroup tile 64x64, four waves as 2x2 wave tiles of 32x32, each 2x2 MFMA tiles of 16x16.
// MFMA operand layout (16x16x4 f64): lane l holds A[l%16][l/16], B[l/16][l%16]; the result
// lane l, register v holds D[4*v + l/16][l%16]. Each output is the sum over k as a chain of
// MFMAs from zero, then subtracted from C once: C = C - sum.
// TRANSB: op(B)[k][j] = B[j*ldb + k]; otherwise B[k*ldb + j].
// LOWER: C is a square diagonal block; tiles wholly above the diagonal are skipped and only
// entries with col <= row are written.
// OVERWRITE: C = A @ op(B) instead of C -= A @ op(B). C may then alias A (a workgroup's output rows are the rows
// it reads, when N fits one tile column) or B (its output columns are the columns it reads, when M fits one tile
// row): every wave finishes its reads before any wave writes.
template <bool TRANSB, bool LOWER, bool OVERWRITE = false>
__global__ __launch_bounds__(256) void gemm_sub_f64_kernel(double* C, int64_t ldc, const double* A, int64_t lda,
                                                           const double* B, int64_t ldb, int64_t M, int64_t N,
                                                           int64_t K, const int32_t* __restrict__ info)
{
    if (info && *info != 0) return;
    const int64_t tr = (int64_t)blockIdx.y * 64, tc = (int64_t)blockIdx.x * 64;
    if (LOWER && tc > tr + 63) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t wr = tr + (wave >> 1) * 32, wc = tc + (wave & 1) * 32;
    const int li = lane & 15, lk = lane >> 4;
    lamq_d4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = lamq_d4{0.0, 0.0, 0.0, 0.0};
    const int64_t r0 = wr + li, r1 = wr + 16 + li, c0 = wc + li, c1 = wc + 16 + li;
    const bool vr0 = r0 < M, vr1 = r1 < M, vc0 = c0 < N, vc1 = c1 < N;
    // k advances in chunks of KC = 16 (four MFMA steps); the next chunk's operands are loaded into registers
    // while the current chunk's MFMAs run, so one memory latency is paid per chunk, overlapped.
    constexpr int KC = 16;
    double pa0[4], pa1[4], pb0[4], pb1[4];
    auto load = [&](int64_t kb) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int64_t kk = kb + 4 * s + lk;
            const bool vk = kk < K;
            pa0[s] = (vr0 && vk) ? A[r0 * lda + kk] : 0.0;
            pa1[s] = (vr1 && vk) ? A[r1 * lda + kk] : 0.0;
            if (TRANSB) {
                pb0[s] = (vc0 && vk) ? B[c0 * ldb + kk] : 0.0;
                pb1[s] = (vc1 && vk) ? B[c1 * ldb + kk] : 0.0;
            } else {
                pb0[s] = (vc0 && vk) ? B[kk * ldb + c0] : 0.0;
                pb1[s] = (vc1 && vk) ? B[kk * ldb + c1] : 0.0;
            }
        }
    };
    load(0);
    for (int64_t k0 = 0; k0 < K; k0 += KC) {
        double a0[4], a1[4], b0[4], b1[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            a0[s] = pa0[s];
            a1[s] = pa1[s];
            b0[s] = pb0[s];
            b1[s] = pb1[s];
        }
        if (k0 + KC < K) load(k0 + KC);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0[s], b0[s], acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0[s], b1[s], acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1[s], b0[s], acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1[s], b1[s], acc[1][1], 0, 0, 0);
        }
    }
    if (OVERWRITE) __syncthreads();
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t row = wr + ti * 16 + 4 * v + lk;
                const int64_t col = wc + tj * 16 + li;
                if (row < M && col < N && (!LOWER || col <= row)) {
                    double* p = C + row * ldc + col;
                    if (OVERWRITE)
                        *p = acc[ti][tj][v];
                    else
                        *p = *p - acc[ti][tj][v];
                }
            }
}

template <bool TRANSB, bool LOWER, bool OVERWRITE = false>
static int gemm_sub_f64(double* C, int64_t ldc, const double* A, int64_t lda, const double* B, int64_t ldb, int64_t M,
                        int64_t N, int64_t K, const int32_t* info, hipStream_t s)
{
    if (M <= 0 || N <= 0 || K <= 0) return LAMQ_OK;
    dim3 grid((unsigned)cdiv(N, 64), (unsigned)cdiv(M, 64));
    hipLaunchKernelGGL((gemm_sub_f64_kernel<TRANSB, LOWER, OVERWRITE>), grid, dim3(256), 0, s, C, ldc, A, lda, B, ldb, M, N,
                       K, info);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
