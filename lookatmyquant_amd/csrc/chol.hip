// Damped Hessian and U = the upper Cholesky factor of its inverse (opgraph/frame.py:515-522).
//
// With J the order reversal, J Hd J = L L^T (L lower) gives Hd = V V^T with V = J L J upper, so
// Hd^-1 = V^-T V^-1 and U = V^-1 = J L^-1 J is upper with a positive diagonal: the factor
// torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(Hd)), upper=True) returns.
// One Cholesky (n^3/3 flops) and one triangular inverse (n^3/3) replace the reference's three
// factorizations (4n^3/3). Both are blocked right-looking with 64-wide panels. One workgroup factors each
// diagonal block in LDS and inverts it (Lkk^-1 kept in the workspace); the panel below, the block rows
// of the inverse and all trailing updates are then fp64 MFMA products: panel = A_panel Lkk^-T,
// X_k = Lkk^-1 B_k.
#include "gemm_f64.h"


#define NBK 64
#ifndef LAMQ_NB2
#define LAMQ_NB2 512
#endif
#define NB2 LAMQ_NB2  // panel width of the two-level blocking (a multiple of NBK)

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

// The nb x nb diagonal block at (k0, k0) of A (lower): its Cholesky factor Lkk and Lkk^-1 (lower, ld NBK, written
// into Linv), and the panel rows below it. One workgroup of four waves keeps the block's ten lower 16 x 16 tiles in
// LDS (21.8 KB: a workgroup fits on a CU beside two workgroups of the 128-tile product, which hold 128 of its 160 KB,
// so the first step of a panel need not wait for the inverse's deep product on the side stream to drain; with the
// whole 64 x 64 block, its inverse and the panel rows in LDS, 108 KB, it waited 200-350 us at n = 9,728), in four
// steps of 16 columns p:
//   (1) wave 0 factors the 16 x 16 diagonal tile D_p in registers (lane i holds row i; column values move
//       between lanes by DPP row broadcasts): column c, d = a[c][c], r = 1/sqrt(d), l[c][c] = d r, l[i][c] = a[i][c] r
//       (a reciprocal scaling, as LAPACK's unblocked potf2 scales by 1/l[c][c]), a[i][j] -= l[i][c] l[j][c];
//       then inverts the factor (lane c holds column c of D_p^-1, forward substitution with the same r) and
//       overwrites the tile with D_p^-1 (nothing reads D_p itself);
//   (2) the tiles below it become L_Ip = A_Ip D_p^-T (one MFMA tile per wave);
//   (3) the lower trailing tiles take A_IJ -= L_Ip L_Jp^T (MFMA).
// Then Lkk^-1 in place, by block rows: Linv_pq = -D_p^-1 sum_{q<=r<p} L_pr Linv_rq, one level per p (tile (p, q) holds
// L_pq until its row's level has read it). Every workgroup of the launch factors the block for itself (the same
// arithmetic, the same result) and then solves its 64 rows of the panel below the block, L_ik = A_ik Lkk^-T (MFMA, the
// rows straight from memory into the operand registers); workgroup 0 writes Lkk^-1. The panel solve thus needs no
// launch of its own after the factor. A block shorter than NBK is padded with the identity. The loops over p run at
// run time, so the code stays a few KB (a fully unrolled 64-step kernel spends most of its time fetching
// instructions).
#define DT_LD 17            // row stride of a 16 x 16 tile in LDS, in doubles
#define DT_SZ (16 * DT_LD)  // doubles of one tile

// 1/sqrt(d) for a positive normal d: the hardware estimate and two Newton steps y <- y + y (1/2 - (d/2) y^2), within
// a few units in the last place (d/2 formed once; halving is exact, so each step rounds as y + (y/2)(1 - d y^2) would)
__device__ __forceinline__ double rsqrt_f64(double d)
{
    double y = __builtin_amdgcn_rsq(d);
    const double h = 0.5 * d;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const double e = fma(-(h * y), y, 0.5);
        y = fma(y, e, y);
    }
    return y;
}

// v of lane 16 (lane / 16) + J in every lane of each row of 16 (DPP row_newbcast, one VALU move of 64 bits: no
// scalar registers, no wait states between the moves). Every lane is written, so the move has no old value to keep
// (mov_dpp: an old operand of 0 would cost a zeroing move before each broadcast)
template <int J>
__device__ __forceinline__ double row_bcast_f64(double v)
{
    return __longlong_as_double(__builtin_amdgcn_mov_dpp(__double_as_longlong(v), 0x150 + J, 0xf, 0xf, false));
}
__device__ __forceinline__ double row_bcast_f64(double v, int j)  // j a constant once the loops are unrolled
{
    switch (j) {
        case 0: return row_bcast_f64<0>(v);
        case 1: return row_bcast_f64<1>(v);
        case 2: return row_bcast_f64<2>(v);
        case 3: return row_bcast_f64<3>(v);
        case 4: return row_bcast_f64<4>(v);
        case 5: return row_bcast_f64<5>(v);
        case 6: return row_bcast_f64<6>(v);
        case 7: return row_bcast_f64<7>(v);
        case 8: return row_bcast_f64<8>(v);
        case 9: return row_bcast_f64<9>(v);
        case 10: return row_bcast_f64<10>(v);
        case 11: return row_bcast_f64<11>(v);
        case 12: return row_bcast_f64<12>(v);
        case 13: return row_bcast_f64<13>(v);
        case 14: return row_bcast_f64<14>(v);
        default: return row_bcast_f64<15>(v);
    }
}

__global__ __launch_bounds__(256) void diag_block_kernel(double* __restrict__ A, int64_t n, int64_t k0, int nb,
                                                        int64_t rest, double* __restrict__ Linv,
                                                        int32_t* __restrict__ info)
{
    __shared__ double tl[10 * DT_SZ];  // tile (I, J), J <= I, at (I (I + 1) / 2 + J) DT_SZ
    __shared__ int sfail;
    if (*info != 0) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lk = lane >> 4;
    const int64_t pr0 = k0 + nb + (int64_t)blockIdx.x * NBK;  // first panel row of this workgroup
    const int prows = (int)(rest - (int64_t)blockIdx.x * NBK < NBK ? rest - (int64_t)blockIdx.x * NBK : NBK);
    // entry (i, j) of the block, for (i, j) in a lower tile (i / 16 >= j / 16)
    auto T = [&](int i, int j) -> double& {
        return tl[((i >> 4) * ((i >> 4) + 1) / 2 + (j >> 4)) * DT_SZ + (i & 15) * DT_LD + (j & 15)];
    };
    // this wave's 16 panel rows as MFMA A operands, pa[kk] = A_rows[16 wave + li][4 kk + lk]: loaded first, used last
    double pa[16];
    {
        const int r = 16 * wave + li;
        const bool rok = r < prows;
        const double* src = A + (rok ? pr0 + r : (int64_t)0) * n + k0;
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            const int c = 4 * kk + lk;
            pa[kk] = (rok && c < nb) ? src[c] : 0.0;
        }
    }
    {  // the block's lower tiles, all loads of a thread in flight at once (rows past nb: the identity's)
        double v[NBK * NBK / 256];
#pragma unroll
        for (int q = 0; q < NBK * NBK / 256; ++q) {
            const int e = tid + 256 * q, i = e >> 6, j = e & 63;
            v[q] = (j <= i && i < nb) ? A[(k0 + i) * n + k0 + j] : 0.0;
        }
#pragma unroll
        for (int q = 0; q < NBK * NBK / 256; ++q) {
            const int e = tid + 256 * q, i = e >> 6, j = e & 63;
            if ((j >> 4) <= (i >> 4)) T(i, j) = i < nb ? v[q] : (i == j ? 1.0 : 0.0);
        }
    }
    if (tid == 0) sfail = 0;
    __syncthreads();
    for (int p = 0; p < 4; ++p) {
        const int c0 = 16 * p;
        if (wave == 0) {  // (1); lanes 16..63 repeat lanes 0..15, so a row broadcast of lane j gives row j's value
            double r[16];
            // row li of the tile, read whole: its upper part (j > li) holds finite values that are updated below but
            // never read by a pivot or a lower entry, and the store after the loop writes zeros there
#pragma unroll
            for (int j = 0; j < 16; ++j) r[j] = T(c0 + li, c0 + j);
            double rc[16];  // 1 / l[c][c], the same in every lane
            // the pivots form the serial chain; each is formed from lane-uniform values with exactly the operations
            // lane c + 1 applies to its own entry, so the chain never waits on the column's update
            double d = row_bcast_f64(r[0], 0);
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const double rs = rsqrt_f64(d);
                rc[c] = rs;
                double dn = 0.0;
                if (c < 15) {  // the next pivot: a[c+1][c+1] - l[c+1][c]^2
                    const double l1 = row_bcast_f64(r[c], c + 1) * rs;
                    dn = fma(-l1, l1, row_bcast_f64(r[c + 1], c + 1));
                }
                // l[li][c] for li >= c: lane c's own r[c] is d bit for bit (the same operations on the same operands
                // as the chain above), so its entry is d rs, the diagonal; lanes li < c compute an upper entry nothing
                // reads
                const double lic = r[c] * rs;
                r[c] = lic;
#pragma unroll
                for (int j = c + 1; j < 16; ++j) r[j] = fma(-lic, row_bcast_f64(lic, j), r[j]);
                d = dn;
            }
            if (lane < 16) {
#pragma unroll
                for (int j = 0; j < 16; ++j) T(c0 + li, c0 + j) = j <= li ? r[j] : 0.0;
            }
            // the first failing pivot, read off the diagonal once: l[c][c] = d rs is positive for a positive finite d,
            // and NaN for a pivot that is not (rs is NaN for d < 0 and infinite for d = 0, and an earlier failure
            // leaves every later pivot NaN), so the lowest lane of the 16 whose diagonal is not positive names it
            const double diag = T(c0 + li, c0 + li);
            const uint64_t badl = __builtin_amdgcn_ballot_w64(!(diag > 0.0)) & 0xffffull;
            const int fail = badl ? (int)(k0 + c0 + __builtin_ctzll(badl) + 1) : 0;
            // the inverse reads the factor back from LDS (the same value in every lane), lane c holding column c of
            // D_p^-1 (x[i] = D_p^-1[i][c]); a wave's LDS accesses take effect in the order it issues them, so the tile
            // can then become D_p^-1 (nothing reads D_p itself)
            double x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = i == li ? 1.0 : 0.0;
#pragma unroll
            for (int l = 0; l < 16; ++l) {
                x[l] = x[l] * rc[l];
#pragma unroll
                for (int i = l + 1; i < 16; ++i) x[i] = fma(-T(c0 + i, c0 + l), x[l], x[i]);
            }
            if (lane < 16) {
#pragma unroll
                for (int i = 0; i < 16; ++i) T(c0 + i, c0 + li) = x[i];
            }
            if (lane == 0 && fail != 0) sfail = fail;
        }
        __syncthreads();
        if (sfail != 0) {  // uniform: every thread leaves
            if (tid == 0) *info = sfail;
            return;
        }
        // (2) wave w: tile I = p + 1 + w. MFMA 16x16x4 operands: lane l gives A[l % 16][k4 + l / 16] and
        // B[k4 + l / 16][l % 16]; result register v of lane l is row 4v + l / 16, column l % 16.
        {
            const int I = p + 1 + wave;
            if (I < 4) {
                lamq_d4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(T(16 * I + li, c0 + 4 * kk + lk),
                                                               T(c0 + li, c0 + 4 * kk + lk), acc, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v) T(16 * I + 4 * v + lk, c0 + li) = acc[v];
            }
        }
        __syncthreads();
        // (3) tiles (I, J), p < J <= I < 4, round-robin over the waves
        {
            const int m = 3 - p;
            const int nt = m * (m + 1) / 2;
            for (int t = wave; t < nt; t += 4) {
                int ii = 0, jj = t;
                while (jj > ii) {
                    jj -= ii + 1;
                    ++ii;
                }
                const int I = p + 1 + ii, J = p + 1 + jj;
                lamq_d4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(T(16 * I + li, c0 + 4 * kk + lk),
                                                               T(16 * J + li, c0 + 4 * kk + lk), acc, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v) T(16 * I + 4 * v + lk, 16 * J + li) -= acc[v];
            }
        }
        __syncthreads();
    }
    // Lkk^-1 below the diagonal tiles: level p, wave q < p; tile (p, q) is overwritten only once every wave of the
    // level has read row p's tiles of L
    for (int p = 1; p < 4; ++p) {
        const int q = wave;
        lamq_d4 o = {0.0, 0.0, 0.0, 0.0};
        if (q < p) {
            lamq_d4 t = {0.0, 0.0, 0.0, 0.0};
            for (int r = q; r < p; ++r) {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    t = __builtin_amdgcn_mfma_f64_16x16x4f64(T(16 * p + li, 16 * r + 4 * kk + lk),
                                                             T(16 * r + 4 * kk + lk, 16 * q + li), t, 0, 0, 0);
            }
            // the result layout of t is the B-operand layout of its k-steps: register kk holds rows 4kk + l / 16
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                o = __builtin_amdgcn_mfma_f64_16x16x4f64(T(16 * p + li, 16 * p + 4 * kk + lk), t[kk], o, 0, 0, 0);
        }
        __syncthreads();
        if (q < p) {
#pragma unroll
            for (int v = 0; v < 4; ++v) T(16 * p + 4 * v + lk, 16 * q + li) = -o[v];
        }
        __syncthreads();
    }
    // the panel rows: P = A_rows Lkk^-T, wave w rows 16w..16w+15, four column tiles (B[k][j] = Lkk^-1[j][k], zero for
    // k / 16 > j / 16; past nb the rows hold zeros and Lkk^-1 the identity)
    if (prows > 0) {
        lamq_d4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = lamq_d4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if ((kk >> 2) <= t)
                    acc[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(pa[kk], T(16 * t + li, 4 * kk + lk), acc[t], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = 16 * wave + 4 * v + lk, c = 16 * t + li;
                if (r < prows && c < nb) A[(pr0 + r) * n + k0 + c] = acc[t][v];
            }
    }
    // Lkk itself is not written back: nothing after this launch reads it (the panel, the updates and the inverse use
    // the panel rows and Lkk^-1), and the other workgroups of this launch read the block as it was, so writing it in
    // place would race with them
    if (blockIdx.x != 0) return;
    for (int e = tid; e < NBK * NBK; e += 256) {
        const int i = e >> 6, j = e & 63;
        Linv[i * NBK + j] = j <= i ? T(i, j) : 0.0;
    }
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

// The blocked steps of the factorization (stream s) and of the inverse (stream si, which may be s: then the step
// events are not used).
static int chol_steps(double* A, int64_t n, double* Linv, double* U, int64_t ldU, int32_t* info, hipStream_t s,
                      hipStream_t si, hipEvent_t step)
{
    // Cholesky of A = J Hd J, lower, in panels of NB2 columns: inside a panel, 64-wide steps update only the panel's
    // own columns; the columns after it get one product of depth NB2 per panel.
    // X = L^-1 into U (right-looking solve of L X = I): X_k = Lkk^-1 B_k, then B_i -= L_ik X_k below, inside the
    // panel at once and below it once per panel (X is lower triangular, so the panel's rows are zero right of
    // their diagonal and one product of depth NB2 carries the panel's steps).
    // The inverse's step k needs Lkk^-1 and the panel L_ik of the factor's step k, nothing the factor writes later: on a
    // side stream it follows the factor one step behind (an event after each step's diagonal block).
    auto inverse_step = [&](int64_t k0, int64_t pe) -> int {
        const int nb = (int)(n - k0 < NBK ? n - k0 : NBK);
        const double* Lk = Linv + (k0 / NBK) * NBK * NBK;
        const double* P = A + (k0 + nb) * n + k0;
        const int64_t pc = pe - (k0 + nb);
        int rc = gemm_sub_f64<false, false, true>(U + k0 * ldU, ldU, Lk, NBK, U + k0 * ldU, ldU, nb, k0 + nb, nb, info, si);
        if (rc || pc <= 0) return rc;
        return gemm_sub_f64<false, false>(U + (k0 + nb) * ldU, ldU, P, n, U + k0 * ldU, ldU, pc, k0 + nb, nb, info, si);
    };
    for (int64_t K0 = 0; K0 < n; K0 += NB2) {
        const int64_t pe = (K0 + NB2 < n) ? K0 + NB2 : n;
        for (int64_t k0 = K0; k0 < pe; k0 += NBK) {
            const int nb = (int)(n - k0 < NBK ? n - k0 : NBK);
            double* Lk = Linv + (k0 / NBK) * NBK * NBK;
            const int64_t rest = n - k0 - nb;
            double* P = A + (k0 + nb) * n + k0;
            // the factor of the diagonal block and the panel below it (P = P Lkk^-T): every workgroup factors the
            // block for itself and solves 64 rows of the panel
            const unsigned pg = rest > 0 ? (unsigned)cdiv(rest, NBK) : 1u;
            hipLaunchKernelGGL(diag_block_kernel, dim3(pg), dim3(256), 0, s, A, n, k0, nb, rest, Lk, info);
            LAMQ_LAUNCH_CHECK();
            if (si != s) {
                LAMQ_HIP_CHECK(hipEventRecord(step, s));
                LAMQ_HIP_CHECK(hipStreamWaitEvent(si, step, 0));
            }
            const int64_t pc = pe - (k0 + nb);
            if (rest > 0 && pc > 0) {
                int rc = gemm_sub_f64<true, true>(A + (k0 + nb) * n + k0 + nb, n, P, n, P, n, rest, pc, nb, info, s);
                if (rc) return rc;
            }
            int rc = inverse_step(k0, pe);
            if (rc) return rc;
        }
        const int64_t rest = n - pe;
        if (rest > 0) {
            const double* P = A + pe * n + K0;
            int rc = gemm_sub_f64<true, true>(A + pe * n + pe, n, P, n, P, n, rest, rest, pe - K0, info, s);
            if (rc) return rc;
            rc = gemm_sub_f64<false, false>(U + pe * ldU, ldU, P, n, U + K0 * ldU, ldU, rest, pe, pe - K0, info, si);
            if (rc) return rc;
        }
    }
    return LAMQ_OK;
}

extern "C" size_t lamq_chol_inv_upper_workspace_size(int64_t n)
{
    if (n < 1) return 0;
    // J Hd J and its factor, the inverses of the diagonal blocks, the damping scalar
    return (size_t)n * (size_t)n * sizeof(double) + (size_t)cdiv(n, NBK) * NBK * NBK * sizeof(double) + 256;
}

// Events of one factorization whose inverse runs on a side stream, made and released by the call (the library keeps
// no state between calls). A released event that is still recorded on a stream lives until the stream reaches it.
// The step event orders the two streams of one device, so it records with a device-scope fence only: a system-scope
// release (HIP's default) writes the caches back and costs about 6 us between a step's kernels, once per 64 columns.
// The fork and join events (once a call) keep the default.
static constexpr unsigned kStepEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;
struct CholEvents {
    hipEvent_t fork = nullptr, step = nullptr, join = nullptr;
    ~CholEvents()
    {
        if (fork) (void)hipEventDestroy(fork);
        if (step) (void)hipEventDestroy(step);
        if (join) (void)hipEventDestroy(join);
    }
};

extern "C" int lamq_chol_inv_upper_ex(const double* H, int64_t n, int64_t ldH, double damp, int flags, double* Hd,
                                      int64_t ldHd, double* U, int64_t ldU, uint8_t* dead, int32_t* info, void* workspace,
                                      size_t workspace_bytes, void* stream, void* side_stream)
{
    if (!H || !U || !info || !workspace || n < 1 || ldH < n || ldU < n || (Hd && ldHd < n)) return LAMQ_EINVAL;
    if (flags & ~LAMQ_CHOL_KEEP_DEAD) return LAMQ_EINVAL;
    const int keep_dead = (flags & LAMQ_CHOL_KEEP_DEAD) ? 1 : 0;
    if (workspace_bytes < lamq_chol_inv_upper_workspace_size(n)) return LAMQ_EINVAL;
    if (n > (int64_t)1 << 20) return LAMQ_EUNSUP;
    hipStream_t s = as_stream(stream);
    hipStream_t si = side_stream ? as_stream(side_stream) : s;
    const bool fork = si != s;
    CholEvents ev;
    if (fork) {
        LAMQ_HIP_CHECK(hipEventCreateWithFlags(&ev.fork, hipEventDisableTiming));
        LAMQ_HIP_CHECK(hipEventCreateWithFlags(&ev.step, kStepEventFlags));
        LAMQ_HIP_CHECK(hipEventCreateWithFlags(&ev.join, hipEventDisableTiming));
    }
    double* A = reinterpret_cast<double*>(workspace);
    double* Linv = A + n * n;  // cdiv(n, NBK) blocks of NBK x NBK
    double* delta = Linv + cdiv(n, NBK) * NBK * NBK;
    hipLaunchKernelGGL(diag_stats_kernel, dim3(1), dim3(256), 0, s, H, n, ldH, damp, keep_dead, dead, delta, info);
    LAMQ_LAUNCH_CHECK();
    const dim3 g2((unsigned)cdiv(n, 64), (unsigned)cdiv(n, 16)), b2(64, 16);
    hipLaunchKernelGGL(prep_kernel, g2, b2, 0, s, H, n, ldH, delta, keep_dead, A, Hd, ldHd);
    LAMQ_LAUNCH_CHECK();
    // The inverse X = L^-1 runs on the side stream (when one is given), one 64-column step behind the factorization:
    // its step k needs Lkk^-1 and the panel L_ik of the factor's step k (an event after that step's panel solve),
    // nothing the factor writes later. The factor's in-panel and trailing updates and the inverse's products then
    // overlap. Without a side stream both run in order on the caller's stream.
    if (fork) {
        LAMQ_HIP_CHECK(hipEventRecord(ev.fork, s));
        LAMQ_HIP_CHECK(hipStreamWaitEvent(si, ev.fork, 0));
    }
    hipLaunchKernelGGL(identity_kernel, g2, b2, 0, si, U, n, ldU);
    LAMQ_LAUNCH_CHECK();
    int rc = chol_steps(A, n, Linv, U, ldU, info, s, si, ev.step);
    if (fork) {
        // the caller's stream waits for the side stream, also after a failed launch
        const hipError_t e1 = hipEventRecord(ev.join, si);
        const hipError_t e2 = e1 == hipSuccess ? hipStreamWaitEvent(s, ev.join, 0) : e1;
        if (rc) return rc;
        if (e2 != hipSuccess) return (int)e2;
    }
    if (rc) return rc;
    hipLaunchKernelGGL(reverse_kernel, g2, b2, 0, s, U, n, ldU, info);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

extern "C" int lamq_chol_inv_upper(const double* H, int64_t n, int64_t ldH, double damp, double* Hd, int64_t ldHd,
                                   double* U, int64_t ldU, uint8_t* dead, int32_t* info, void* workspace,
                                   size_t workspace_bytes, void* stream)
{
    return lamq_chol_inv_upper_ex(H, n, ldH, damp, 0, Hd, ldHd, U, ldU, dead, info, workspace, workspace_bytes, stream,
                                  nullptr);
}
