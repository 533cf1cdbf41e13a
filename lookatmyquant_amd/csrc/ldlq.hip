// Width-1 block-LDLQ onto a scalar set, the lazy trailing update, and dead-column zeroing.
#include "gemm_f64.h"

// ------------------------------------------------------------------------------------------------
// ldlq_scalar_block: one wave per row walks the columns of the lazy block [b0, b1), b1-b0 <= 128;
// lane c holds columns b0+c and b0+64+c of the row in registers.
//   mode 0 (opgraph/nested.py:127-140): t = T[j] (T is X/S), index = first argmin_i (t - lv_i)^2,
//          q = lv[index]
//   mode 1 (opgraph/codes.py:322-332, 442-450): index = bucketize(t/S, midpoints) (halfway to the
//          lower level), q = lv[index]*S
//   z = (t - q) / U[j][j];  T[col] = T[col] - z*U[j][col] for col in (j, b1)   (syntax.py:117-121,
//   a K = 1 product: rounded, then subtracted)
// The columns are a chain (each z needs the refits of all before it), so a step's cost is its latency: the upper
// triangle of the block's diagonal part of U, U[b0:b1, b0:b1], is staged in LDS once per workgroup of R rows (one
// wave each; 66 KB, two workgroups a CU), and each step reads its U row and diagonal from there instead of from
// memory. R = 4 while the rows fill the CUs four at a time; past that 8 or 16 rows share a workgroup, so that each
// SIMD interleaves up to eight rows' chains.
// ------------------------------------------------------------------------------------------------
#define SC_MAXW 128
// row r of the staged triangle (columns r .. SC_MAXW - 1) starts at sc_tri(r)
__host__ __device__ constexpr int sc_tri(int r) { return r * SC_MAXW - r * (r - 1) / 2; }
#define SC_REGK 16  // level sets up to this size are searched from registers
template <bool B>
struct BoolC {
    static constexpr bool value = B;
};
template <int I>
struct IntK {
    static constexpr int value = I;
};
// P: 0 (levels read from LDS), or a power of two >= K (levels held in registers, P of them)
template <int P, int R, int MODE>
__global__ __launch_bounds__(64 * R) void ldlq_scalar_block_kernel(const double* __restrict__ T, int64_t m, int64_t ldT,
                                                                const double* __restrict__ U, int64_t ldU,
                                                                const double* __restrict__ S,
                                                                const double* __restrict__ levels, int K,
                                                                int64_t b0, int64_t b1, int32_t* __restrict__ idx,
                                                                int64_t ldi, double* __restrict__ Z, int64_t ldZ)
{
    __shared__ double ub[sc_tri(SC_MAXW)];  // U[b0 + r][b0 + c], c >= r, at sc_tri(r) + c - r
    __shared__ double lv[256];
    __shared__ double mid[256];
    const int bw = (int)(b1 - b0);
    constexpr int NTH = 64 * R;
    for (int i = threadIdx.x; i < K; i += NTH) lv[i] = levels[i];
    // eight loads in flight per thread before their stores (each store waits for its load); element e of the staged
    // block is row e / SC_MAXW, column e % SC_MAXW
    for (int e0 = threadIdx.x; e0 < bw * SC_MAXW; e0 += NTH * 8) {
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = e0 + NTH * u, r = e / SC_MAXW, c = e % SC_MAXW;
            v[u] = (r < bw && c < bw && c >= r) ? U[(b0 + r) * ldU + b0 + c] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = e0 + NTH * u, r = e / SC_MAXW, c = e % SC_MAXW;
            if (e < bw * SC_MAXW && c >= r) ub[sc_tri(r) + c - r] = v[u];
        }
    }
    __syncthreads();
    if constexpr (MODE == 1) {
        for (int i = threadIdx.x; i + 1 < K; i += NTH) mid[i] = (lv[i + 1] + lv[i]) / 2;
        __syncthreads();
    }
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * R + (threadIdx.x >> 6);
    if (row >= m) return;
    // up to P levels and midpoints in registers (the same values in every lane)
    constexpr bool REG = P > 0;
    constexpr int NR = REG ? P : 1;
    double lr[NR], mr[NR];
    if (REG) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            if (MODE == 0) lr[i] = i < K ? lv[i] : 0.0;
            if (MODE == 1) mr[i] = i + 1 < K ? mid[i] : __builtin_inf();
        }
    }
    const double* Tr = T + row * ldT + b0;
    double t0 = lane < bw ? Tr[lane] : 0.0;
    double t1 = lane + 64 < bw ? Tr[lane + 64] : 0.0;
    const double Sr = MODE == 1 ? S[row] : 1.0;
    // the U row a step uses (its diagonal and this lane's two columns) is read one step ahead, off the chain of
    // dependent operations; entries left of the diagonal are read too (inside the staged triangle) and not used
    const auto urow = [&](int c, double& ud, double& u0, double& u1) {
        const double* Uj = ub + sc_tri(c) - c;  // Uj[col] = U[b0 + c][b0 + col] for col >= c
        ud = Uj[c];
        u0 = Uj[lane];
        u1 = Uj[lane + 64];
    };
    if constexpr (MODE == 0 && REG) {
        // The search from registers: levels past K are +inf (distance +inf, never strictly below another), so no
        // step needs K
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            lr[i] = i < K ? lr[i] : __builtin_inf();
            // held as vector registers (opaque to the uniformity analysis): the tournament's selects are then
            // v_cndmask on the compares' lane masks, not scalar selects fed back and forth between the vector and
            // scalar units
            asm volatile("" : "+v"(lr[i]));
        }
        // z = (t - q) / U[j][j] through the hardware division's own sequence split at its divisor: the reciprocal
        // refinement of U[j][j] (it depends on the divisor alone) before the steps, then on the chain the quotient
        // q0 = E r, the exact residual fma(-d, q0, E) and the corrected quotient: the values the division E / d forms
        // wherever its operand scaling is the identity and its final fix-up passes the quotient through, as for every
        // divisor and nonzero residual within 2^-300 .. 2^300. Divisors outside that range send the block to the plain
        // division below before it starts; a residual outside it (zero and subnormal included) is noted (the
        // extremes of its biased exponents, no branch on the chain) and the block is then done again with the plain
        // division.
        const auto recip = [](double d) {
            double r = __builtin_amdgcn_rcp(d);
            r = fma(r, fma(-d, r, 1.0), r);
            r = fma(r, fma(-d, r, 1.0), r);
            return r;
        };
        const auto in_range = [](double v) {
            const double a = __builtin_fabs(v);
            return a >= 0x1p-300 && a <= 0x1p300;
        };
        // every divisor U[j][j] of the block and its reciprocal, formed before the steps: lane l holds those of
        // columns l and l + 64, and step c reads them with readlane (no step waits on the reciprocal's chain)
        const double dg0 = lane < bw ? ub[sc_tri(lane)] : 1.0;
        const double dg1 = lane + 64 < bw ? ub[sc_tri(lane + 64)] : 1.0;
        const double rc0 = recip(dg0), rc1 = recip(dg1);
        const bool dg_ok = __builtin_amdgcn_ballot_w64(!(in_range(dg0) && in_range(dg1))) == 0;
        if (dg_ok) {
            double zk0 = 0.0, zk1 = 0.0;  // z of this lane's columns (lane, lane + 64)
            int ik0 = 0, ik1 = 0;
            uint32_t bmin = 0x7FFu, bmax = 0u;  // extremes of the residuals' biased binary exponents
            // the U row of step c + 2 is read from LDS during step c (its two columns of each lane), into a ring of
            // three register pairs: step c's row in slot c % 3 (the steps unrolled by three, so no row is moved)
            double us[3][2];
            const auto urow2 = [&](int c, double (&u)[2]) {
                const double* Uj = ub + sc_tri(c) - c;
                u[0] = Uj[lane];
                u[1] = Uj[lane + 64];
            };
            urow2(0, us[0]);
            urow2(bw > 1 ? 1 : 0, us[1]);
            // step c: a tournament over the squared distances with strict comparisons, the left (lower) index keeping
            // a tie: the first argmin, as the sequential scan finds it (a NaN t: index 0, as the reference's argmin);
            // the winner's index (the same in every lane) then reads its level from the register array. LO: columns
            // below 64 still open (their lanes' first registers take the refit).
            const auto step = [&](auto slot_c, auto lo_c, const int c) {
                constexpr int SL = decltype(slot_c)::value;
                constexpr bool LO = decltype(lo_c)::value;
                const double t = LO ? readlane_f64(t0, c) : readlane_f64(t1, c - 64);
                const double ud = LO ? readlane_f64(dg0, c) : readlane_f64(dg1, c - 64);
                const double rd = LO ? readlane_f64(rc0, c) : readlane_f64(rc1, c - 64);
                const double u0 = us[SL][0], u1 = us[SL][1];
                if (c + 2 < bw) urow2(c + 2, us[(SL + 2) % 3]);
                double d[NR];
                int bi[NR];
#pragma unroll
                for (int i = 0; i < NR; ++i) {
                    const double e = t - lr[i];
                    d[i] = e * e;
                    bi[i] = i;
                }
#pragma unroll
                for (int span = 1; span < NR; span *= 2)
#pragma unroll
                    for (int i = 0; i + span < NR; i += 2 * span)
                        if (d[i + span] < d[i]) {
                            d[i] = d[i + span];
                            bi[i] = bi[i + span];
                        }
                const int best = __builtin_amdgcn_readfirstlane(bi[0]);
                const double E = t - lr[best];
                const double q0 = E * rd;
                const double r = fma(-ud, q0, E);
                // div_fmas without its scaling flag is this fma, and div_fixup returns the quotient unchanged for
                // finite operands whose quotient neither overflows nor underflows (both within 2^-300 .. 2^300)
                const double zj = fma(r, rd, q0);
                const uint32_t be = ((uint32_t)(__double_as_longlong(E) >> 52)) & 0x7FFu;  // 0: zero or subnormal
                bmin = be < bmin ? be : bmin;
                bmax = be > bmax ? be : bmax;
                // every lane's open columns take the refit: those at or left of c are settled and those past the
                // block unused, so their values (formed from entries of the staged triangle outside this row) are
                // never read
                if constexpr (LO) {
                    const double p0 = zj * u0;
                    t0 = t0 - p0;
                }
                {
                    const double p1 = zj * u1;
                    t1 = t1 - p1;
                }
                if constexpr (LO) {
                    zk0 = lane == c ? zj : zk0;
                    ik0 = lane == c ? best : ik0;
                } else {
                    zk1 = lane + 64 == c ? zj : zk1;
                    ik1 = lane + 64 == c ? best : ik1;
                }
            };
            // steps cb .. ce - 1 (slot c % 3 for step c)
            const auto run = [&](const int cb, const int ce, auto lo_c) {
                int c = cb;
                for (; c < ce && c % 3 != 0; ++c) {
                    if (c % 3 == 1)
                        step(IntK<1>{}, lo_c, c);
                    else
                        step(IntK<2>{}, lo_c, c);
                }
                for (; c + 3 <= ce; c += 3) {
                    step(IntK<0>{}, lo_c, c);
                    step(IntK<1>{}, lo_c, c + 1);
                    step(IntK<2>{}, lo_c, c + 2);
                }
                for (; c < ce; ++c) {
                    if (c % 3 == 0)
                        step(IntK<0>{}, lo_c, c);
                    else if (c % 3 == 1)
                        step(IntK<1>{}, lo_c, c);
                    else
                        step(IntK<2>{}, lo_c, c);
                }
            };
            run(0, bw < 64 ? bw : 64, BoolC<true>{});
            run(64, bw, BoolC<false>{});
            // every |E| in 2^-300 .. 2^300 (biased exponent 723 .. 1322): no zero, subnormal or extreme residual
            if (bmin >= 723u && bmax <= 1322u) {
                if (lane < bw) {
                    idx[row * ldi + b0 + lane] = ik0;
                    Z[row * ldZ + lane] = zk0;
                }
                if (lane + 64 < bw) {
                    idx[row * ldi + b0 + lane + 64] = ik1;
                    Z[row * ldZ + lane + 64] = zk1;
                }
                return;
            }
            // a residual out of the fast quotient's range: the block again with the plain division
            t0 = lane < bw ? Tr[lane] : 0.0;
            t1 = lane + 64 < bw ? Tr[lane + 64] : 0.0;
        }
    }
    double ud_n, u0_n, u1_n;
    urow(0, ud_n, u0_n, u1_n);
    for (int c = 0; c < bw; ++c) {
        const double ud = ud_n, u0 = u0_n, u1 = u1_n;
        if (c + 1 < bw) urow(c + 1, ud_n, u0_n, u1_n);
        const double t = c < 64 ? readlane_f64(t0, c) : readlane_f64(t1, c - 64);
        int best = 0;
        double q;
        if constexpr (MODE == 0) {
            const double d0 = t - lv[0];
            double bd = d0 * d0;
            for (int i = 1; i < K; ++i) {
                double d = t - lv[i];
                d = d * d;
                if (d < bd) { bd = d; best = i; }
            }
            q = lv[best];
        } else {
            const double ts = t / Sr;
            if (REG) {
                // bucketize on the midpoints: the midpoints passed before the first that ts does not exceed (halfway
                // goes to the lower level), as the scan below counts them
                bool up = true;
#pragma unroll
                for (int i = 0; i + 1 < NR; ++i) {
                    up = up && ts > mr[i];
                    best += up ? 1 : 0;
                }
            } else {
                while (best < K - 1 && ts > mid[best]) ++best;
            }
            q = lv[best] * Sr;
        }
        const int64_t j = b0 + c;
        const double zj = (t - q) / ud;
        if (lane > c && lane < bw) {
            const double p = zj * u0;
            t0 = t0 - p;
        }
        if (lane + 64 > c && lane + 64 < bw) {
            const double p = zj * u1;
            t1 = t1 - p;
        }
        if (lane == (c & 63)) {
            idx[row * ldi + j] = best;
            Z[row * ldZ + c] = zj;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// ldlq_multirate_block: the same sweep for R rates at once (opgraph/nested.py:104-147 without output shaping). The
// rates' copies of the rows are stacked rate-major in T and Z (copy r of row i is row r*m + i, as X.repeat(R, 1)); one
// wave takes row i and its R copies, lane c holding columns b0+c and b0+64+c of each. Per column one index for all
// copies: first argmin_i sum_r w_r (t_r - tab[r][i])^2, each term w_r times the rounded square, summed in rate order;
// then copy r settles on tab[r][index] and is refit for its own error: z_r = (t_r - tab[r][index]) / U[j][j],
// T_r[col] -= z_r U[j][col]. U == NULL: no refit (every column alone, the sweep without H).
// ------------------------------------------------------------------------------------------------
#define MR_MAXR 4
template <int R>
__global__ __launch_bounds__(256) void ldlq_multirate_block_kernel(const double* __restrict__ T, int64_t m, int64_t ldT,
                                                                   const double* __restrict__ U, int64_t ldU,
                                                                   const double* __restrict__ tables, int K,
                                                                   const double* __restrict__ weights, int64_t b0,
                                                                   int64_t b1, int32_t* __restrict__ idx, int64_t ldi,
                                                                   double* __restrict__ Z, int64_t ldZ)
{
    __shared__ double ub[sc_tri(SC_MAXW)];
    __shared__ double tab[MR_MAXR * 256];
    const int bw = (int)(b1 - b0);
    for (int i = threadIdx.x; i < R * K; i += 256) tab[i] = tables[i];
    if (U) {
        for (int e0 = threadIdx.x; e0 < bw * SC_MAXW; e0 += 256 * 8) {
            double v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int e = e0 + 256 * u, r = e / SC_MAXW, c = e % SC_MAXW;
                v[u] = (r < bw && c < bw && c >= r) ? U[(b0 + r) * ldU + b0 + c] : 0.0;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int e = e0 + 256 * u, r = e / SC_MAXW, c = e % SC_MAXW;
                if (e < bw * SC_MAXW && c >= r) ub[sc_tri(r) + c - r] = v[u];
            }
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    double w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = weights[r];
    double t0[R], t1[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const double* Tr = T + (r * m + row) * ldT + b0;
        t0[r] = lane < bw ? Tr[lane] : 0.0;
        t1[r] = lane + 64 < bw ? Tr[lane + 64] : 0.0;
    }
    for (int c = 0; c < bw; ++c) {
        double t[R];
#pragma unroll
        for (int r = 0; r < R; ++r) t[r] = c < 64 ? readlane_f64(t0[r], c) : readlane_f64(t1[r], c - 64);
        int best = 0;
        double bc = 0.0;
        for (int i = 0; i < K; ++i) {
            double cost = 0.0;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const double d = t[r] - tab[r * K + i];
                const double p = w[r] * (d * d);
                cost = r == 0 ? p : cost + p;
            }
            if (i == 0 || cost < bc) {
                bc = cost;
                best = i;
            }
        }
        const int64_t j = b0 + c;
        if (lane == (c & 63)) idx[row * ldi + j] = best;
        if (!U) continue;
        const double* Uj = ub + sc_tri(c) - c;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const double zr = (t[r] - tab[r * K + best]) / Uj[c];
            if (lane > c && lane < bw) {
                const double pr = zr * Uj[lane];
                t0[r] = t0[r] - pr;
            }
            if (lane + 64 > c && lane + 64 < bw) {
                const double pr = zr * Uj[lane + 64];
                t1[r] = t1[r] - pr;
            }
            if (lane == (c & 63)) Z[(r * m + row) * ldZ + c] = zr;
        }
    }
}

extern "C" int lamq_ldlq_multirate_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                         const double* tables, int R, int K, const double* weights, int64_t b0,
                                         int64_t b1, int32_t* idx, int64_t ldi, double* Z, int64_t ldZ, void* stream)
{
    if (!T || !tables || !weights || !idx || (U && !Z)) return LAMQ_EINVAL;
    if (m < 0 || n < 1 || ldT < n || (U && ldU < n) || ldi < n || b0 < 0 || b1 <= b0 || b1 > n || K < 1 || K > 256)
        return LAMQ_EINVAL;
    if (U && ldZ < b1 - b0) return LAMQ_EINVAL;
    if (R < 1 || R > MR_MAXR) return LAMQ_EUNSUP;
    if (b1 - b0 > SC_MAXW) return LAMQ_EUNSUP;
    if (m == 0) return LAMQ_OK;
    const dim3 grid((unsigned)cdiv(m, 4));
    hipStream_t s = as_stream(stream);
    switch (R) {
    case 1: hipLaunchKernelGGL(ldlq_multirate_block_kernel<1>, grid, dim3(256), 0, s, T, m, ldT, U, ldU, tables, K, weights, b0, b1, idx, ldi, Z, ldZ); break;
    case 2: hipLaunchKernelGGL(ldlq_multirate_block_kernel<2>, grid, dim3(256), 0, s, T, m, ldT, U, ldU, tables, K, weights, b0, b1, idx, ldi, Z, ldZ); break;
    case 3: hipLaunchKernelGGL(ldlq_multirate_block_kernel<3>, grid, dim3(256), 0, s, T, m, ldT, U, ldU, tables, K, weights, b0, b1, idx, ldi, Z, ldZ); break;
    default: hipLaunchKernelGGL(ldlq_multirate_block_kernel<4>, grid, dim3(256), 0, s, T, m, ldT, U, ldU, tables, K, weights, b0, b1, idx, ldi, Z, ldZ); break;
    }
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

template <int P, int MODE>
static int scalar_launch_r(int R, const double* T, int64_t m, int64_t ldT, const double* U, int64_t ldU,
                           const double* S, const double* levels, int K, int64_t b0, int64_t b1, int32_t* idx,
                           int64_t ldi, double* Z, int64_t ldZ, hipStream_t s)
{
    if (R == 16)
        hipLaunchKernelGGL((ldlq_scalar_block_kernel<P, 16, MODE>), dim3((unsigned)cdiv(m, 16)), dim3(1024), 0, s, T, m,
                           ldT, U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ);
    else if (R == 8)
        hipLaunchKernelGGL((ldlq_scalar_block_kernel<P, 8, MODE>), dim3((unsigned)cdiv(m, 8)), dim3(512), 0, s, T, m, ldT,
                           U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ);
    else
        hipLaunchKernelGGL((ldlq_scalar_block_kernel<P, 4, MODE>), dim3((unsigned)cdiv(m, 4)), dim3(256), 0, s, T, m, ldT,
                           U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

template <int MODE>
static int scalar_launch_p(int P, int R, const double* T, int64_t m, int64_t ldT, const double* U, int64_t ldU,
                           const double* S, const double* levels, int K, int64_t b0, int64_t b1, int32_t* idx,
                           int64_t ldi, double* Z, int64_t ldZ, hipStream_t s)
{
    switch (P) {
    case 2: return scalar_launch_r<2, MODE>(R, T, m, ldT, U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ, s);
    case 4: return scalar_launch_r<4, MODE>(R, T, m, ldT, U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ, s);
    case 8: return scalar_launch_r<8, MODE>(R, T, m, ldT, U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ, s);
    case SC_REGK: return scalar_launch_r<SC_REGK, MODE>(R, T, m, ldT, U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ, s);
    default: return scalar_launch_r<0, MODE>(R, T, m, ldT, U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ, s);
    }
}

static int scalar_launch(int P, int R, const double* T, int64_t m, int64_t ldT, const double* U, int64_t ldU,
                         const double* S, const double* levels, int K, int mode, int64_t b0, int64_t b1, int32_t* idx,
                         int64_t ldi, double* Z, int64_t ldZ, hipStream_t s)
{
    if (mode == 0) return scalar_launch_p<0>(P, R, T, m, ldT, U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ, s);
    return scalar_launch_p<1>(P, R, T, m, ldT, U, ldU, S, levels, K, b0, b1, idx, ldi, Z, ldZ, s);
}

extern "C" int lamq_ldlq_scalar_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                      const double* S, const double* levels, int K, int mode, int64_t b0, int64_t b1,
                                      int32_t* idx, int64_t ldi, double* Z, int64_t ldZ, void* stream)
{
    if (!T || !U || !levels || !idx || !Z || (mode == 1 && !S) || (mode != 0 && mode != 1)) return LAMQ_EINVAL;
    if (m < 0 || n < 1 || ldT < n || ldU < n || ldi < n || b0 < 0 || b1 <= b0 || b1 > n || K < 1 || K > 256)
        return LAMQ_EINVAL;
    if (ldZ < b1 - b0) return LAMQ_EINVAL;
    if (b1 - b0 > SC_MAXW) return LAMQ_EUNSUP;
    if (m == 0) return LAMQ_OK;
    // rows per workgroup: as many as keep at least 256 workgroups (one per CU), between 4 and 16
    const int R = m >= 16 * 256 ? 16 : (m >= 8 * 256 ? 8 : 4);
    const int P = K <= 2 ? 2 : (K <= 4 ? 4 : (K <= 8 ? 8 : (K <= SC_REGK ? SC_REGK : 0)));
    return scalar_launch(P, R, T, m, ldT, U, ldU, S, levels, K, mode, b0, b1, idx, ldi, Z, ldZ, as_stream(stream));
}

extern "C" int lamq_trailing_update_f64(double* T, int64_t m, int64_t n, int64_t ldT, const double* Z, int64_t ldZ,
                                        const double* U, int64_t ldU, int64_t b0, int64_t b1, void* stream)
{
    if (!T || !Z || !U || m < 0 || n < 1 || ldT < n || ldU < n || b0 < 0 || b1 <= b0 || b1 > n || ldZ < b1 - b0)
        return LAMQ_EINVAL;
    if (b1 - b0 > 1024) return LAMQ_EUNSUP;
    if (m == 0 || b1 == n) return LAMQ_OK;
    return gemm_sub_f64<false, false>(T + b1, ldT, Z, ldZ, U + b0 * ldU + b1, ldU, m, n - b1, b1 - b0, nullptr,
                                      as_stream(stream));
}

// C -= A op(B), fp64, with op(B) optionally triangular (tri 1: op(B)[k][j] = 0 for k < j; tri 2: for k > j): the
// products of the QEP targets with the inverse factor U (quantize.py:1330-1335: (H + lambda I)^-1 = U^T U).
extern "C" int lamq_gemm_sub_f64(double* C, int64_t ldc, const double* A, int64_t lda, const double* B, int64_t ldb,
                                 int64_t M, int64_t N, int64_t K, int transb, int tri, void* stream)
{
    if (!C || !A || !B || M < 0 || N < 0 || K < 0 || ldc < N || lda < K || ldb < (transb ? K : N)) return LAMQ_EINVAL;
    if (tri < 0 || tri > 2 || (transb != 0 && transb != 1)) return LAMQ_EINVAL;
    if (M == 0 || N == 0 || K == 0) return LAMQ_OK;
    hipStream_t s = as_stream(stream);
    if (transb) {
        if (tri == 1) return gemm_sub_f64<true, false, false, LAMQ_TRI_KGE>(C, ldc, A, lda, B, ldb, M, N, K, nullptr, s);
        if (tri == 2) return gemm_sub_f64<true, false, false, LAMQ_TRI_KLE>(C, ldc, A, lda, B, ldb, M, N, K, nullptr, s);
        return gemm_sub_f64<true, false>(C, ldc, A, lda, B, ldb, M, N, K, nullptr, s);
    }
    if (tri == 1) return gemm_sub_f64<false, false, false, LAMQ_TRI_KGE>(C, ldc, A, lda, B, ldb, M, N, K, nullptr, s);
    if (tri == 2) return gemm_sub_f64<false, false, false, LAMQ_TRI_KLE>(C, ldc, A, lda, B, ldb, M, N, K, nullptr, s);
    return gemm_sub_f64<false, false>(C, ldc, A, lda, B, ldb, M, N, K, nullptr, s);
}

// T[:, dead] = 0 at the start of a sweep (opgraph/syntax.py:101).
__global__ void zero_columns_kernel(double* __restrict__ T, int64_t m, int64_t n, int64_t ldT, const uint8_t* __restrict__ dead)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m * n) return;
    const int64_t r = i / n, c = i - r * n;
    if (dead[c]) T[r * ldT + c] = 0.0;
}

extern "C" int lamq_zero_columns(double* T, int64_t m, int64_t n, int64_t ldT, const uint8_t* dead, void* stream)
{
    if (!T || !dead || m < 0 || n < 1 || ldT < n) return LAMQ_EINVAL;
    if (m == 0) return LAMQ_OK;
    hipLaunchKernelGGL(zero_columns_kernel, dim3((unsigned)cdiv(m * n, 256)), dim3(256), 0, as_stream(stream), T, m, n, ldT,
                       dead);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

// ------------------------------------------------------------------------------------------------
// One step of the generic sweep (opgraph/syntax.py:117-121) for a projection computed elsewhere:
//   E = T[:, j:j+w] - Q;  z = E U_BB^-1 (forward substitution, an fma chain in l);
//   T[:, col] = T[:, col] - sum_l z[l] U[j+l][col] for col in [j+w, b1);  Z[:, j-b0+c] = z[c]
// One wave per row (w <= 64), four rows per workgroup. The arithmetic is the fused kernels'.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void refit_step_kernel(double* __restrict__ T, int64_t m, int64_t ldT,
                                                         const double* __restrict__ U, int64_t ldU,
                                                         const double* __restrict__ Q, int64_t ldq, int64_t j, int w,
                                                         int64_t b0, int64_t b1, double* __restrict__ Z, int64_t ldZ)
{
    __shared__ double zsh[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= m) return;  // whole waves leave; no workgroup barrier follows
    double* Tr = T + row * ldT;
    double acc = 0.0;
    if (lane < w) {
        const double q = Q[row * ldq + lane];
        acc = Tr[j + lane] - q;
    }
    double zmine = 0.0;
    for (int l = 0; l < w; ++l) {
        double zl = 0.0;
        if (lane == l) zl = acc / U[(j + l) * ldU + j + l];
        zl = __shfl(zl, l);
        if (lane > l && lane < w) acc = fma(-zl, U[(j + l) * ldU + j + lane], acc);
        if (lane == l) zmine = zl;
    }
    // the coefficients go through this wave's LDS slot: the column loop below has a trip count per lane
    zsh[wave][lane] = zmine;
    __builtin_amdgcn_wave_barrier();
    for (int64_t col = j + w + lane; col < b1; col += 64) {
        double a2 = 0.0;
        for (int l = 0; l < w; ++l) a2 = fma(zsh[wave][l], U[(j + l) * ldU + col], a2);
        Tr[col] = Tr[col] - a2;
    }
    if (lane < w) Z[row * ldZ + (j - b0) + lane] = zmine;
}

extern "C" int lamq_refit_step(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU, const double* Q,
                               int64_t ldq, int64_t j, int w, int64_t b0, int64_t b1, double* Z, int64_t ldZ, void* stream)
{
    if (!T || !U || !Q || !Z || m < 0 || n < 1 || ldT < n || ldU < n || w < 1 || ldq < w || b0 < 0 || j < b0 ||
        b1 > n || j + w > b1 || ldZ < b1 - b0)
        return LAMQ_EINVAL;
    if (w > 64) return LAMQ_EUNSUP;
    if (m == 0) return LAMQ_OK;
    hipLaunchKernelGGL(refit_step_kernel, dim3((unsigned)cdiv(m, 4)), dim3(256), 0, as_stream(stream), T, m, ldT, U, ldU, Q,
                       ldq, j, w, b0, b1, Z, ldZ);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

// ------------------------------------------------------------------------------------------------
// Output shaping (opgraph/nested.py:104-147, multirate_sweep with G, one rate): within a column the rows are settled
// `block` at a time, each block's entries on their nearest levels, and the later rows re-solved for the block's
// error through the factor V of the damped output sensitivity: u[b:] -= (u[a:b] - q[a:b]) M_q with
// M_q = V[a:b, a:b]^-1 V[a:b, b:] (nested.py:127-136).
//
// lamq_shaping_feedback: every block's M_q (rows a..b of V's upper factor), packed one after the other, M_q row-major
// [(b - a) x (m - b)]. One workgroup per block but the last (whose M is empty); thread c solves the columns c, c + 256,
// ... of V[a:b, a:b] M = V[a:b, b:] by back substitution (rows from b - 1 down, an fma chain over the rows solved,
// then the division by the diagonal), reading the rows it has solved back from memory.
// ------------------------------------------------------------------------------------------------
extern "C" size_t lamq_shaping_feedback_size(int64_t m, int block)
{
    if (m < 1 || block < 1) return 0;
    const int64_t nb = cdiv(m, (int64_t)block), B = block;
    return (size_t)(B * ((nb - 1) * m - B * (nb - 1) * nb / 2)) * sizeof(double);
}

__global__ __launch_bounds__(256) void shaping_feedback_kernel(const double* __restrict__ V, int64_t m, int64_t ldV,
                                                               int block, double* __restrict__ M)
{
    const int64_t q = blockIdx.x, B = block;
    const int64_t a = q * B, b = a + B;  // a full block: every block but the last is
    const int64_t w = m - b;
    double* Mq = M + B * (q * m - B * q * (q + 1) / 2);
    for (int64_t c = threadIdx.x; c < w; c += 256) {
        for (int64_t r = b - 1; r >= a; --r) {
            double acc = V[r * ldV + b + c];
            for (int64_t s = r + 1; s < b; ++s) acc = fma(-V[r * ldV + s], Mq[(s - a) * w + c], acc);
            Mq[(r - a) * w + c] = acc / V[r * ldV + r];
        }
    }
}

extern "C" int lamq_shaping_feedback(const double* V, int64_t m, int64_t ldV, int block, double* M, void* stream)
{
    if (!V || !M || m < 1 || ldV < m || block < 1) return LAMQ_EINVAL;
    if (block > LAMQ_SHAPE_MAX_BLOCK) return LAMQ_EUNSUP;
    const int64_t nb = cdiv(m, (int64_t)block);
    if (nb < 2) return LAMQ_OK;
    hipLaunchKernelGGL(shaping_feedback_kernel, dim3((unsigned)(nb - 1)), dim3(256), 0, as_stream(stream), V, m, ldV,
                       block, M);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

// lamq_ldlq_shaped_column: column j of T, settled row block by row block (the projection of multirate_sweep with G):
// one 1024-thread workgroup, the column in LDS. Per block the first b - a threads take their entry's nearest level
// (the first least |u - level|, as argmin of the absolute difference), write its index into idx[:, j] and its level into
// Q, and leave the error in LDS; then every later row r subtracts sum_rows e M_q[., r] (an fma chain from 0 in row
// order). T is only read.
__global__ __launch_bounds__(1024) void ldlq_shaped_column_kernel(const double* __restrict__ T, int64_t m, int64_t ldT,
                                                                  int64_t j, const double* __restrict__ M, int block,
                                                                  const double* __restrict__ levels, int K,
                                                                  int32_t* __restrict__ idx, int64_t ldi,
                                                                  double* __restrict__ Q)
{
    __shared__ double u[LAMQ_SHAPE_MAX_M];
    __shared__ double lv[256];
    __shared__ double e[LAMQ_SHAPE_MAX_BLOCK];
    const int tid = threadIdx.x;
    for (int64_t r = tid; r < m; r += 1024) u[r] = T[r * ldT + j];
    for (int l = tid; l < K; l += 1024) lv[l] = levels[l];
    __syncthreads();
    const int64_t B = block;
    for (int64_t a = 0, q = 0; a < m; a += B, ++q) {
        const int64_t b = a + B < m ? a + B : m;
        if (tid < b - a) {
            const double x = u[a + tid];
            int bi = 0;
            double bd = fabs(x - lv[0]);
            for (int l = 1; l < K; ++l) {
                const double d = fabs(x - lv[l]);
                if (d < bd) {
                    bd = d;
                    bi = l;
                }
            }
            idx[(a + tid) * ldi + j] = bi;
            Q[a + tid] = lv[bi];
            e[tid] = x - lv[bi];
        }
        __syncthreads();
        if (b < m) {
            const int64_t w = m - b;
            const double* Mq = M + B * (q * m - B * q * (q + 1) / 2);
            for (int64_t c = tid; c < w; c += 1024) {
                double acc = 0.0;
                for (int64_t r = 0; r < b - a; ++r) acc = fma(e[r], Mq[r * w + c], acc);
                u[b + c] = u[b + c] - acc;
            }
        }
        __syncthreads();
    }
}

extern "C" int lamq_ldlq_shaped_column(const double* T, int64_t m, int64_t n, int64_t ldT, int64_t j, const double* M,
                                       int block, const double* levels, int K, int32_t* idx, int64_t ldi, double* Q,
                                       void* stream)
{
    if (!T || !levels || !idx || !Q || m < 1 || n < 1 || ldT < n || j < 0 || j >= n || block < 1 || K < 1 || ldi < n)
        return LAMQ_EINVAL;
    if (!M && cdiv(m, (int64_t)block) > 1) return LAMQ_EINVAL;
    if (m > LAMQ_SHAPE_MAX_M || block > LAMQ_SHAPE_MAX_BLOCK || K > 256) return LAMQ_EUNSUP;
    hipLaunchKernelGGL(ldlq_shaped_column_kernel, dim3(1), dim3(1024), 0, as_stream(stream), T, m, ldT, j, M, block,
                       levels, K, idx, ldi, Q);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
