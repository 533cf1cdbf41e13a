// Randomized Hadamard transform of rows in Kronecker-factored form, and an fp64 transpose.
//
// R = (A (x) B)/sqrt(n) diag(s) with A, B the +/-1 factors of hadamard_factors (opgraph/codes.py:
// 104-119) and s the random signs of rht (codes.py:129-132). For one row w, reshaped as the a x b
// matrix M = reshape(s * w) (index ia*b + ib), out = w R^T = vec(A M B^T) / sqrt(n): a*b*(a+b)
// additions instead of the dense product's n^2 multiply-adds. The products run on fp64 MFMA
// (rht_mfma_rc_kernel, rht_mfma_kernel below: exact +/-1 products, fp64 sums) whenever the two factors'
// operand tables and one row fit the LDS; rht_rows_kernel (sums in LDS) covers the other shapes.
#include "gemm_f64.h"

#define RHT_MAXO 64  // outputs per thread: n <= 64 * 256

__global__ __launch_bounds__(256) void rht_rows_kernel(const double* in, int n, int64_t ldi, double* out, int64_t ldo,
                                                       const int8_t* __restrict__ signs, const int8_t* __restrict__ A,
                                                       int a, const int8_t* __restrict__ B, int b, double* __restrict__ rms,
                                                       double sqrt_n, int inverse)
{
    extern __shared__ double smem[];
    double* buf = smem;
    int8_t* Bs = reinterpret_cast<int8_t*>(buf + n);
    int8_t* As = Bs + b * b;
    __shared__ double part[256];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    // inverse: out = in R = vec(A^T M B) diag(s) / sqrt(n), i.e. the transposed factors, signs after
    for (int e = tid; e < b * b; e += 256) Bs[e] = inverse ? B[(e % b) * b + e / b] : B[e];
    for (int e = tid; e < a * a; e += 256) As[e] = inverse ? A[(e % a) * a + e / a] : A[e];
    const double* x = in + row * ldi;
    for (int j = tid; j < n; j += 256) buf[j] = (inverse || signs[j] > 0) ? x[j] : -x[j];
    __syncthreads();
    double o[RHT_MAXO];
    // M2 = M B^T: M2[ia][ib] = sum_j B[ib][j] M[ia][j]
#pragma unroll
    for (int i = 0; i < RHT_MAXO; ++i) {
        const int idx = tid + i * 256;
        double acc = 0.0;
        if (idx < n) {
            const int ia = idx / b, ib = idx - ia * b;
            const double* mr = buf + ia * b;
            const int8_t* br = Bs + ib * b;
            for (int j = 0; j < b; ++j) acc += br[j] > 0 ? mr[j] : -mr[j];
        }
        o[i] = acc;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RHT_MAXO; ++i) {
        const int idx = tid + i * 256;
        if (idx < n) buf[idx] = o[i];
    }
    __syncthreads();
    // Y = A M2: Y[ia][ib] = sum_j A[ia][j] M2[j][ib]
    double ss = 0.0;
    double* y = out + row * ldo;
#pragma unroll
    for (int i = 0; i < RHT_MAXO; ++i) {
        const int idx = tid + i * 256;
        if (idx < n) {
            const int ia = idx / b, ib = idx - ia * b;
            const int8_t* ar = As + ia * a;
            double acc = 0.0;
            for (int j = 0; j < a; ++j) acc += ar[j] > 0 ? buf[j * b + ib] : -buf[j * b + ib];
            double v = acc / sqrt_n;
            if (inverse && signs[idx] < 0) v = -v;
            o[i] = v;
            ss += v * v;
        }
    }
    __syncthreads();  // every read of buf is done before out (which may alias in) is written
#pragma unroll
    for (int i = 0; i < RHT_MAXO; ++i) {
        const int idx = tid + i * 256;
        if (idx < n) y[idx] = o[i];
    }
    if (rms) {
        part[tid] = ss;
        __syncthreads();
        for (int w = 128; w > 0; w >>= 1) {
            if (tid < w) part[tid] += part[tid + w];
            __syncthreads();
        }
        if (tid == 0) {
            const double r = sqrt(part[0] / (double)n);
            rms[row] = r > 1e-12 ? r : 1e-12;
        }
    }
}

// The same transform as two MFMA products per row (v_mfma_f64_16x16x4f64 with +/-1 operands, exact products and
// fp64 sums): M2 = M B^T (the B side), then Y = A M2 (the A side), with M the a x b reshape of the signed row in
// LDS. Operand layout (16x16x4): lane l gives A[l % 16][k4 + l / 16] and B[k4 + l / 16][l % 16]; result register v
// of lane l is row 4v + l / 16, column l % 16. The +/-1 operands of both factors are laid out once per workgroup in
// LDS as bytes in exactly the lane order the MFMAs read them (0 in the padding of a or b to 4 and 16), so each
// MFMA reads one byte and converts it. The inverse uses A^T and B in place of A and B^T. A workgroup keeps the
// tables and walks rows blockIdx.x, blockIdx.x + gridDim.x, ...
// x = the row (times the signs sg, kept in LDS, when forward): eight loads per thread in flight at a time, from
// clamped (always valid) addresses so that no load sits behind a branch
__device__ __forceinline__ void rht_load_row(double* x, const double* xin, int n, const int8_t* sg, int inverse,
                                             int tid)
{
    for (int j0 = 0; j0 < n; j0 += 8 * 256) {
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = j0 + 256 * u + tid;
            v[u] = xin[j < n ? j : n - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = j0 + 256 * u + tid;
            if (j < n) x[j] = (inverse || sg[j] > 0) ? v[u] : -v[u];
        }
    }
}

#define RHT2_TILES 16  // result tiles of 16 x 16 per wave at most: a/16 x b/16 <= 64

// TW result tiles per wave: tile t = wave + 4q (q < TW) is row tile t % nrt and column tile t / nrt, so a wave's
// tiles share row and column tiles. The k-steps run outermost and the TW independent accumulators inside, so the
// MFMAs of different tiles overlap. Tiles past nt read clamped (valid) operands and are not stored.
template <int TW>
__global__ __launch_bounds__(256) void rht_mfma_kernel(const double* in, int64_t rows, int n, int64_t ldi, double* out,
                                                       int64_t ldo, const int8_t* __restrict__ signs,
                                                       const int8_t* __restrict__ A, int a, const int8_t* __restrict__ B,
                                                       int b, double* __restrict__ rms, double sqrt_n, int inverse)
{
    extern __shared__ double smem[];
    double* x = smem;                                     // n: the row, then M2
    double* part = x + n;                                 // 256: the row's sum of squares
    int8_t* Aop = reinterpret_cast<int8_t*>(part + 256);  // nrt x nka x 64
    const int nrt = (a + 15) / 16, nct = (b + 15) / 16, nka = (a + 3) / 4, nkb = (b + 3) / 4;
    int8_t* Bop = Aop + nrt * nka * 64;                   // nct x nkb x 64
    int8_t* sg = Bop + nct * nkb * 64;                    // n: the signs
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int j = tid; j < n; j += 256) sg[j] = signs[j];
    const int li = lane & 15, lk = lane >> 4;
    for (int e = tid; e < nrt * nka * 64; e += 256) {
        const int l = e & 63, q = e >> 6, rt = q / nka, ks = q - rt * nka;
        const int r = 16 * rt + (l & 15), k = 4 * ks + (l >> 4);
        Aop[e] = (r < a && k < a) ? (inverse ? A[k * a + r] : A[r * a + k]) : (int8_t)0;
    }
    for (int e = tid; e < nct * nkb * 64; e += 256) {
        const int l = e & 63, q = e >> 6, ct = q / nkb, ks = q - ct * nkb;
        const int c = 16 * ct + (l & 15), k = 4 * ks + (l >> 4);
        Bop[e] = (c < b && k < b) ? (inverse ? B[k * b + c] : B[c * b + k]) : (int8_t)0;
    }
    __syncthreads();  // the tables and signs are read by every wave
    const int nt = nrt * nct;
    int rq[TW], cq[TW];
    bool vq[TW];
#pragma unroll
    for (int q = 0; q < TW; ++q) {
        const int t = wave + 4 * q;
        vq[q] = t < nt;
        const int tc = vq[q] ? t : nt - 1;
        rq[q] = tc % nrt;
        cq[q] = tc / nrt;
    }
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        rht_load_row(x, in + row * ldi, n, sg, inverse, tid);
        __syncthreads();
        // B side: M2 = M B^T (inverse: M B)
        lamq_d4 acc[TW];
#pragma unroll
        for (int q = 0; q < TW; ++q) acc[q] = lamq_d4{0.0, 0.0, 0.0, 0.0};
#pragma unroll 1
        for (int ks = 0; ks < nkb; ++ks) {
            const int k = 4 * ks + lk;
#pragma unroll
            for (int q = 0; q < TW; ++q) {
                const int r = 16 * rq[q] + li;
                const double av = (r < a && k < b) ? x[r * b + k] : 0.0;
                const double bv = (double)Bop[(cq[q] * nkb + ks) * 64 + lane];
                acc[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc[q], 0, 0, 0);
            }
        }
        __syncthreads();  // every read of M is done
#pragma unroll
        for (int q = 0; q < TW; ++q) {
            const int c = 16 * cq[q] + li;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = 16 * rq[q] + 4 * v + lk;
                if (vq[q] && r < a && c < b) x[r * b + c] = acc[q][v];
            }
        }
        __syncthreads();
        // A side: Y = A M2 (inverse: A^T M2), back into x, then out with the scale (and the signs)
#pragma unroll
        for (int q = 0; q < TW; ++q) acc[q] = lamq_d4{0.0, 0.0, 0.0, 0.0};
#pragma unroll 1
        for (int ks = 0; ks < nka; ++ks) {
            const int k = 4 * ks + lk;
#pragma unroll
            for (int q = 0; q < TW; ++q) {
                const int c = 16 * cq[q] + li;
                const double av = (double)Aop[(rq[q] * nka + ks) * 64 + lane];
                const double bv = (k < a && c < b) ? x[k * b + c] : 0.0;
                acc[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc[q], 0, 0, 0);
            }
        }
        __syncthreads();  // every read of M2 is done
#pragma unroll
        for (int q = 0; q < TW; ++q) {
            const int c = 16 * cq[q] + li;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = 16 * rq[q] + 4 * v + lk;
                if (vq[q] && r < a && c < b) x[r * b + c] = acc[q][v];
            }
        }
        __syncthreads();
        double ss = 0.0;
        double* y = out + row * ldo;
        for (int j = tid; j < n; j += 256) {
            double val = x[j] / sqrt_n;
            if (inverse && sg[j] < 0) val = -val;
            y[j] = val;
            ss += val * val;
        }
        if (rms) {
            part[tid] = ss;
            __syncthreads();
            for (int w = 128; w > 0; w >>= 1) {
                if (tid < w) part[tid] += part[tid + w];
                __syncthreads();
            }
            if (tid == 0) {
                const double r = sqrt(part[0] / (double)n);
                rms[row] = r > 1e-12 ? r : 1e-12;
            }
        }
        __syncthreads();  // x is rewritten by the next row
    }
}

// The common shapes: RT row tiles (wave, wave + 4, ...) and all CT column tiles per wave, so each k-step loads
// RT + CT operands for RT x CT MFMAs, and the operands of the next k-step are loaded while this one's MFMAs run.
template <int RT, int CT>
__global__ __launch_bounds__(256) void rht_mfma_rc_kernel(const double* in, int64_t rows, int n, int64_t ldi,
                                                          double* out, int64_t ldo, const int8_t* __restrict__ signs,
                                                          const int8_t* __restrict__ A, int a,
                                                          const int8_t* __restrict__ B, int b,
                                                          double* __restrict__ rms, double sqrt_n, int inverse)
{
    extern __shared__ double smem[];
    double* x = smem;
    double* part = x + n;
    int8_t* Aop = reinterpret_cast<int8_t*>(part + 256);
    const int nrt = (a + 15) / 16, nka = (a + 3) / 4, nkb = (b + 3) / 4;
    int8_t* Bop = Aop + nrt * nka * 64;
    int8_t* sg = Bop + ((b + 15) / 16) * nkb * 64;  // n: the signs
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int j = tid; j < n; j += 256) sg[j] = signs[j];
    const int li = lane & 15, lk = lane >> 4;
    for (int e = tid; e < nrt * nka * 64; e += 256) {
        const int l = e & 63, q = e >> 6, rt = q / nka, ks = q - rt * nka;
        const int r = 16 * rt + (l & 15), k = 4 * ks + (l >> 4);
        Aop[e] = (r < a && k < a) ? (inverse ? A[k * a + r] : A[r * a + k]) : (int8_t)0;
    }
    for (int e = tid; e < CT * nkb * 64; e += 256) {
        const int l = e & 63, q = e >> 6, ct = q / nkb, ks = q - ct * nkb;
        const int c = 16 * ct + (l & 15), k = 4 * ks + (l >> 4);
        Bop[e] = (c < b && k < b) ? (inverse ? B[k * b + c] : B[c * b + k]) : (int8_t)0;
    }
    __syncthreads();  // the tables and signs are read by every wave
    // this lane's rows (B side) and columns (A side); rows past a and columns past b read index 0 and are not stored
    int arow[RT], aop[RT];
    bool rok[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        const int r = 16 * (wave + 4 * i) + li;
        rok[i] = r < a;
        arow[i] = rok[i] ? r * b : 0;
        aop[i] = ((wave + 4 * i) < nrt ? (wave + 4 * i) : 0) * nka * 64 + lane;
    }
    int bop[CT], col[CT];
    bool cok[CT];
#pragma unroll
    for (int j = 0; j < CT; ++j) {
        bop[j] = j * nkb * 64 + lane;
        col[j] = 16 * j + li;
        cok[j] = col[j] < b;
    }
    const bool active = wave < nrt;  // a wave with no row tile only helps with the loads and stores
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        rht_load_row(x, in + row * ldi, n, sg, inverse, tid);
        __syncthreads();
        lamq_d4 acc[RT][CT];
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int j = 0; j < CT; ++j) acc[i][j] = lamq_d4{0.0, 0.0, 0.0, 0.0};
        if (active) {  // B side: M2 = M B^T (inverse: M B)
            // two operand sets alternate: the next k-step's operands are loaded raw (valid addresses, bytes
            // unconverted) while this k-step's MFMAs run, and masked or converted only when used
            double av0[RT], av1[RT];
            int bv0[CT], bv1[CT];
            auto fetch = [&](int ks, double(&av)[RT], int(&bv)[CT]) {
                const int k = 4 * ks + lk;
#pragma unroll
                for (int i = 0; i < RT; ++i) av[i] = x[arow[i] + (k < b ? k : 0)];
#pragma unroll
                for (int j = 0; j < CT; ++j) bv[j] = Bop[bop[j] + 64 * ks];
            };
            // all of a k-step's operands are converted into registers of their own before its MFMAs: an operand
            // register rewritten right after the MFMA that reads it holds the next MFMA until the first has read it
            auto step = [&](int ks, const double(&av)[RT], const int(&bv)[CT]) {
                const bool kok = 4 * ks + lk < b;
                double am[RT], bd[CT];
#pragma unroll
                for (int i = 0; i < RT; ++i) {
                    am[i] = (rok[i] && kok) ? av[i] : 0.0;
                    asm volatile("" : "+v"(am[i]));
                }
#pragma unroll
                for (int j = 0; j < CT; ++j) {
                    bd[j] = (double)bv[j];
                    asm volatile("" : "+v"(bd[j]));
                }
#pragma unroll
                for (int i = 0; i < RT; ++i)
#pragma unroll
                    for (int j = 0; j < CT; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(am[i], bd[j], acc[i][j], 0, 0, 0);
            };
            fetch(0, av0, bv0);
#pragma unroll 1
            for (int ks = 0; ks < nkb; ks += 2) {
                const bool two = ks + 1 < nkb;
                if (two) fetch(ks + 1, av1, bv1);
                step(ks, av0, bv0);
                if (ks + 2 < nkb) fetch(ks + 2, av0, bv0);
                if (two) step(ks + 1, av1, bv1);
            }
        }
        __syncthreads();  // every read of M is done
        if (active) {
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int j = 0; j < CT; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int r = 16 * (wave + 4 * i) + 4 * v + lk;
                        if (r < a && cok[j]) x[r * b + col[j]] = acc[i][j][v];
                    }
        }
        __syncthreads();
        if (active) {  // A side: Y = A M2 (inverse: A^T M2)
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int j = 0; j < CT; ++j) acc[i][j] = lamq_d4{0.0, 0.0, 0.0, 0.0};
            int av0[RT], av1[RT];
            double bv0[CT], bv1[CT];
            auto fetch = [&](int ks, int(&av)[RT], double(&bv)[CT]) {
                const int k = 4 * ks + lk;
#pragma unroll
                for (int i = 0; i < RT; ++i) av[i] = Aop[aop[i] + 64 * ks];
#pragma unroll
                for (int j = 0; j < CT; ++j) bv[j] = x[(k < a ? k : 0) * b + (cok[j] ? col[j] : 0)];
            };
            auto step = [&](int ks, const int(&av)[RT], const double(&bv)[CT]) {
                const bool kok = 4 * ks + lk < a;
                double am[RT], bd[CT];
#pragma unroll
                for (int i = 0; i < RT; ++i) {
                    am[i] = (double)av[i];
                    asm volatile("" : "+v"(am[i]));
                }
#pragma unroll
                for (int j = 0; j < CT; ++j) {
                    bd[j] = (cok[j] && kok) ? bv[j] : 0.0;
                    asm volatile("" : "+v"(bd[j]));
                }
#pragma unroll
                for (int i = 0; i < RT; ++i)
#pragma unroll
                    for (int j = 0; j < CT; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(am[i], bd[j], acc[i][j], 0, 0, 0);
            };
            fetch(0, av0, bv0);
#pragma unroll 1
            for (int ks = 0; ks < nka; ks += 2) {
                const bool two = ks + 1 < nka;
                if (two) fetch(ks + 1, av1, bv1);
                step(ks, av0, bv0);
                if (ks + 2 < nka) fetch(ks + 2, av0, bv0);
                if (two) step(ks + 1, av1, bv1);
            }
        }
        __syncthreads();  // every read of M2 is done
        if (active) {
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int j = 0; j < CT; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int r = 16 * (wave + 4 * i) + 4 * v + lk;
                        if (r < a && cok[j]) x[r * b + col[j]] = acc[i][j][v];
                    }
        }
        __syncthreads();
        double ss = 0.0;
        double* y = out + row * ldo;
        for (int j = tid; j < n; j += 256) {
            double val = x[j] / sqrt_n;
            if (inverse && sg[j] < 0) val = -val;
            y[j] = val;
            ss += val * val;
        }
        if (rms) {
            part[tid] = ss;
            __syncthreads();
            for (int w = 128; w > 0; w >>= 1) {
                if (tid < w) part[tid] += part[tid + w];
                __syncthreads();
            }
            if (tid == 0) {
                const double r = sqrt(part[0] / (double)n);
                rms[row] = r > 1e-12 ? r : 1e-12;
            }
        }
        __syncthreads();  // x is rewritten by the next row
    }
}

static size_t rht_mfma_lds(int a, int b)
{
    const size_t nrt = (a + 15) / 16, nct = (b + 15) / 16, nka = (a + 3) / 4, nkb = (b + 3) / 4;
    return (size_t)a * b * sizeof(double) + 256 * sizeof(double) + nrt * nka * 64 + nct * nkb * 64 + (size_t)a * b;
}

static bool rht_mfma_ok(int a, int b)
{
    return ((a + 15) / 16) * ((b + 15) / 16) <= 4 * RHT2_TILES && rht_mfma_lds(a, b) <= 150 * 1024;
}

extern "C" int lamq_rht_rows(const double* in, int64_t rows, int64_t n, int64_t ldi, double* out, int64_t ldo,
                             const int8_t* signs, const int8_t* A, int a, const int8_t* B, int b, int inverse,
                             double* rms, void* stream)
{
    if (!in || !out || !signs || !A || !B || rows < 0 || n < 1 || ldi < n || ldo < n || a < 1 || b < 1)
        return LAMQ_EINVAL;
    if ((int64_t)a * b != n) return LAMQ_EINVAL;
    if (n > RHT_MAXO * 256 || rows > 0x7fffffff) return LAMQ_EUNSUP;
    const size_t lds = (size_t)n * sizeof(double) + (size_t)b * b + (size_t)a * a;
    if (lds > 150 * 1024) return LAMQ_EUNSUP;
    if (rows == 0) return LAMQ_OK;
    if (rht_mfma_ok(a, b)) {
        const int nrt = (a + 15) / 16, nct = (b + 15) / 16;
        const int rt = (nrt + 3) / 4;
        const unsigned grid0 = (unsigned)(rows < 1024 ? rows : 1024);
        const size_t lds0 = rht_mfma_lds(a, b);
#define RHT_RC(R, C)                                                                                                  \
    if (rt == R && nct == C) {                                                                                        \
        hipError_t e = hipFuncSetAttribute((const void*)rht_mfma_rc_kernel<R, C>,                                      \
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);                    \
        if (e != hipSuccess) return (int)e;                                                                           \
        hipLaunchKernelGGL((rht_mfma_rc_kernel<R, C>), dim3(grid0), dim3(256), lds0, as_stream(stream), in, rows,      \
                           (int)n, ldi, out, ldo, signs, A, a, B, b, rms, sqrt((double)n), inverse);                   \
        LAMQ_LAUNCH_CHECK();                                                                                          \
        return LAMQ_OK;                                                                                               \
    }
        RHT_RC(1, 1) RHT_RC(1, 2) RHT_RC(1, 4) RHT_RC(1, 8) RHT_RC(1, 10) RHT_RC(2, 2) RHT_RC(4, 1) RHT_RC(4, 2)
#undef RHT_RC
        const int tw = (nrt * nct + 3) / 4;
        const unsigned grid = (unsigned)(rows < 1024 ? rows : 1024);
        const size_t lds = rht_mfma_lds(a, b);
#define RHT2_LAUNCH(T)                                                                                                \
    do {                                                                                                              \
        hipError_t e = hipFuncSetAttribute((const void*)rht_mfma_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                           150 * 1024);                                                              \
        if (e != hipSuccess) return (int)e;                                                                           \
        hipLaunchKernelGGL(rht_mfma_kernel<T>, dim3(grid), dim3(256), lds, as_stream(stream), in, rows, (int)n, ldi,    \
                           out, ldo, signs, A, a, B, b, rms, sqrt((double)n), inverse);                                \
    } while (0)
        if (tw <= 1) RHT2_LAUNCH(1);
        else if (tw <= 2) RHT2_LAUNCH(2);
        else if (tw <= 4) RHT2_LAUNCH(4);
        else if (tw <= 8) RHT2_LAUNCH(8);
        else if (tw <= 10) RHT2_LAUNCH(10);
        else if (tw <= 12) RHT2_LAUNCH(12);
        else RHT2_LAUNCH(16);
#undef RHT2_LAUNCH
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
    hipError_t e = hipFuncSetAttribute((const void*)rht_rows_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       150 * 1024);
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(rht_rows_kernel, dim3((unsigned)rows), dim3(256), lds, as_stream(stream), in, (int)n, ldi, out, ldo,
                       signs, A, a, B, b, rms, sqrt((double)n), inverse);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

__global__ __launch_bounds__(256) void transpose_f64_kernel(const double* __restrict__ in, int64_t rows, int64_t cols,
                                                            int64_t ldi, double* __restrict__ out, int64_t ldo)
{
    __shared__ double t[32][33];
    const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int i = ty; i < 32; i += 8) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) t[i][tx] = in[r * ldi + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int64_t r = c0 + i, c = r0 + tx;  // out[r][c] = in[c][r]
        if (r < cols && c < rows) out[r * ldo + c] = t[tx][i];
    }
}

extern "C" int lamq_transpose_f64(const double* in, int64_t rows, int64_t cols, int64_t ldi, double* out, int64_t ldo,
                                  void* stream)
{
    if (!in || !out || rows < 0 || cols < 0 || ldi < cols || ldo < rows || in == out) return LAMQ_EINVAL;
    if (rows == 0 || cols == 0) return LAMQ_OK;
    hipLaunchKernelGGL(transpose_f64_kernel, dim3((unsigned)cdiv(cols, 32), (unsigned)cdiv(rows, 32)), dim3(256), 0,
                       as_stream(stream), in, rows, cols, ldi, out, ldo);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

// S_r = max(sqrt(mean_j X[r, j]^2), 1e-12) (opgraph/codes.py:436, nested.py:168), one workgroup per row,
// summed in a fixed order.
__global__ __launch_bounds__(256) void row_rms_kernel(const double* __restrict__ X, int64_t n, int64_t ldx,
                                                      double* __restrict__ S)
{
    __shared__ double part[256];
    const double* x = X + (int64_t)blockIdx.x * ldx;
    double ss = 0.0;
    for (int64_t j = threadIdx.x; j < n; j += 256) ss += x[j] * x[j];
    part[threadIdx.x] = ss;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const double r = sqrt(part[0] / (double)n);
        S[blockIdx.x] = r > 1e-12 ? r : 1e-12;
    }
}

extern "C" int lamq_row_rms(const double* X, int64_t rows, int64_t n, int64_t ldx, double* S, void* stream)
{
    if (!X || !S || rows < 0 || n < 1 || ldx < n) return LAMQ_EINVAL;
    if (rows == 0) return LAMQ_OK;
    if (rows > 0x7fffffff) return LAMQ_EUNSUP;
    hipLaunchKernelGGL(row_rms_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), X, n, ldx, S);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
