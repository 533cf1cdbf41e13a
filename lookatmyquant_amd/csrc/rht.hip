// Randomized Hadamard transform of rows in Kronecker-factored form, and an fp64 transpose.
//
// R = (A (x) B)/sqrt(n) diag(s) with A, B the +/-1 factors of hadamard_factors (opgraph/codes.py:
// 104-119) and s the random signs of rht (codes.py:129-132). For one row w, reshaped as the a x b
// matrix M = reshape(s * w) (index ia*b + ib), out = w R^T = vec(A M B^T) / sqrt(n): a*b*(a+b)
// additions instead of the dense product's n^2 multiply-adds.
#include "common.h"

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
