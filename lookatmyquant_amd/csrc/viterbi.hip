// Trellis search kernels: standalone Viterbi over rows, and one lazy block of the row-trellis
// block-LDLQ sweep (the search fused with the block's fp64 refit).
#include "common.h"

#define LAMQ_TV_LDS 32  // longest standalone path whose back-pointers stay in LDS
#define LAMQ_TV_BLK 24  // longest search of the fused block (width + look): with lazy <= 128 the block kernel's
                        // LDS stays under 40 KB, four workgroups per CU
#define LAMQ_LAZY_MAX 128

// ------------------------------------------------------------------------------------------------
// viterbi_rows: one workgroup per row (opgraph/codes.py:151-181).
// ------------------------------------------------------------------------------------------------
template <int L, int K, bool BACK_GLOBAL>
__global__ __launch_bounds__(LAMQ_NT) void viterbi_rows_kernel(const float* __restrict__ x, int T, int64_t ldx,
                                                               const float* __restrict__ C,
                                                               const int32_t* __restrict__ start,
                                                               int32_t* __restrict__ states, int64_t lds,
                                                               uint8_t* __restrict__ back_ws)
{
    using V = Vit<L, K>;
    __shared__ __align__(16) float cost[2][V::NS];
    __shared__ uint8_t back_lds[BACK_GLOBAL ? 1 : LAMQ_TV_LDS * V::ACT];
    __shared__ float red[8];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    float Cr[V::SPT];
    if (tid < V::ACT) {
#pragma unroll
        for (int i = 0; i < V::SPT; ++i) Cr[i] = C[tid * V::SPT + i];
    }
    uint8_t* back = BACK_GLOBAL ? back_ws + row * (int64_t)T * V::ACT : back_lds;
    const int st = start ? start[row] : -1;
    viterbi_wg<L, K>(x + row * ldx, T, Cr, st, cost[0], cost[1], back, states + row * lds, red);
}

template <int L, int K>
struct ViterbiRows {
    static int run(const float* x, int64_t B, int T, int64_t ldx, const float* C, const int32_t* start,
                   int32_t* states, int64_t lds, void* ws, size_t ws_bytes, hipStream_t s)
    {
        if (T <= LAMQ_TV_LDS) {
            hipLaunchKernelGGL((viterbi_rows_kernel<L, K, false>), dim3((unsigned)B), dim3(LAMQ_NT), 0, s, x, T, ldx, C,
                               start, states, lds, (uint8_t*)nullptr);
        } else {
            const size_t need = (size_t)B * (size_t)T * Vit<L, K>::ACT;
            if (!ws || ws_bytes < need) return LAMQ_EINVAL;
            hipLaunchKernelGGL((viterbi_rows_kernel<L, K, true>), dim3((unsigned)B), dim3(LAMQ_NT), 0, s, x, T, ldx, C,
                               start, states, lds, (uint8_t*)ws);
        }
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
};

template <int L, int K>
struct ActOf {
    static int run(size_t* out) { *out = Vit<L, K>::ACT; return LAMQ_OK; }
};

extern "C" size_t lamq_viterbi_workspace_size(int64_t B, int T, int L, int k)
{
    if (B < 0 || T <= LAMQ_TV_LDS) return 0;
    size_t act = 0;
    if (dispatch_lk<ActOf>(L, k, &act) != LAMQ_OK) return 0;
    return (size_t)B * (size_t)T * act;
}

extern "C" int lamq_viterbi_rows(const float* x, int64_t B, int T, int64_t ldx, const float* C, int L, int k,
                                 const int32_t* start, int32_t* states, int64_t lds, void* workspace,
                                 size_t workspace_bytes, void* stream)
{
    if (B < 0 || T < 1 || ldx < T || lds < T || !C || !states || !x) return LAMQ_EINVAL;
    if (B == 0) return LAMQ_OK;
    if (B > 0x7fffffff) return LAMQ_EUNSUP;
    return dispatch_lk<ViterbiRows>(L, k, x, B, T, ldx, C, start, states, lds, workspace, workspace_bytes,
                                    as_stream(stream));
}

// ------------------------------------------------------------------------------------------------
// ldlq_trellis_block: one workgroup per row walks the steps j = b0, b0+width, ... of the lazy block
// [b0, b1). Per step (opgraph/syntax.py:109-121 with codes.py:442-450 and :397-404):
//   xs    = float32(T[j : j+w+a] / S)       w settled columns, a <= look look-ahead columns, which
//           beyond b1 still lack this block's trailing update (they are read as they stand)
//   path  = viterbi(xs, start = state)[:w];  state = path[w-1]
//   E     = T[j+c] - table64[path[c]] * S
//   z     = E U_BB^-1: z[c] = (E[c] - sum_{l<c} z[l] U[j+l][j+c]) / U[j+c][j+c], an fma chain in l
//   T[col] = T[col] - sum_l z[l] U[j+l][col] for col in [j+w, b1), the sum an fma chain from 0
// The block's columns of T live in LDS for the whole block; T in HBM is not written (the settled
// values are table64[states] * S; columns >= b1 get the trailing update from Z afterwards).
// ------------------------------------------------------------------------------------------------
template <int L, int K>
__global__ __launch_bounds__(LAMQ_NT) void ldlq_trellis_block_kernel(
    const double* __restrict__ T, int64_t n, int64_t ldT, const double* __restrict__ U, int64_t ldU,
    const double* __restrict__ S, const double* __restrict__ table64, const float* __restrict__ table32,
    int64_t b0, int64_t b1, int width, int look, int32_t* __restrict__ state, int32_t* __restrict__ states,
    int64_t lds, double* __restrict__ Z, int64_t ldZ)
{
    using V = Vit<L, K>;
    __shared__ __align__(16) float cost[2][V::NS];
    __shared__ uint8_t back[LAMQ_TV_BLK * V::ACT];
    __shared__ double trow[LAMQ_LAZY_MAX + LAMQ_TV_BLK];
    __shared__ float xs[LAMQ_TV_BLK];
    __shared__ int path[LAMQ_TV_BLK];
    __shared__ double es[LAMQ_TV_BLK];
    __shared__ double zs[LAMQ_TV_BLK];
    __shared__ float red[8];

    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    float Cr[V::SPT];
    if (tid < V::ACT) {
#pragma unroll
        for (int i = 0; i < V::SPT; ++i) Cr[i] = table32[tid * V::SPT + i];
    }
    const int64_t cend = (b1 + look < n) ? b1 + look : n;
    const double* Tr = T + row * ldT;
    for (int64_t c = tid; c < cend - b0; c += LAMQ_NT) trow[c] = Tr[b0 + c];
    const double Sr = S[row];
    int st = state[row];
    __syncthreads();

    for (int64_t j = b0; j < b1; j += width) {
        const int w = (int)((j + width <= b1) ? width : (b1 - j));
        const int64_t ahead = n - (j + w);
        const int a = (int)(ahead < look ? ahead : look);
        const int TV = w + a;
        const int jo = (int)(j - b0);
        if (tid < TV) xs[tid] = (float)(trow[jo + tid] / Sr);
        __syncthreads();
        viterbi_wg<L, K>(xs, TV, Cr, st, cost[0], cost[1], back, path, red);
        if (tid < w) {
            const int p = path[tid];
            states[row * lds + j + tid] = p;
            const double qs = table64[p] * Sr;
            es[tid] = trow[jo + tid] - qs;
        }
        __syncthreads();
        if (tid < 64) {
            double acc = tid < w ? es[tid] : 0.0;
            for (int l = 0; l < w; ++l) {
                double zl = 0.0;
                if (tid == l) zl = acc / U[(j + l) * ldU + j + l];
                zl = __shfl(zl, l);
                if (tid > l && tid < w) acc = fma(-zl, U[(j + l) * ldU + j + tid], acc);
                if (tid == l) zs[l] = zl;
            }
        }
        __syncthreads();
        for (int64_t col = j + w + tid; col < b1; col += LAMQ_NT) {
            double acc = 0.0;
            for (int l = 0; l < w; ++l) acc = fma(zs[l], U[(j + l) * ldU + col], acc);
            trow[col - b0] = trow[col - b0] - acc;
        }
        if (tid < w) Z[row * ldZ + jo + tid] = zs[tid];
        st = path[w - 1];
        __syncthreads();
    }
    if (tid == 0) state[row] = st;
}

template <int L, int K>
struct TrellisBlock {
    static int run(const double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU, const double* S,
                   const double* table64, const float* table32, int64_t b0, int64_t b1, int width, int look,
                   int32_t* state, int32_t* states, int64_t lds, double* Z, int64_t ldZ, hipStream_t s)
    {
        hipLaunchKernelGGL((ldlq_trellis_block_kernel<L, K>), dim3((unsigned)m), dim3(LAMQ_NT), 0, s, T, n, ldT, U, ldU, S,
                           table64, table32, b0, b1, width, look, state, states, lds, Z, ldZ);
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
};

extern "C" int lamq_ldlq_trellis_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                       const double* S, const double* table64, const float* table32, int L, int k,
                                       int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                                       int64_t lds, double* Z, int64_t ldZ, void* stream)
{
    if (!T || !U || !S || !table64 || !table32 || !state || !states || !Z) return LAMQ_EINVAL;
    if (m < 0 || n < 1 || ldT < n || ldU < n || lds < n || b0 < 0 || b1 <= b0 || b1 > n || width < 1 || look < 0)
        return LAMQ_EINVAL;
    if (ldZ < b1 - b0) return LAMQ_EINVAL;
    if (width + look > LAMQ_TV_BLK || b1 - b0 > LAMQ_LAZY_MAX || m > 0x7fffffff) return LAMQ_EUNSUP;
    if (m == 0) return LAMQ_OK;
    return dispatch_lk<TrellisBlock>(L, k, T, m, n, ldT, U, ldU, S, table64, table32, b0, b1, width, look, state,
                                     states, lds, Z, ldZ, as_stream(stream));
}
