// Trellis search kernels: standalone Viterbi over rows, and one lazy block of the row-trellis
// block-LDLQ sweep (the search fused with the block's fp64 refit).
#include "trellis.h"

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
    using V = VX<L, K, LAMQ_NT>;
    __shared__ __align__(16) float buf[2 * V::R];
    __shared__ uint8_t back_lds[BACK_GLOBAL ? 1 : (LAMQ_TV_LDS - 1) * V::ACT];
    __shared__ float red[2 * (LAMQ_NT / 64)];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    TabF32<V> tab;
    if (tid < V::ACT) tab.load(C, tid);
    uint8_t* back = BACK_GLOBAL ? back_ws + row * (int64_t)(T - 1) * V::ACT : back_lds;
    const int st = start ? start[row] : -1;
    viterbi_gx<L, K, LAMQ_NT, true, BACK_GLOBAL>(x + row * ldx, T, tab, st, buf, back, states + row * lds, red);
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
            const size_t need = (size_t)B * (size_t)T * VX<L, K, LAMQ_NT>::ACT;
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
    static int run(size_t* out) { *out = VX<L, K, LAMQ_NT>::ACT; return LAMQ_OK; }
};

// ------------------------------------------------------------------------------------------------
// viterbi_wide: the same search for the (L, k) the kernels above are not built for: k = 5..8 (and k = L), with
// 2^L <= 2^LAMQ_WIDE_MAX_L states. One 256-thread workgroup per row; the 2^L path costs live in LDS. Per position
// the R = 2^(L-k) group minima over h (cost[h R + g], h < 2^k) are formed first: with R < 256 groups, 256 / R
// consecutive threads share a group, each scanning its members h = j, j + 256/R, ... in increasing order (a strict
// compare keeps the lowest h), and the group's first thread combines their (value, h) pairs, the lower h winning a
// tie; with R >= 256 a thread scans whole groups. The new cost of state s is then best[s >> k] + (x - C[s])^2 with
// the reference's three rounded operations (opgraph/codes.py:170-173), and the winning h of each group is its
// back-pointer byte (uint8, as the reference keeps them), in the workspace: T * R bytes per row. The final state is
// the lowest one of least cost; the traceback is s = (s >> k) + back[t][s >> k] * R (codes.py:175-178).
// ------------------------------------------------------------------------------------------------
#define LAMQ_WIDE_MAX_L 14
#define LAMQ_WIDE_NT 256

__device__ __forceinline__ bool wide_better(float v, int h, float bv, int bh)
{
    return v < bv || (v == bv && h < bh);
}

__global__ __launch_bounds__(LAMQ_WIDE_NT) void viterbi_wide_kernel(const float* __restrict__ x, int T, int64_t ldx,
                                                                    const float* __restrict__ C, int L, int k,
                                                                    const int32_t* __restrict__ start,
                                                                    int32_t* __restrict__ states, int64_t lds,
                                                                    uint8_t* __restrict__ back_ws)
{
    __shared__ float cost[1 << LAMQ_WIDE_MAX_L];
    __shared__ float pv[LAMQ_WIDE_NT];
    __shared__ int ph[LAMQ_WIDE_NT];
    __shared__ float best[LAMQ_WIDE_NT];  // group minima (R < 256), or the final reduction's values
    __shared__ int arg_s;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const float* xr = x + row * ldx;
    const int NS = 1 << L, NB = 1 << k, R = 1 << (L - k);
    uint8_t* back = back_ws + row * (int64_t)T * R;
    // position 0: every state (a free first state), or the 2^k successors of the given start
    const int st0 = start ? start[row] : -1;
    {
        const float x0 = xr[0];
        for (int s = tid; s < NS; s += LAMQ_WIDE_NT) {
            const float d = x0 - C[s];
            const float q = d * d;
            cost[s] = (st0 < 0 || (s >> k) == (st0 & (R - 1))) ? q : __builtin_inff();
        }
    }
    const int tpg = R < LAMQ_WIDE_NT ? LAMQ_WIDE_NT / R : 1;  // threads per group
    for (int t = 1; t < T; ++t) {
        __syncthreads();  // cost of position t - 1 complete
        if (R < LAMQ_WIDE_NT) {
            const int g = tid / tpg, j = tid - g * tpg;
            float bv = __builtin_inff();
            int bh = NB;
            for (int h = j; h < NB; h += tpg) {
                const float v = cost[h * R + g];
                if (v < bv || bh == NB) {  // the first member, then strictly smaller ones: the lowest h of a tie
                    bv = v;
                    bh = h;
                }
            }
            pv[tid] = bv;
            ph[tid] = bh;
            __syncthreads();
            if (j == 0) {
                for (int i = 1; i < tpg; ++i)
                    if (wide_better(pv[tid + i], ph[tid + i], bv, bh)) {
                        bv = pv[tid + i];
                        bh = ph[tid + i];
                    }
                best[g] = bv;
                back[(int64_t)t * R + g] = (uint8_t)bh;
            }
            __syncthreads();  // every read of cost and pv done, best complete
            const float xt = xr[t];
            for (int s = tid; s < NS; s += LAMQ_WIDE_NT) {
                const float d = xt - C[s];
                const float q = d * d;
                cost[s] = best[s >> k] + q;
            }
        } else {
            // R >= 256 groups (k small against L): each thread scans its groups whole; the minima go to the
            // registers of the states' owners through the cost array itself, group g's minimum written over its
            // member h = 0 (cost[g]) once every thread has read its groups
            // (register arrays with compile-time bounds, the loops unrolled and guarded: no scratch)
            constexpr int MAXI = (1 << LAMQ_WIDE_MAX_L) / LAMQ_WIDE_NT;
            float gm[MAXI / 2];
            const int gpt = R / LAMQ_WIDE_NT;
#pragma unroll
            for (int i = 0; i < MAXI / 2; ++i) {
                if (i < gpt) {
                    const int g = tid + LAMQ_WIDE_NT * i;
                    float bv = cost[g];
                    int bh = 0;
                    for (int h = 1; h < NB; ++h) {
                        const float v = cost[h * R + g];
                        if (v < bv) {
                            bv = v;
                            bh = h;
                        }
                    }
                    gm[i] = bv;
                    back[(int64_t)t * R + g] = (uint8_t)bh;
                }
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < MAXI / 2; ++i)
                if (i < gpt) cost[tid + LAMQ_WIDE_NT * i] = gm[i];
            __syncthreads();
            // every state's new cost reads a minimum (cost[s >> k], s >> k < R) before any is overwritten (a barrier
            // between)
            const float xt = xr[t];
            float nc[MAXI];
            const int spt = NS / LAMQ_WIDE_NT;
#pragma unroll
            for (int i = 0; i < MAXI; ++i) {
                if (i < spt) {
                    const int s = tid + LAMQ_WIDE_NT * i;
                    const float d = xt - C[s];
                    nc[i] = cost[s >> k] + d * d;
                }
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < MAXI; ++i)
                if (i < spt) cost[tid + LAMQ_WIDE_NT * i] = nc[i];
        }
    }
    __syncthreads();
    // the final state: the lowest state of least cost
    {
        float bv = __builtin_inff();
        int bs = NS;
        for (int s = tid; s < NS; s += LAMQ_WIDE_NT) {
            const float v = cost[s];
            if (v < bv || bs == NS) {
                bv = v;
                bs = s;
            }
        }
        pv[tid] = bv;
        ph[tid] = bs;
        __syncthreads();
        if (tid == 0) {
            for (int i = 1; i < LAMQ_WIDE_NT; ++i)
                if (ph[i] < NS && wide_better(pv[i], ph[i], bv, bs)) {
                    bv = pv[i];
                    bs = ph[i];
                }
            arg_s = bs;
        }
        __syncthreads();
    }
    if (tid == 0) {
        int32_t* out = states + row * lds;
        int s = arg_s;
        out[T - 1] = s;
        for (int t = T - 1; t > 0; --t) {
            const int r = s >> k;
            s = r + (int)back[(int64_t)t * R + r] * R;
            out[t - 1] = s;
        }
    }
}

// (L, k) the wide search takes: what dispatch_lk has no kernel for, up to k = 8 (the reference's uint8
// back-pointers) and 2^LAMQ_WIDE_MAX_L states
static bool wide_lk(int L, int k)
{
    size_t act = 0;
    return L >= 1 && L <= LAMQ_WIDE_MAX_L && k >= 1 && k <= 8 && k <= L &&
           dispatch_lk<ActOf>(L, k, &act) == LAMQ_EUNSUP;
}



// ------------------------------------------------------------------------------------------------
// ldlq_trellis_block: one workgroup per row walks the steps j = b0, b0+width, ... of the lazy block
// [b0, b1). Per step (opgraph/syntax.py:109-121 with codes.py:442-450 and :397-404):
//   xs    = float32(T[j : j+w+a] / S)       w settled columns, a <= look look-ahead columns, which
//           beyond b1 still lack this block's trailing update (they are read as they stand)
//   path  = viterbi(xs, start = state)[:w];  state = path[w-1]
//   then the refit of trellis.h (E, z = E U_BB^-1, the in-block update of the columns up to b1).
// The block's columns of T live in LDS for the whole block; T in HBM is not written (the settled
// values are table64[states] * S; columns >= b1 get the trailing update from Z afterwards).
// ------------------------------------------------------------------------------------------------
template <int L, int K>
struct alignas(16) BlkSmem {
    using V = VX<L, K, LAMQ_NT>;
    float buf[2 * V::R];
    uint8_t back[(LAMQ_TV_BLK - 1) * V::ACT];
    double trow[LAMQ_LAZY_MAX + LAMQ_TV_BLK];
    double urows[LAMQ_WMAX][LAMQ_LAZY_MAX];
    double zs[LAMQ_WMAX];
    float xs[LAMQ_TV_BLK];
    int path[LAMQ_TV_BLK];
    float red[2 * (LAMQ_NT / 64)];
};

// One row's lazy block [b0, b1): `row` indexes T, S, state, states and Z.
template <int L, int K>
__device__ __forceinline__ void trellis_block_row(BlkSmem<L, K>& sm, int64_t row, const double* __restrict__ T, int64_t n,
                                                  int64_t ldT, const double* __restrict__ U, int64_t ldU,
                                                  const double* __restrict__ S, const double* __restrict__ table64,
                                                  const float* __restrict__ table32, int64_t b0, int64_t b1, int width,
                                                  int look, int32_t* __restrict__ state, int32_t* __restrict__ states,
                                                  int64_t lds, double* __restrict__ Z, int64_t ldZ, int pre)
{
    using V = VX<L, K, LAMQ_NT>;
    const int tid = threadIdx.x;
    const int64_t cend = (b1 + look < n) ? b1 + look : n;
    load_block_row<LAMQ_NT>(sm.trow, T + row * ldT, b0, (int)(b1 - b0), (int)(cend - b0), Z + row * ldZ - pre, pre, U,
                            ldU);
    TabF32<V> tab;
    if (tid < V::ACT) tab.load(table32, tid);
    const double Sr = S[row];
    int st = state[row];
    lds_barrier();

    for (int64_t j = b0; j < b1; j += width) {
        const int w = (int)((j + width <= b1) ? width : (b1 - j));
        const int64_t ahead = n - (j + w);
        const int a = (int)(ahead < look ? ahead : look);
        const int TV = w + a;
        const int jo = (int)(j - b0);
        const int nc = (int)(b1 - j - w);
        refit_fetch_lds<LAMQ_NT, LAMQ_LAZY_MAX>(sm.urows, U, ldU, j, w, b1);
        if (tid < TV) sm.xs[tid] = (float)(sm.trow[jo + tid] / Sr);
        lds_barrier();
        const int pv = viterbi_gx<L, K, LAMQ_NT, true, false, true>(sm.xs, TV, tab, st, sm.buf, sm.back, sm.path, sm.red);
        refit_apply_lds<LAMQ_NT, LAMQ_LAZY_MAX>(sm.urows, sm.trow, jo, w, nc, pv, table64, Sr, states + row * lds + j,
                                                Z + row * ldZ + jo, sm.zs);
        st = sm.path[w - 1];
    }
    if (tid == 0) state[row] = st;
}

template <int L, int K>
__global__ __launch_bounds__(LAMQ_NT) void ldlq_trellis_block_kernel(
    const double* __restrict__ T, int64_t n, int64_t ldT, const double* __restrict__ U, int64_t ldU,
    const double* __restrict__ S, const double* __restrict__ table64, const float* __restrict__ table32,
    int64_t b0, int64_t b1, int width, int look, int32_t* __restrict__ state, int32_t* __restrict__ states,
    int64_t lds, double* __restrict__ Z, int64_t ldZ, int pre)
{
    __shared__ BlkSmem<L, K> sm;
    trellis_block_row<L, K>(sm, blockIdx.x, T, n, ldT, U, ldU, S, table64, table32, b0, b1, width, look, state, states,
                            lds, Z, ldZ, pre);
}

template <int L, int K>
struct TrellisBlock {
    static int run(const double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU, const double* S,
                   const double* table64, const float* table32, int64_t b0, int64_t b1, int width, int look,
                   int32_t* state, int32_t* states, int64_t lds, double* Z, int64_t ldZ, int pre, hipStream_t s)
    {
        hipLaunchKernelGGL((ldlq_trellis_block_kernel<L, K>), dim3((unsigned)m), dim3(LAMQ_NT), 0, s, T, n, ldT, U, ldU, S,
                           table64, table32, b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
};

extern "C" int lamq_ldlq_trellis_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                       const double* S, const double* table64, const float* table32, int L, int k,
                                       int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                                       int64_t lds, double* Z, int64_t ldZ, int64_t pre, void* stream)
{
    if (!T || !U || !S || !table64 || !table32 || !state || !states || !Z) return LAMQ_EINVAL;
    if (m < 0 || n < 1 || ldT < n || ldU < n || lds < n || b0 < 0 || b1 <= b0 || b1 > n || width < 1 || look < 0)
        return LAMQ_EINVAL;
    if (pre < 0 || pre > b0 || ldZ < pre + (b1 - b0)) return LAMQ_EINVAL;
    if (pre > LAMQ_PRE_MAX) return LAMQ_EUNSUP;
    if (width > LAMQ_WMAX || width + look > LAMQ_TV_BLK || b1 - b0 > LAMQ_LAZY_MAX || m > 0x7fffffff)
        return LAMQ_EUNSUP;
    if (m == 0) return LAMQ_OK;
    return dispatch_lk<TrellisBlock>(L, k, T, m, n, ldT, U, ldU, S, table64, table32, b0, b1, width, look, state,
                                     states, lds, Z, ldZ, (int)pre, as_stream(stream));
}

// ------------------------------------------------------------------------------------------------ row groups at once
// One launch for every row group of a stage at L = 12 (the reference's fitted tables): a launch per group ends in a
// tail of partly idle CUs (four 256-thread rows per CU, so ceil(rows / 1024) rounds), which one launch over all their
// rows does not have. Workgroup b takes row b of the concatenated groups (in the table's order), finds its group (a
// uniform scan of at most LAMQ_TRELLIS_MAX_GROUPS entries) and runs that width's block in that width's LDS layout
// over one shared array (the widest layout's size: four workgroups per CU as for each width alone).
#define LAMQ_GROUPS_L 12
struct BlkGroup {
    int64_t r0, rows;
    const double* table64;
    const float* table32;
    int k;
};
struct BlkGroups {
    BlkGroup g[LAMQ_TRELLIS_MAX_GROUPS];
    int count;
};

template <int L>
constexpr int blk_groups_smem_bytes()
{
    int b = (int)sizeof(BlkSmem<L, 1>);
    b = (int)sizeof(BlkSmem<L, 2>) > b ? (int)sizeof(BlkSmem<L, 2>) : b;
    b = (int)sizeof(BlkSmem<L, 3>) > b ? (int)sizeof(BlkSmem<L, 3>) : b;
    b = (int)sizeof(BlkSmem<L, 4>) > b ? (int)sizeof(BlkSmem<L, 4>) : b;
    return b;
}

template <int L>
__global__ __launch_bounds__(LAMQ_NT) void ldlq_trellis_groups_kernel(
    const double* __restrict__ T, int64_t n, int64_t ldT, const double* __restrict__ U, int64_t ldU,
    const double* __restrict__ S, int64_t b0, int64_t b1, int width, int look, int32_t* __restrict__ state,
    int32_t* __restrict__ states, int64_t lds, double* __restrict__ Z, int64_t ldZ, int pre, BlkGroups groups)
{
    static_assert(blk_groups_smem_bytes<L>() * 4 <= 160 * 1024, "four workgroups per CU");
    __shared__ __align__(16) uint8_t raw[blk_groups_smem_bytes<L>()];
    int64_t b = blockIdx.x;
    int i = 0;
    while (i + 1 < groups.count && b >= groups.g[i].rows) {
        b -= groups.g[i].rows;
        ++i;
    }
    const BlkGroup& G = groups.g[i];
    const int64_t row = G.r0 + b;
    switch (G.k) {
    case 1:
        trellis_block_row<L, 1>(*reinterpret_cast<BlkSmem<L, 1>*>(raw), row, T, n, ldT, U, ldU, S, G.table64, G.table32,
                                b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        break;
    case 2:
        trellis_block_row<L, 2>(*reinterpret_cast<BlkSmem<L, 2>*>(raw), row, T, n, ldT, U, ldU, S, G.table64, G.table32,
                                b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        break;
    case 3:
        trellis_block_row<L, 3>(*reinterpret_cast<BlkSmem<L, 3>*>(raw), row, T, n, ldT, U, ldU, S, G.table64, G.table32,
                                b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        break;
    default:
        trellis_block_row<L, 4>(*reinterpret_cast<BlkSmem<L, 4>*>(raw), row, T, n, ldT, U, ldU, S, G.table64, G.table32,
                                b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        break;
    }
}

extern "C" int lamq_ldlq_trellis_block_groups(double* T, int64_t m, int64_t n, int64_t ldT, const double* U,
                                              int64_t ldU, const double* S, int L,
                                              const lamq_trellis_group32* groups, int ngroups, int64_t b0, int64_t b1,
                                              int width, int look, int32_t* state, int32_t* states, int64_t lds,
                                              double* Z, int64_t ldZ, int64_t pre, void* stream)
{
    if (!T || !U || !S || !state || !states || !Z || !groups) return LAMQ_EINVAL;
    if (ngroups < 1 || ngroups > LAMQ_TRELLIS_MAX_GROUPS) return LAMQ_EINVAL;
    if (m < 0 || n < 1 || ldT < n || ldU < n || lds < n || b0 < 0 || b1 <= b0 || b1 > n || width < 1 || look < 0)
        return LAMQ_EINVAL;
    if (pre < 0 || pre > b0 || ldZ < pre + (b1 - b0)) return LAMQ_EINVAL;
    if (pre > LAMQ_PRE_MAX) return LAMQ_EUNSUP;
    if (width > LAMQ_WMAX || width + look > LAMQ_TV_BLK || b1 - b0 > LAMQ_LAZY_MAX || m > 0x7fffffff)
        return LAMQ_EUNSUP;
    if (L != LAMQ_GROUPS_L) return LAMQ_EUNSUP;
    BlkGroups gg{};
    int64_t total = 0;
    for (int i = 0; i < ngroups; ++i) {
        const lamq_trellis_group32& g = groups[i];
        if (g.r0 < 0 || g.rows < 0 || g.r0 > m - g.rows) return LAMQ_EINVAL;
        if (!g.table64 || !g.table32) return LAMQ_EINVAL;
        if (g.k < 1 || g.k > 4) return LAMQ_EUNSUP;
        for (int j = 0; j < i; ++j)  // the row ranges do not overlap
            if (g.rows && groups[j].rows && g.r0 < groups[j].r0 + groups[j].rows && groups[j].r0 < g.r0 + g.rows)
                return LAMQ_EINVAL;
        gg.g[i].r0 = g.r0;
        gg.g[i].rows = g.rows;
        gg.g[i].table64 = g.table64;
        gg.g[i].table32 = g.table32;
        gg.g[i].k = g.k;
        total += g.rows;
    }
    gg.count = ngroups;
    if (total == 0) return LAMQ_OK;
    hipLaunchKernelGGL((ldlq_trellis_groups_kernel<LAMQ_GROUPS_L>), dim3((unsigned)total), dim3(LAMQ_NT), 0,
                       as_stream(stream), T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, (int)pre,
                       gg);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

extern "C" size_t lamq_viterbi_workspace_size(int64_t B, int T, int L, int k)
{
    if (B < 0 || T < 1) return 0;
    if (wide_lk(L, k)) return (size_t)B * (size_t)T * ((size_t)1 << (L - k));  // a byte per group and position
    if (T <= LAMQ_TV_LDS) return 0;
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
    if (wide_lk(L, k)) {
        if (!workspace || workspace_bytes < lamq_viterbi_workspace_size(B, T, L, k)) return LAMQ_EINVAL;
        hipLaunchKernelGGL(viterbi_wide_kernel, dim3((unsigned)B), dim3(LAMQ_WIDE_NT), 0, as_stream(stream), x, T, ldx,
                           C, L, k, start, states, lds, (uint8_t*)workspace);
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
    return dispatch_lk<ViterbiRows>(L, k, x, B, T, ldx, C, start, states, lds, workspace, workspace_bytes,
                                    as_stream(stream));
}
