// Trellis search with 2^13 .. 2^16 states (the 16-bit-state configurations), standalone and fused into the
// row-trellis LDLQ block. One 1024-thread workgroup per row; the state values are packed fp16 in VGPRs (the
// kernels take tables whose values fp16 holds exactly, as the 16-bit configurations' Gaussian-quantile table;
// x - C is then exact in float32). Back-pointers are one 32-bit word per thread and step (G*k <= 32 bits), in LDS.
//
// Up to 2^14 groups (every configuration but L = 16, k = 1) the search is trellis.h's: only the group minima
// (at most 64 KB) pass through LDS each step.
//
// L = 16, k = 1 (2^15 groups, 128 KB of minima) keeps the quarter-window search below. The states are cut into
// four quarters of QS = 2^(L-2); thread t owns the SQ = 2^L/4096 consecutive states [q*QS + SQ*t, q*QS + SQ*t + SQ)
// of every quarter q. Those are exactly the successors of its predecessor groups r = q*QS/2^k + SQ*t/2^k + g
// (g < SQ/2^k), so a thread needs, per step, the path costs of the states h*2^(L-k) + r of its groups, which
// other threads own. They are exchanged through an LDS window of one quarter: in phase p every thread writes its
// own states of quarter p and then folds those of its predecessors that lie in quarter p, so all 16 waves work in
// every phase. Predecessors reach a group in increasing h (a quarter index never decreases with h, and within a
// phase h is visited in increasing order), so the strict comparison keeps the lowest h on ties, as torch's min
// does. Between steps a thread keeps only the minimum of each of its groups: the path cost of its state (g, b) is
// bprev[g] + (x_prev - C)^2, formed again when written to the window with the same three rounded operations,
// hence the same float32 value.
#include "trellis.h"

#define BIG_NT 1024
#define BIG_TV 24       // longest fused search: width + look
#define BIG_LAZY 128
#define BIG_GX_MAX_R 16384  // most groups of the minima-exchange search (64 KB of LDS)
// most groups whose back-pointers the merged row-group kernel keeps in LDS; above, they go to the workspace, and the
// LDS they leave holds a second minima buffer (one barrier a step instead of two)
#ifndef BIG_BACK_LDS_MAX_R
#define BIG_BACK_LDS_MAX_R 8192
#endif

template <int L, int K>
struct VBig {
    static constexpr int NS = 1 << L;
    static constexpr int R = 1 << (L - K);
    static constexpr int NB = 1 << K;
    static constexpr int SPT = NS / BIG_NT;  // states per thread
    static constexpr int SQ = SPT / 4;       // states per thread and quarter
    static constexpr int QS = NS / 4;        // states per quarter (the exchange window)
    static constexpr int GQ = SQ / NB;       // predecessor groups per thread and quarter
    static constexpr int G = 4 * GQ;         // predecessor groups per thread
    static constexpr int RQ = QS / NB;       // group indices per quarter of states
    static_assert(SQ >= NB && SQ >= 2 && G * K <= 32, "layout");
    // quarter of the predecessors h*R + r of the groups of quarter q (independent of the thread, see above)
    static constexpr int quarter(int h, int q) { return (h * R + q * RQ) / QS; }
    // with K = 1 the second predecessors of the quarters' groups are visited in increasing quarter (phases in order)
    static constexpr bool second_in_order()
    {
        for (int q = 1; q < 4; ++q)
            if (quarter(1, q) < quarter(1, q - 1)) return false;
        return true;
    }
    static constexpr int offset(int h, int q) { return (h * R + q * RQ) % QS; }
};

template <int SPT>
__device__ __forceinline__ float xmc(float x, const uint32_t (&Ch)[SPT / 2], int i)
{
    return (i & 1) ? xmc_hi(x, Ch[i >> 1]) : xmc_lo(x, Ch[i >> 1]);
}

// Search one path of TV steps; thread 0 writes path[0..TV). xs: TV float32 targets. start < 0: free first state.
// xbuf: QS floats of LDS (indexed through swz). back: (TV-1)*1024 words (LDS or global). red: 32 words of LDS.
template <int L, int K>
__device__ void viterbi_big(const float* xs, int TV, uint32_t (&Ch)[VBig<L, K>::SPT / 2], int start, float* xbuf,
                            uint32_t* back, int* path, float* red)
{
    using V = VBig<L, K>;
    static_assert(K != 1 || V::second_in_order(), "K = 1 shifts the groups' bits in increasing group order");
    const int tid = threadIdx.x;
    float bprev[V::G];  // index q*GQ + g
    {
        const int rs = start >= 0 ? (start & (V::R - 1)) : -1;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int g = 0; g < V::GQ; ++g)
                bprev[q * V::GQ + g] = (rs >= 0 && q * V::RQ + V::GQ * tid + g != rs) ? __builtin_inff() : 0.0f;
    }
    float xprev = xs[0];
    for (int t = 1; t < TV; ++t) {
        // best[j]: minimum so far of group j = q*GQ + g; hw[j]: its winning h, packed into bits [j*K, j*K+K) once per
        // step. With 16 predecessors (K = 4) hw holds h itself, an inline constant of the selects (the compiler
        // schedules this form better there); otherwise h already shifted into place. With more than 16 groups a
        // thread has no registers to spare for hw: the h go straight into bits.
        constexpr bool SEP = V::G <= 16;
        constexpr bool SMALL_H = K >= 4;
        float best[V::G];
        uint32_t hw[SEP ? V::G : 1];
        uint32_t bits = 0;  // the winning h of group j in bits [j*K, j*K+K)
#pragma unroll
        for (int p = 0; p < 4; ++p) {
#pragma unroll
            for (int i = 0; i < V::SPT / 2; ++i) asm volatile("" : "+v"(Ch[i]));
            {
                float c[V::SQ];
#pragma unroll
                for (int i = 0; i < V::SQ; ++i) {
                    const float d = xmc<V::SPT>(xprev, Ch, p * V::SQ + i);
                    const float dd = d * d;
                    c[i] = bprev[p * V::GQ + i / V::NB] + dd;
                }
                lds_store_swz<V::SQ>(xbuf, V::SQ * tid, c);
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int h = 0; h < V::NB; ++h) {
                    if (V::quarter(h, q) != p) continue;
                    float c[V::GQ];
                    lds_load_swz<V::GQ>(xbuf, V::offset(h, q) + V::GQ * tid, c);
#pragma unroll
                    for (int g = 0; g < V::GQ; ++g) {
                        const int j = q * V::GQ + g;
                        if (h == 0) {  // the first predecessor of every group (phases visit h in increasing order)
                            best[j] = c[g];
                            if (SEP) hw[j] = 0;
                        } else if constexpr (K == 1) {
                            // the second predecessor wins only if strictly lower; its bit enters `bits` as a carry-in,
                            // groups in increasing j (static_assert below), so group j's bit lands at G - 1 - j
                            const uint64_t lt = __builtin_amdgcn_ballot_w64(c[g] < best[j]);
                            best[j] = fminf(best[j], c[g]);
                            bits = shift_in(bits, lt);
                        } else {
                            const bool lt = c[g] < best[j];  // strict: the lowest h keeps a tie
                            best[j] = lt ? c[g] : best[j];
                            if (SEP) {
                                hw[j] = lt ? (SMALL_H ? (uint32_t)h : (uint32_t)h << (j * K)) : hw[j];
                            } else {
                                const uint32_t mk = (uint32_t)(V::NB - 1) << (j * K);
                                bits = lt ? ((bits & ~mk) | ((uint32_t)h << (j * K))) : bits;
                            }
                        }
                    }
                }
            __syncthreads();
        }
        if (SEP && SMALL_H) {
            // the empty asm keeps the compiler from folding the shift back into the selects
#pragma unroll
            for (int j = 0; j < V::G; ++j) asm volatile("" : "+v"(hw[j]));
#pragma unroll
            for (int j = 0; j < V::G; ++j) bits |= hw[j] << (j * K);
        } else if (SEP) {
#pragma unroll
            for (int j = 0; j < V::G; ++j) bits |= hw[j];
        }
#pragma unroll
        for (int j = 0; j < V::G; ++j) bprev[j] = best[j];
        back[(t - 1) * BIG_NT + tid] = bits;
        xprev = xs[t];
    }
    // final argmin, lowest state on ties (a thread's states increase with (q, i))
    float bv = __builtin_inff();
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < V::SPT / 2; ++i) asm volatile("" : "+v"(Ch[i]));
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < V::SQ; ++i) {
            const float d = xmc<V::SPT>(xprev, Ch, q * V::SQ + i);
            const float dd = d * d;
            const float c = bprev[q * V::GQ + i / V::NB] + dd;
            if ((q == 0 && i == 0) || c < bv) { bv = c; bi = q * V::QS + V::SQ * tid + i; }
        }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov < bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    int* redi = reinterpret_cast<int*>(red + 16);
    if ((tid & 63) == 0) { red[tid >> 6] = bv; redi[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
        float v = red[0];
        int s = redi[0];
        for (int w = 1; w < BIG_NT / 64; ++w)
            if (red[w] < v || (red[w] == v && redi[w] < s)) { v = red[w]; s = redi[w]; }
        path[TV - 1] = s;
        for (int t = TV - 1; t > 0; --t) {
            const int r = s >> K;
            const int q = r / V::RQ, rem = r - q * V::RQ;
            const int owner = rem / V::GQ, g = rem - owner * V::GQ;
            const int j = q * V::GQ + g;
            const int pos = K == 1 ? V::G - 1 - j : j * K;  // K = 1: the bits were shifted in, group 0 first
            const int h = (int)((back[(t - 1) * BIG_NT + owner] >> pos) & (uint32_t)(V::NB - 1));
            s = r + h * V::R;
            path[t - 1] = s;
        }
    }
    __syncthreads();
}

// this thread's state values: quarter q, states q*QS + SQ*t + i, packed two per register in (q, i) order
template <int L, int K>
__device__ __forceinline__ void load_half_table(const uint16_t* __restrict__ table16, uint32_t (&Ch)[VBig<L, K>::SPT / 2])
{
    using V = VBig<L, K>;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(table16 + q * V::QS + V::SQ * threadIdx.x);
#pragma unroll
        for (int i = 0; i < V::SQ / 2; ++i) Ch[q * V::SQ / 2 + i] = src[i];
    }
}

// ------------------------------------------------------------------------------------------------ standalone
template <int L, int K, bool BACK_GLOBAL>
__global__ __launch_bounds__(BIG_NT) void viterbi_rows_big_kernel(const float* __restrict__ x, int T, int64_t ldx,
                                                                  const uint16_t* __restrict__ table16,
                                                                  const int32_t* __restrict__ start,
                                                                  int32_t* __restrict__ states, int64_t lds,
                                                                  uint32_t* __restrict__ back_ws)
{
    using V = VBig<L, K>;
    __shared__ __align__(16) float xbuf[V::QS];
    __shared__ uint32_t back_lds[BACK_GLOBAL ? 1 : (BIG_TV - 1) * BIG_NT];
    __shared__ float red[32];
    const int64_t row = blockIdx.x;
    uint32_t Ch[V::SPT / 2];
    load_half_table<L, K>(table16, Ch);
    uint32_t* back = BACK_GLOBAL ? back_ws + row * (int64_t)(T - 1) * BIG_NT : back_lds;
    viterbi_big<L, K>(x + row * ldx, T, Ch, start ? start[row] : -1, xbuf, back, states + row * lds, red);
}

// minima-exchange search (trellis.h), for up to BIG_GX_MAX_R groups
template <int L, int K, bool BACK_GLOBAL>
__global__ __launch_bounds__(BIG_NT) void viterbi_rows_gx_kernel(const float* __restrict__ x, int T, int64_t ldx,
                                                                 const uint16_t* __restrict__ table16,
                                                                 const int32_t* __restrict__ start,
                                                                 int32_t* __restrict__ states, int64_t lds,
                                                                 uint32_t* __restrict__ back_ws)
{
    using V = VX<L, K, BIG_NT>;
    constexpr bool DBL = V::R <= 4096;
    __shared__ __align__(16) float buf[(DBL ? 2 : 1) * V::R];
    __shared__ uint32_t back_lds[BACK_GLOBAL ? 1 : (BIG_TV - 1) * V::ACT];
    __shared__ float red[2 * (BIG_NT / 64)];
    const int64_t row = blockIdx.x;
    TabF16<V> tab;
    tab.load(table16, threadIdx.x);
    uint32_t* back = BACK_GLOBAL ? back_ws + row * (int64_t)(T - 1) * BIG_NT : back_lds;
    viterbi_gx<L, K, BIG_NT, DBL, BACK_GLOBAL>(x + row * ldx, T, tab, start ? start[row] : -1, buf, back,
                                             states + row * lds, red);
}

template <int L, int K>
struct ViterbiRowsBig {
    static int run(const float* x, int64_t B, int T, int64_t ldx, const uint16_t* table16, const int32_t* start,
                   int32_t* states, int64_t lds, void* ws, size_t ws_bytes, hipStream_t s)
    {
        constexpr bool GX = VX<L, K, BIG_NT>::R <= BIG_GX_MAX_R;
        if (T <= BIG_TV) {
            if constexpr (GX)
                hipLaunchKernelGGL((viterbi_rows_gx_kernel<L, K, false>), dim3((unsigned)B), dim3(BIG_NT), 0, s, x, T, ldx,
                                   table16, start, states, lds, (uint32_t*)nullptr);
            else
                hipLaunchKernelGGL((viterbi_rows_big_kernel<L, K, false>), dim3((unsigned)B), dim3(BIG_NT), 0, s, x, T, ldx,
                                   table16, start, states, lds, (uint32_t*)nullptr);
        } else {
            const size_t need = (size_t)B * (size_t)(T - 1) * BIG_NT * sizeof(uint32_t);
            if (!ws || ws_bytes < need) return LAMQ_EINVAL;
            if constexpr (GX)
                hipLaunchKernelGGL((viterbi_rows_gx_kernel<L, K, true>), dim3((unsigned)B), dim3(BIG_NT), 0, s, x, T, ldx,
                                   table16, start, states, lds, (uint32_t*)ws);
            else
                hipLaunchKernelGGL((viterbi_rows_big_kernel<L, K, true>), dim3((unsigned)B), dim3(BIG_NT), 0, s, x, T, ldx,
                                   table16, start, states, lds, (uint32_t*)ws);
        }
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
};

template <template <int, int> class F, typename... Args>
static int dispatch_big(int L, int K, Args&&... args)
{
#define BIG_CASE(l, k) \
    if (L == l && K == k) return F<l, k>::run(args...);
    BIG_CASE(16, 1) BIG_CASE(16, 2) BIG_CASE(16, 3) BIG_CASE(16, 4)
    BIG_CASE(15, 1) BIG_CASE(15, 2) BIG_CASE(15, 3)
    BIG_CASE(14, 1) BIG_CASE(14, 2)
    BIG_CASE(13, 1)
#undef BIG_CASE
    return LAMQ_EUNSUP;
}

extern "C" size_t lamq_viterbi16_workspace_size(int64_t B, int T, int L, int k)
{
    (void)L;
    (void)k;
    if (B < 0 || T <= BIG_TV) return 0;
    return (size_t)B * (size_t)(T - 1) * BIG_NT * sizeof(uint32_t);
}

extern "C" int lamq_viterbi16_rows(const float* x, int64_t B, int T, int64_t ldx, const uint16_t* table16, int L, int k,
                                   const int32_t* start, int32_t* states, int64_t lds, void* workspace,
                                   size_t workspace_bytes, void* stream)
{
    if (!x || !table16 || !states || B < 0 || T < 1 || ldx < T || lds < T) return LAMQ_EINVAL;
    if (((uintptr_t)table16 % 4) != 0) return LAMQ_EINVAL;
    if (B == 0) return LAMQ_OK;
    if (B > 0x7fffffff) return LAMQ_EUNSUP;
    return dispatch_big<ViterbiRowsBig>(L, k, x, B, T, ldx, table16, start, states, lds, workspace, workspace_bytes,
                                        as_stream(stream));
}

// ------------------------------------------------------------------------------------------------ fused block
// The same per-step arithmetic as ldlq_trellis_block_kernel (viterbi.hip), with the 16-bit-state search.
template <int L, int K>
__global__ __launch_bounds__(BIG_NT) void ldlq_trellis_block_big_kernel(
    const double* __restrict__ T, int64_t n, int64_t ldT, const double* __restrict__ U, int64_t ldU,
    const double* __restrict__ S, const double* __restrict__ table64, const uint16_t* __restrict__ table16,
    int64_t b0, int64_t b1, int width, int look, int32_t* __restrict__ state, int32_t* __restrict__ states,
    int64_t lds, double* __restrict__ Z, int64_t ldZ, int pre)
{
    using V = VBig<L, K>;
    __shared__ __align__(16) float xbuf[V::QS];
    __shared__ uint32_t back[(BIG_TV - 1) * BIG_NT];
    __shared__ double trow[BIG_LAZY + BIG_TV];
    __shared__ float xs[BIG_TV];
    __shared__ int path[BIG_TV];
    __shared__ double es[BIG_TV];
    __shared__ double zs[BIG_TV];
    __shared__ float red[32];

    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    uint32_t Ch[V::SPT / 2];
    load_half_table<L, K>(table16, Ch);
    const int64_t cend = (b1 + look < n) ? b1 + look : n;
    load_block_row<BIG_NT>(trow, T + row * ldT, b0, (int)(b1 - b0), (int)(cend - b0), Z + row * ldZ - pre, pre, U,
                            ldU);
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
        viterbi_big<L, K>(xs, TV, Ch, st, xbuf, back, path, red);
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
        for (int64_t col = j + w + tid; col < b1; col += BIG_NT) {
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

// LDS of the fused minima-exchange kernel below: the block row and small arrays, the group minima (two buffers when
// they fit, which spares each step its second barrier: 2^12 groups, and 2^13 with the back-pointers in LDS, 163,456 of
// the 163,840 bytes), and the back-pointers unless they go to a workspace (BG).
template <int L, int K, bool BG>
constexpr int gx_lds_bytes(bool dbl)
{
    using V = VX<L, K, BIG_NT>;
    return 8 * (BIG_LAZY + BIG_TV) + 8 * LAMQ_WMAX * LAMQ_WMAX + 8 * LAMQ_WMAX + 4 * BIG_TV + 4 * BIG_TV +
           4 * 2 * (BIG_NT / 64) + 4 * (dbl ? 2 : 1) * V::R + 4 * (BG ? 1 : (BIG_TV - 1) * V::ACT);
}
template <int L, int K, bool BG>
constexpr bool gx_double_buffered() { return gx_lds_bytes<L, K, BG>(true) <= 160 * 1024; }

// The same with the minima-exchange search and the prefetched refit of trellis.h (four threads per column of the
// in-block update).
// BG: the back-pointers in back_ws, (BIG_TV - 1) * BIG_NT words per row, instead of LDS (the 2^15-group search,
// whose 128 KB of group minima leave no LDS for them)
template <int L, int K, bool BG>
struct alignas(16) GxSmem {
    using V = VX<L, K, BIG_NT>;
    static constexpr bool DBL = gx_double_buffered<L, K, BG>();
    // small arrays first: their addresses stay within the 16-bit offset of LDS instructions
    double trow[BIG_LAZY + BIG_TV];
    double ubb[LAMQ_WMAX * LAMQ_WMAX];
    double zs[LAMQ_WMAX];
    float xs[BIG_TV];
    int path[BIG_TV];
    float red[2 * (BIG_NT / 64)];
    float buf[(DBL ? 2 : 1) * V::R];
    uint32_t back[BG ? 1 : (BIG_TV - 1) * V::ACT];
};

// One row's lazy block [b0, b1): `row` indexes T, S, state, states and Z; `wrow` the row's back-pointer slot in back_ws
// (BG).
template <int L, int K, bool BG>
__device__ __forceinline__ void gx_block_row(GxSmem<L, K, BG>& sm, int64_t row, int64_t wrow,
                                             const double* __restrict__ T, int64_t n, int64_t ldT,
                                             const double* __restrict__ U, int64_t ldU, const double* __restrict__ S,
                                             const double* __restrict__ table64, const uint16_t* __restrict__ table16,
                                             int64_t b0, int64_t b1, int width, int look, int32_t* __restrict__ state,
                                             int32_t* __restrict__ states, int64_t lds, double* __restrict__ Z,
                                             int64_t ldZ, uint32_t* __restrict__ back_ws, int pre)
{
    using V = VX<L, K, BIG_NT>;
    constexpr bool DBL = GxSmem<L, K, BG>::DBL;
    double* trow = sm.trow;
    double* ubb = sm.ubb;
    double* zs = sm.zs;
    float* xs = sm.xs;
    int* path = sm.path;
    float* red = sm.red;
    float* buf = sm.buf;
    uint32_t* back = BG ? back_ws + wrow * (int64_t)((BIG_TV - 1) * V::ACT) : sm.back;
    const int tid = threadIdx.x;
    const int64_t cend = (b1 + look < n) ? b1 + look : n;
    load_block_row<BIG_NT>(trow, T + row * ldT, b0, (int)(b1 - b0), (int)(cend - b0), Z + row * ldZ - pre, pre, U,
                            ldU);
    TabF16<V> tab;
    tab.load(table16, tid);
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
        if (tid < TV) xs[tid] = (float)(trow[jo + tid] / Sr);
        lds_barrier();
        // the refit's U operands are fetched when the forward pass ends, under the final argmin and the traceback
        RefitRegs<4> ops;
        const int pv = viterbi_gx<L, K, BIG_NT, DBL, BG, true>(
            xs, TV, tab, st, buf, back, path, red, [&]() { refit_fetch_regs<BIG_NT, 4>(ops, U, ldU, j, w, nc); });
        refit_apply_regs<BIG_NT, 4>(ops, trow, jo, w, nc, pv, table64, Sr, states + row * lds + j, Z + row * ldZ + jo, ubb,
                               zs);
        st = path[w - 1];
    }
    if (tid == 0) state[row] = st;
}

template <int L, int K, bool BG>
__global__ __launch_bounds__(BIG_NT) void ldlq_trellis_block_gx_kernel(
    const double* __restrict__ T, int64_t n, int64_t ldT, const double* __restrict__ U, int64_t ldU,
    const double* __restrict__ S, const double* __restrict__ table64, const uint16_t* __restrict__ table16,
    int64_t b0, int64_t b1, int width, int look, int32_t* __restrict__ state, int32_t* __restrict__ states,
    int64_t lds, double* __restrict__ Z, int64_t ldZ, uint32_t* __restrict__ back_ws, int pre)
{
    __shared__ GxSmem<L, K, BG> sm;
    gx_block_row<L, K, BG>(sm, blockIdx.x, blockIdx.x, T, n, ldT, U, ldU, S, table64, table16, b0, b1, width, look, state,
                           states, lds, Z, ldZ, back_ws, pre);
}

// ------------------------------------------------------------------------------------------------ row groups at once
// One launch for every row group of a stage: the groups differ in bits per weight (k), and a launch per group ends in
// a tail of idle CUs (one 1024-thread row per CU, so ceil(rows / 256) rounds), which one launch over all their rows
// does not have. Workgroup b takes row b of the concatenated groups, finds its group (a uniform scan of at most
// LAMQ_TRELLIS_MAX_GROUPS entries) and runs that width's search in that width's LDS layout over one shared array.
struct GxGroup {
    int64_t r0, rows;
    const double* table64;
    const uint16_t* table16;
    uint32_t* back_ws;
    int k;
};
struct GxGroups {
    GxGroup g[LAMQ_TRELLIS_MAX_GROUPS];
    int count;
};

// back-pointers outside LDS: more groups than LDS holds next to their minima
template <int L, int K>
constexpr bool gx_back_global() { return VX<L, K, BIG_NT>::R > BIG_BACK_LDS_MAX_R; }

template <int L, int K>
constexpr int gx_smem_bytes() { return (int)sizeof(GxSmem<L, K, gx_back_global<L, K>()>); }

template <int L>
constexpr int gx_groups_smem_bytes()
{
    int b = 0;
    if constexpr (L - 12 >= 1) b = gx_smem_bytes<L, 1>() > b ? gx_smem_bytes<L, 1>() : b;
    if constexpr (L - 12 >= 2) b = gx_smem_bytes<L, 2>() > b ? gx_smem_bytes<L, 2>() : b;
    if constexpr (L - 12 >= 3) b = gx_smem_bytes<L, 3>() > b ? gx_smem_bytes<L, 3>() : b;
    if constexpr (L - 12 >= 4) b = gx_smem_bytes<L, 4>() > b ? gx_smem_bytes<L, 4>() : b;
    return b;
}

template <int L, int K>
__device__ __forceinline__ void gx_group_row(uint8_t* raw, const GxGroup& G, int64_t b, const double* T, int64_t n,
                                             int64_t ldT, const double* U, int64_t ldU, const double* S, int64_t b0,
                                             int64_t b1, int width, int look, int32_t* state, int32_t* states,
                                             int64_t lds, double* Z, int64_t ldZ, int pre)
{
    constexpr bool BG = gx_back_global<L, K>();
    gx_block_row<L, K, BG>(*reinterpret_cast<GxSmem<L, K, BG>*>(raw), G.r0 + b, b, T, n, ldT, U, ldU, S, G.table64,
                           G.table16, b0, b1, width, look, state, states, lds, Z, ldZ, G.back_ws, pre);
}

template <int L>
__global__ __launch_bounds__(BIG_NT) void ldlq_trellis_groups_gx_kernel(
    const double* __restrict__ T, int64_t n, int64_t ldT, const double* __restrict__ U, int64_t ldU,
    const double* __restrict__ S, int64_t b0, int64_t b1, int width, int look, int32_t* __restrict__ state,
    int32_t* __restrict__ states, int64_t lds, double* __restrict__ Z, int64_t ldZ, int pre, GxGroups groups)
{
    __shared__ __align__(16) uint8_t raw[gx_groups_smem_bytes<L>()];
    int64_t b = blockIdx.x;
    int i = 0;
    while (i + 1 < groups.count && b >= groups.g[i].rows) {
        b -= groups.g[i].rows;
        ++i;
    }
    const GxGroup& G = groups.g[i];
    switch (G.k) {
    case 1:
        if constexpr (L - 12 >= 1) gx_group_row<L, 1>(raw, G, b, T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        break;
    case 2:
        if constexpr (L - 12 >= 2) gx_group_row<L, 2>(raw, G, b, T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        break;
    case 3:
        if constexpr (L - 12 >= 3) gx_group_row<L, 3>(raw, G, b, T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        break;
    default:
        if constexpr (L - 12 >= 4) gx_group_row<L, 4>(raw, G, b, T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        break;
    }
}

template <int L, int K>
struct TrellisBlockBig {
    static int run(const double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU, const double* S,
                   const double* table64, const uint16_t* table16, int64_t b0, int64_t b1, int width, int look,
                   int32_t* state, int32_t* states, int64_t lds, double* Z, int64_t ldZ, uint32_t* back_ws, int pre,
                   hipStream_t s)
    {
        if constexpr (VX<L, K, BIG_NT>::R <= BIG_GX_MAX_R) {
            if (gx_back_global<L, K>() && back_ws)  // the back-pointers in the workspace, two minima buffers in LDS
                hipLaunchKernelGGL((ldlq_trellis_block_gx_kernel<L, K, true>), dim3((unsigned)m), dim3(BIG_NT), 0, s, T,
                                   n, ldT, U, ldU, S, table64, table16, b0, b1, width, look, state, states, lds, Z, ldZ,
                                   back_ws, pre);
            else
                hipLaunchKernelGGL((ldlq_trellis_block_gx_kernel<L, K, false>), dim3((unsigned)m), dim3(BIG_NT), 0, s, T,
                                   n, ldT, U, ldU, S, table64, table16, b0, b1, width, look, state, states, lds, Z, ldZ,
                                   nullptr, pre);
        } else if (back_ws)
            hipLaunchKernelGGL((ldlq_trellis_block_gx_kernel<L, K, true>), dim3((unsigned)m), dim3(BIG_NT), 0, s, T, n,
                               ldT, U, ldU, S, table64, table16, b0, b1, width, look, state, states, lds, Z, ldZ, back_ws,
                               pre);
        else
            hipLaunchKernelGGL((ldlq_trellis_block_big_kernel<L, K>), dim3((unsigned)m), dim3(BIG_NT), 0, s, T, n, ldT, U,
                               ldU, S, table64, table16, b0, b1, width, look, state, states, lds, Z, ldZ, pre);
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
};

extern "C" int lamq_ldlq_trellis16_block(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                         const double* S, const double* table64, const uint16_t* table16, int L, int k,
                                         int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                                         int64_t lds, double* Z, int64_t ldZ, int64_t pre, void* stream)
{
    if (!T || !U || !S || !table64 || !table16 || !state || !states || !Z) return LAMQ_EINVAL;
    if (((uintptr_t)table16 % 4) != 0) return LAMQ_EINVAL;
    if (m < 0 || n < 1 || ldT < n || ldU < n || lds < n || b0 < 0 || b1 <= b0 || b1 > n || width < 1 || look < 0)
        return LAMQ_EINVAL;
    if (pre < 0 || pre > b0 || ldZ < pre + (b1 - b0)) return LAMQ_EINVAL;
    if (width > LAMQ_WMAX || width + look > BIG_TV || b1 - b0 > BIG_LAZY || m > 0x7fffffff || pre > LAMQ_PRE_MAX)
        return LAMQ_EUNSUP;
    if (m == 0) return LAMQ_OK;
    return dispatch_big<TrellisBlockBig>(L, k, T, m, n, ldT, U, ldU, S, table64, table16, b0, b1, width, look, state,
                                         states, lds, Z, ldZ, (uint32_t*)nullptr, (int)pre, as_stream(stream));
}

extern "C" size_t lamq_ldlq_trellis16_block_workspace_size(int64_t m, int L, int k)
{
    if (m < 1 || L < 13 || L > 16 || k < 1 || k > L - 12 || k > 4) return 0;
    if ((1 << (L - k)) <= BIG_BACK_LDS_MAX_R) return 0;  // the back-pointers stay in LDS
    return (size_t)m * (size_t)(BIG_TV - 1) * BIG_NT * sizeof(uint32_t);
}

extern "C" int lamq_ldlq_trellis16_block_ws(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                                            const double* S, const double* table64, const uint16_t* table16, int L, int k,
                                            int64_t b0, int64_t b1, int width, int look, int32_t* state, int32_t* states,
                                            int64_t lds, double* Z, int64_t ldZ, int64_t pre, void* workspace,
                                            size_t workspace_bytes, void* stream)
{
    const size_t need = lamq_ldlq_trellis16_block_workspace_size(m, L, k);
    if (need == 0)
        return lamq_ldlq_trellis16_block(T, m, n, ldT, U, ldU, S, table64, table16, L, k, b0, b1, width, look, state,
                                         states, lds, Z, ldZ, pre, stream);
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace % 4) != 0) return LAMQ_EINVAL;
    if (!T || !U || !S || !table64 || !table16 || !state || !states || !Z) return LAMQ_EINVAL;
    if (((uintptr_t)table16 % 4) != 0) return LAMQ_EINVAL;
    if (m < 0 || n < 1 || ldT < n || ldU < n || lds < n || b0 < 0 || b1 <= b0 || b1 > n || width < 1 || look < 0)
        return LAMQ_EINVAL;
    if (pre < 0 || pre > b0 || ldZ < pre + (b1 - b0)) return LAMQ_EINVAL;
    if (width > LAMQ_WMAX || width + look > BIG_TV || b1 - b0 > BIG_LAZY || m > 0x7fffffff || pre > LAMQ_PRE_MAX)
        return LAMQ_EUNSUP;
    return dispatch_big<TrellisBlockBig>(L, k, T, m, n, ldT, U, ldU, S, table64, table16, b0, b1, width, look, state,
                                         states, lds, Z, ldZ, reinterpret_cast<uint32_t*>(workspace), (int)pre,
                                         as_stream(stream));
}

template <int L>
static void launch_groups(const GxGroups& gg, int64_t total, double* T, int64_t n, int64_t ldT, const double* U,
                          int64_t ldU, const double* S, int64_t b0, int64_t b1, int width, int look, int32_t* state,
                          int32_t* states, int64_t lds, double* Z, int64_t ldZ, int pre, hipStream_t s)
{
    hipLaunchKernelGGL((ldlq_trellis_groups_gx_kernel<L>), dim3((unsigned)total), dim3(BIG_NT), 0, s, T, n, ldT, U, ldU,
                       S, b0, b1, width, look, state, states, lds, Z, ldZ, pre, gg);
}

extern "C" int lamq_ldlq_trellis16_block_groups(double* T, int64_t m, int64_t n, int64_t ldT, const double* U,
                                                int64_t ldU, const double* S, int L, const lamq_trellis_group* groups,
                                                int ngroups, int64_t b0, int64_t b1, int width, int look,
                                                int32_t* state, int32_t* states, int64_t lds, double* Z, int64_t ldZ,
                                                int64_t pre, void* stream)
{
    if (!T || !U || !S || !state || !states || !Z || !groups) return LAMQ_EINVAL;
    if (ngroups < 1 || ngroups > LAMQ_TRELLIS_MAX_GROUPS) return LAMQ_EINVAL;
    if (m < 0 || n < 1 || ldT < n || ldU < n || lds < n || b0 < 0 || b1 <= b0 || b1 > n || width < 1 || look < 0)
        return LAMQ_EINVAL;
    if (pre < 0 || pre > b0 || ldZ < pre + (b1 - b0)) return LAMQ_EINVAL;
    if (width > LAMQ_WMAX || width + look > BIG_TV || b1 - b0 > BIG_LAZY || m > 0x7fffffff || pre > LAMQ_PRE_MAX)
        return LAMQ_EUNSUP;
    if (L < 13 || L > 16) return LAMQ_EUNSUP;
    GxGroups gg{};
    int64_t total = 0;
    for (int i = 0; i < ngroups; ++i) {
        const lamq_trellis_group& g = groups[i];
        if (g.r0 < 0 || g.rows < 0 || g.r0 > m - g.rows) return LAMQ_EINVAL;
        if (!g.table64 || !g.table16 || ((uintptr_t)g.table16 % 4) != 0) return LAMQ_EINVAL;
        if (g.k < 1 || g.k > 4 || g.k > L - 12) return LAMQ_EUNSUP;
        const size_t need = lamq_ldlq_trellis16_block_workspace_size(g.rows, L, g.k);
        if (need && (!g.workspace || g.workspace_bytes < need || ((uintptr_t)g.workspace % 4) != 0)) return LAMQ_EINVAL;
        for (int j = 0; j < i; ++j)  // the row ranges do not overlap
            if (g.rows && groups[j].rows && g.r0 < groups[j].r0 + groups[j].rows && groups[j].r0 < g.r0 + g.rows)
                return LAMQ_EINVAL;
        gg.g[i].r0 = g.r0;
        gg.g[i].rows = g.rows;
        gg.g[i].table64 = g.table64;
        gg.g[i].table16 = g.table16;
        gg.g[i].back_ws = reinterpret_cast<uint32_t*>(g.workspace);
        gg.g[i].k = g.k;
        total += g.rows;
    }
    gg.count = ngroups;
    if (total == 0) return LAMQ_OK;
    hipStream_t s = as_stream(stream);
    switch (L) {
    case 13: launch_groups<13>(gg, total, T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, (int)pre, s); break;
    case 14: launch_groups<14>(gg, total, T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, (int)pre, s); break;
    case 15: launch_groups<15>(gg, total, T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, (int)pre, s); break;
    default: launch_groups<16>(gg, total, T, n, ldT, U, ldU, S, b0, b1, width, look, state, states, lds, Z, ldZ, (int)pre, s); break;
    }
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
