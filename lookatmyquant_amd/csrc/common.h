// Shared definitions for the gfx950 kernels of the per-matrix quantization hot path.
// Every translation unit is built with -ffp-contract=off: each rounding step is the one written,
// and fused multiply-adds appear only where fma() is called.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lamq.h"

#define LAMQ_NT 256  // threads per workgroup of the row kernels (four wave64s)

#define LAMQ_LAUNCH_CHECK()                                   \
    do {                                                      \
        hipError_t e_ = hipGetLastError();                    \
        if (e_ != hipSuccess) return (int)e_;                 \
    } while (0)

static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------------------------------------
// Bitshift trellis with 2^L states and k bits per step, searched by one 256-thread workgroup.
// Thread t (t < ACT) owns the predecessor groups r in [t*G, t*G+G) and the SPT = G*2^k consecutive
// states s = r*2^k + b they feed, so the float32 state values of its states stay in registers for
// the whole search. Path costs live in LDS (two buffers of 2^L floats); back-pointers are one byte
// per active thread and step (G*k <= 8 bits: the winning h of each of its groups).
// ------------------------------------------------------------------------------------------------
template <int L, int K>
struct Vit {
    static constexpr int NS = 1 << L;
    static constexpr int R = 1 << (L - K);
    static constexpr int NB = 1 << K;
    static constexpr int ACT = R >= LAMQ_NT ? LAMQ_NT : R;
    static constexpr int G = R >= LAMQ_NT ? R / LAMQ_NT : 1;
    static constexpr int SPT = G * NB;
    static_assert(G * K <= 8, "one back-pointer byte per thread and step");
};

// LDS float index -> bank-spread index: the 16-byte chunk index (x >> 2) has its low two bits xor'ed with bits
// 4-5 of itself, a bijection within every 64 floats. Writes of consecutive threads at a stride of 16 floats then
// fall on 16 different 16-byte bank groups, and reads of consecutive 16-byte chunks stay conflict-free.
__device__ __forceinline__ int swz(int x) { return x ^ (((x >> 6) & 3) << 2); }

// N floats at logical index x (x a multiple of min(N, 4)), chunk by chunk through swz.
template <int N>
__device__ __forceinline__ void lds_load_swz(const float* __restrict__ base, int x, float (&dst)[N])
{
    if constexpr (N >= 4) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            float4 v = *reinterpret_cast<const float4*>(base + swz(x + i));
            dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
        }
    } else if constexpr (N == 2) {
        float2 v = *reinterpret_cast<const float2*>(base + swz(x));
        dst[0] = v.x; dst[1] = v.y;
    } else {
        dst[0] = base[swz(x)];
    }
}

template <int N>
__device__ __forceinline__ void lds_store_swz(float* __restrict__ base, int x, const float (&src)[N])
{
    if constexpr (N >= 4) {
#pragma unroll
        for (int i = 0; i < N; i += 4)
            *reinterpret_cast<float4*>(base + swz(x + i)) = make_float4(src[i], src[i + 1], src[i + 2], src[i + 3]);
    } else if constexpr (N == 2) {
        *reinterpret_cast<float2*>(base + swz(x)) = make_float2(src[0], src[1]);
    } else {
        base[swz(x)] = src[0];
    }
}

template <int N>
__device__ __forceinline__ void lds_load(const float* __restrict__ src, float (&dst)[N])
{
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            float4 v = *reinterpret_cast<const float4*>(src + i);
            dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
        }
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 2) {
            float2 v = *reinterpret_cast<const float2*>(src + i);
            dst[i] = v.x; dst[i + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

template <int N>
__device__ __forceinline__ void lds_store(float* __restrict__ dst, const float (&src)[N])
{
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 4) *reinterpret_cast<float4*>(dst + i) = make_float4(src[i], src[i + 1], src[i + 2], src[i + 3]);
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 2) *reinterpret_cast<float2*>(dst + i) = make_float2(src[i], src[i + 1]);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

// Search one path of TV steps. xs: TV float32 targets (any address space); Cr: this thread's state
// values; start < 0 leaves the first state free, else only states (start << K | b) & (2^L-1) may
// begin (opgraph/codes.py:164-167). cost0/cost1: 2*2^L floats of LDS, indexed through swz. back: TV*ACT bytes (LDS or
// global). path: TV ints written by thread 0. red: 8 words of LDS. Every thread of the workgroup
// must call this; it ends with a barrier after which path[] is complete.
//   forward step  (codes.py:170-172): best(r) = min_h cost[h*R + r] (lowest h on ties),
//                 cost'(r*2^K + b) = best(r) + (x_t - C)^2, rounded after the subtraction, the
//                 product and the sum, as torch's separate kernels round them
//   final state   (codes.py:173): the lowest state among the minimal costs
//   traceback     (codes.py:176-179)
template <int L, int K>
__device__ void viterbi_wg(const float* xs, int TV, const float (&Cr)[Vit<L, K>::SPT], int start, float* cost0,
                           float* cost1, uint8_t* back, int* path, float* red)
{
    using V = Vit<L, K>;
    const int tid = threadIdx.x;
    const bool act = tid < V::ACT;
    if (act) {
        const float x0 = xs[0];
        const int rs = start >= 0 ? (start & (V::R - 1)) : -1;
        float c[V::SPT];
#pragma unroll
        for (int i = 0; i < V::SPT; ++i) {
            const float d = x0 - Cr[i];
            c[i] = d * d;
            if (rs >= 0 && ((tid * V::SPT + i) >> K) != rs) c[i] = __builtin_inff();
        }
        lds_store_swz<V::SPT>(cost0, tid * V::SPT, c);
    }
    __syncthreads();
    float* cur = cost0;
    float* nxt = cost1;
    for (int t = 1; t < TV; ++t) {
        if (act) {
            const float xt = xs[t];
            float best[V::G];
            int arg[V::G];
            lds_load_swz<V::G>(cur, tid * V::G, best);
#pragma unroll
            for (int g = 0; g < V::G; ++g) arg[g] = 0;
#pragma unroll
            for (int h = 1; h < V::NB; ++h) {
                float c[V::G];
                lds_load_swz<V::G>(cur, h * V::R + tid * V::G, c);
#pragma unroll
                for (int g = 0; g < V::G; ++g)
                    if (c[g] < best[g]) { best[g] = c[g]; arg[g] = h; }
            }
            float o[V::SPT];
            unsigned bits = 0;
#pragma unroll
            for (int g = 0; g < V::G; ++g) {
                bits |= (unsigned)arg[g] << (g * K);
#pragma unroll
                for (int b = 0; b < V::NB; ++b) {
                    const float d = xt - Cr[g * V::NB + b];
                    const float dd = d * d;
                    o[g * V::NB + b] = best[g] + dd;
                }
            }
            lds_store_swz<V::SPT>(nxt, tid * V::SPT, o);
            back[t * V::ACT + tid] = (uint8_t)bits;
        }
        __syncthreads();
        float* tmp = cur;
        cur = nxt;
        nxt = tmp;
    }
    // final argmin, lowest state on ties
    float bv = __builtin_inff();
    int bi = 0x7fffffff;
    if (act) {
        float c[V::SPT];
        lds_load_swz<V::SPT>(cur, tid * V::SPT, c);
        bv = c[0];
        bi = tid * V::SPT;
#pragma unroll
        for (int i = 1; i < V::SPT; ++i)
            if (c[i] < bv) { bv = c[i]; bi = tid * V::SPT + i; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov < bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    int* redi = reinterpret_cast<int*>(red + 4);
    if ((tid & 63) == 0) { red[tid >> 6] = bv; redi[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
        float v = red[0];
        int s = redi[0];
        for (int wv = 1; wv < LAMQ_NT / 64; ++wv)
            if (red[wv] < v || (red[wv] == v && redi[wv] < s)) { v = red[wv]; s = redi[wv]; }
        path[TV - 1] = s;
        for (int t = TV - 1; t > 0; --t) {
            const int r = s >> K;
            const int owner = r / V::G;
            const int g = r - owner * V::G;
            const int h = (back[t * V::ACT + owner] >> (g * K)) & (V::NB - 1);
            s = r + h * V::R;
            path[t - 1] = s;
        }
    }
    __syncthreads();
}

// s_waitcnt vmcnt(n): at most n of this wave's vector-memory operations still outstanding
template <int N>
__device__ __forceinline__ void wait_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One direct global->LDS load (16 bytes per lane into m0 + 16 * lane). M0 is saved and restored around it.
__device__ __forceinline__ void load_lds16(const void* g, uint32_t m)
{
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep)
                 : "v"(g), "s"(m)
                 : "memory");
}

// Dispatch a functor over the (L, K) pairs the kernels are instantiated for: 2 <= L <= 12 with
// K = 1..min(4, L-1) (at L = 12 every thread then owns 16 states). Returns LAMQ_EUNSUP otherwise.
template <template <int, int> class F, typename... Args>
static int dispatch_lk(int L, int K, Args&&... args)
{
#define LAMQ_CASE(l, k) \
    if (L == l && K == k) return F<l, k>::run(args...);
    LAMQ_CASE(12, 1) LAMQ_CASE(12, 2) LAMQ_CASE(12, 3) LAMQ_CASE(12, 4)
    LAMQ_CASE(11, 1) LAMQ_CASE(11, 2) LAMQ_CASE(11, 3) LAMQ_CASE(11, 4)
    LAMQ_CASE(10, 1) LAMQ_CASE(10, 2) LAMQ_CASE(10, 3) LAMQ_CASE(10, 4)
    LAMQ_CASE(9, 1) LAMQ_CASE(9, 2) LAMQ_CASE(9, 3) LAMQ_CASE(9, 4)
    LAMQ_CASE(8, 1) LAMQ_CASE(8, 2) LAMQ_CASE(8, 3) LAMQ_CASE(8, 4)
    LAMQ_CASE(7, 1) LAMQ_CASE(7, 2) LAMQ_CASE(7, 3) LAMQ_CASE(7, 4)
    LAMQ_CASE(6, 1) LAMQ_CASE(6, 2) LAMQ_CASE(6, 3) LAMQ_CASE(6, 4)
    LAMQ_CASE(5, 1) LAMQ_CASE(5, 2) LAMQ_CASE(5, 3) LAMQ_CASE(5, 4)
    LAMQ_CASE(4, 1) LAMQ_CASE(4, 2) LAMQ_CASE(4, 3)
    LAMQ_CASE(3, 1) LAMQ_CASE(3, 2)
    LAMQ_CASE(2, 1)
#undef LAMQ_CASE
    return LAMQ_EUNSUP;
}
