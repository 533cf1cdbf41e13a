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

// a HIP runtime call's error, returned as the entry point's status
#define LAMQ_HIP_CHECK(call)                                  \
    do {                                                      \
        hipError_t e_ = (call);                               \
        if (e_ != hipSuccess) return (int)e_;                 \
    } while (0)

static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// MI355X dispatches the workgroups of a grid to its 8 XCDs round-robin (workgroup b to XCD b % 8), and each XCD
// has its own L2. xcd_remap(b, G) renumbers the grid so that XCD x runs one contiguous range of logical
// workgroups, in order: workgroups resident on one XCD at one time are neighbours in the logical order and
// share the data they read through that XCD's L2. A bijection on [0, G): XCD x receives G / 8 workgroups, one
// more for the first G % 8 XCDs.
// v of lane `lane` (a wave-uniform index) in every lane
__device__ __forceinline__ double readlane_f64(double v, int lane)
{
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

#define LAMQ_XCDS 8
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t G)
{
    const int64_t x = b % LAMQ_XCDS, r = b / LAMQ_XCDS;
    const int64_t q = G / LAMQ_XCDS, extra = G % LAMQ_XCDS;
    return x < extra ? x * (q + 1) + r : extra * (q + 1) + (x - extra) * q + r;
}

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

// s_waitcnt vmcnt(n): at most n of this wave's vector-memory operations still outstanding
template <int N>
__device__ __forceinline__ void wait_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One direct global->LDS load (16 bytes per lane into m0 + 16 * lane). M0 is saved and restored around it. A load
// to LDS that reads M0 needs one wait state after a scalar write of M0 (the compiler inserts it for its own code, not
// inside inline asm): the s_nop 0. Without it the load can take the previous M0 and land in the wrong LDS rows.
__device__ __forceinline__ void load_lds16(const void* g, uint32_t m)
{
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep)
                 : "v"(g), "s"(m)
                 : "memory");
}

// One direct global->LDS load of 4 bytes per lane (into m0 + 4 * lane), with the same wait state after the M0 write.
__device__ __forceinline__ void load_lds4(const void* g, uint32_t m)
{
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep)
                 : "v"(g), "s"(m)
                 : "memory");
}

// LDS byte address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
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
