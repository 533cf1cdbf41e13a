// Token-weighted Gram matrices on bf16 MFMA (v_mfma_f32_32x32x16_bf16) with fp32 accumulation:
//   H += scale * X^T diag(w) X   (lower triangle; quantize.py:1465, compiler.py:244, frame.py:498-505)
//   D += scale * Xr^T diag(w) Xq (all of D; quantize.py:1457)
// bf16 x bf16 products are exact in fp32. With per-token weights the weighted operand w*x (fp32) is
// split into bf16 hi + lo parts (hi = bf16(w*x), lo = bf16(w*x - hi), exact up to 2^-16 relative)
// and both are multiplied, so the products keep the precision of the reference's fp32 w*x.
#include "common.h"

typedef __bf16 lamq_bf16x8 __attribute__((ext_vector_type(8)));
typedef float lamq_f32x16 __attribute__((ext_vector_type(16)));

#define HT 128     // output tile edge (features)
#define KT 32      // tokens per LDS stage
#define KPAD 40    // LDS row stride in bf16: 80 bytes keeps the 16-byte fragment reads conflict-free

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Stage KT tokens x HT features of X (feature pairs per thread) into LDS as [feature][token].
// mode 0: plain; mode 1: hi part of w*x; mode 2: both hi and lo parts (lo into dst2).
template <int MODE>
__device__ __forceinline__ void stage_tile(const uint16_t* __restrict__ X, int64_t ldx, int64_t N, int64_t n, int64_t t0,
                                           int64_t f0, const float* __restrict__ w, uint16_t* dst, uint16_t* dst2)
{
    const int fp = threadIdx.x & 63, tg = threadIdx.x >> 6;
    const int64_t f = f0 + 2 * fp;
    uint32_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int64_t t = t0 + 8 * tg + e;
        v[e] = (t < N && f < n) ? *reinterpret_cast<const uint32_t*>(X + t * ldx + f) : 0u;
    }
    uint32_t lo[8];
    if (MODE != 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t t = t0 + 8 * tg + e;
            const float wt = t < N ? w[t] : 0.0f;
            const float p0 = bf16_to_f32(v[e] & 0xFFFFu) * wt, p1 = bf16_to_f32(v[e] >> 16) * wt;
            const uint32_t h0 = f32_to_bf16_rne(p0), h1 = f32_to_bf16_rne(p1);
            const uint32_t l0 = f32_to_bf16_rne(p0 - bf16_to_f32(h0)), l1 = f32_to_bf16_rne(p1 - bf16_to_f32(h1));
            v[e] = h0 | (h1 << 16);
            lo[e] = l0 | (l1 << 16);
        }
    }
    uint4 a, b;
    a.x = (v[0] & 0xFFFFu) | (v[1] << 16); b.x = (v[0] >> 16) | (v[1] & 0xFFFF0000u);
    a.y = (v[2] & 0xFFFFu) | (v[3] << 16); b.y = (v[2] >> 16) | (v[3] & 0xFFFF0000u);
    a.z = (v[4] & 0xFFFFu) | (v[5] << 16); b.z = (v[4] >> 16) | (v[5] & 0xFFFF0000u);
    a.w = (v[6] & 0xFFFFu) | (v[7] << 16); b.w = (v[6] >> 16) | (v[7] & 0xFFFF0000u);
    *reinterpret_cast<uint4*>(dst + (2 * fp) * KPAD + 8 * tg) = a;
    *reinterpret_cast<uint4*>(dst + (2 * fp + 1) * KPAD + 8 * tg) = b;
    if (MODE == 2) {
        a.x = (lo[0] & 0xFFFFu) | (lo[1] << 16); b.x = (lo[0] >> 16) | (lo[1] & 0xFFFF0000u);
        a.y = (lo[2] & 0xFFFFu) | (lo[3] << 16); b.y = (lo[2] >> 16) | (lo[3] & 0xFFFF0000u);
        a.z = (lo[4] & 0xFFFFu) | (lo[5] << 16); b.z = (lo[4] >> 16) | (lo[5] & 0xFFFF0000u);
        a.w = (lo[6] & 0xFFFFu) | (lo[7] << 16); b.w = (lo[6] >> 16) | (lo[7] & 0xFFFF0000u);
        *reinterpret_cast<uint4*>(dst2 + (2 * fp) * KPAD + 8 * tg) = a;
        *reinterpret_cast<uint4*>(dst2 + (2 * fp + 1) * KPAD + 8 * tg) = b;
    }
}

// One workgroup: one 128x128 output tile (features I x features J) over the tokens [kb, ke).
// SYM: the tile list is the lower triangle (I >= J) and A, B read the same X.
// WEIGHTED: the B operand is w*x split into hi and lo.
// out: H itself (partial == 0: H += scale*acc) or a partial slab (partial == 1: slab = acc).
template <bool SYM, bool WEIGHTED>
__global__ __launch_bounds__(256) void gram_kernel(const uint16_t* __restrict__ Xa, const uint16_t* __restrict__ Xb,
                                                   int64_t N, int64_t n, int64_t ldx, const float* __restrict__ w,
                                                   float scale, float* __restrict__ out, int64_t ldo, int64_t slab,
                                                   int partial, int64_t tokens_per_split)
{
    __shared__ __align__(16) uint16_t As[HT * KPAD];
    __shared__ __align__(16) uint16_t Bs[HT * KPAD];
    __shared__ __align__(16) uint16_t Ls[WEIGHTED ? HT * KPAD : 8];
    int64_t I, J;
    if (SYM) {
        const int64_t tt = blockIdx.x;
        int64_t i = (int64_t)((sqrt(8.0 * (double)tt + 1.0) - 1.0) / 2.0);
        while ((i + 1) * (i + 2) / 2 <= tt) ++i;
        while (i * (i + 1) / 2 > tt) --i;
        I = i;
        J = tt - i * (i + 1) / 2;
    } else {
        const int64_t nt = cdiv(n, HT);
        I = blockIdx.x / nt;
        J = blockIdx.x - I * nt;
    }
    const int64_t split = blockIdx.y;
    const int64_t kb = split * tokens_per_split;
    const int64_t ke = kb + tokens_per_split < N ? kb + tokens_per_split : N;
    const int64_t fi = I * HT, fj = J * HT;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wi = wave >> 1, wj = wave & 1;
    lamq_f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    for (int64_t t0 = kb; t0 < ke; t0 += KT) {
        stage_tile<0>(Xa, ldx, ke, n, t0, fi, nullptr, As, nullptr);
        if (WEIGHTED)
            stage_tile<2>(Xb, ldx, ke, n, t0, fj, w, Bs, Ls);
        else
            stage_tile<0>(Xb, ldx, ke, n, t0, fj, nullptr, Bs, nullptr);
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < KT; ks += 16) {
            const int kofs = ks + 8 * (lane >> 5);
            lamq_bf16x8 af[2], bf[2], lf[2];
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
                af[ti] = *reinterpret_cast<const lamq_bf16x8*>(As + (wi * 64 + ti * 32 + (lane & 31)) * KPAD + kofs);
#pragma unroll
            for (int tj = 0; tj < 2; ++tj) {
                bf[tj] = *reinterpret_cast<const lamq_bf16x8*>(Bs + (wj * 64 + tj * 32 + (lane & 31)) * KPAD + kofs);
                if (WEIGHTED)
                    lf[tj] = *reinterpret_cast<const lamq_bf16x8*>(Ls + (wj * 64 + tj * 32 + (lane & 31)) * KPAD + kofs);
            }
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                for (int tj = 0; tj < 2; ++tj) {
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ti], bf[tj], acc[ti][tj], 0, 0, 0);
                    if (WEIGHTED)
                        acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ti], lf[tj], acc[ti][tj], 0, 0, 0);
                }
        }
        __syncthreads();
    }
    // result layout (32x32): lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, column l%32
    float* o = out + (partial ? split * slab : 0);
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t i = fi + wi * 64 + ti * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const int64_t j = fj + wj * 64 + tj * 32 + (lane & 31);
                if (i < n && j < n && (!SYM || j <= i)) {
                    float* p = o + i * ldo + j;
                    if (partial)
                        *p = acc[ti][tj][v];
                    else
                        *p = *p + scale * acc[ti][tj][v];
                }
            }
}

// out[i][j] += scale * sum_s slab_s[i][j], s ascending (lower triangle when SYM).
__global__ void gram_reduce_kernel(const float* __restrict__ parts, int64_t splits, int64_t slab, int64_t n,
                                   float scale, float* __restrict__ out, int64_t ldo, int sym)
{
    const int64_t i = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6);
    const int64_t j = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
    if (i >= n || j >= n || (sym && j > i)) return;
    float s = 0.0f;
    for (int64_t k = 0; k < splits; ++k) s += parts[k * slab + i * n + j];
    float* p = out + i * ldo + j;
    *p = *p + scale * s;
}

static int64_t gram_splits(int64_t N, int64_t n, bool sym)
{
    const int64_t nt = cdiv(n, HT);
    const int64_t tiles = sym ? nt * (nt + 1) / 2 : nt * nt;
    int64_t s = cdiv(1024, tiles);
    const int64_t maxs = N / 1024 > 1 ? N / 1024 : 1;
    if (s > maxs) s = maxs;
    if (s < 1) s = 1;
    return s;
}

extern "C" size_t lamq_gram_workspace_size(int64_t N, int64_t n, int sym)
{
    if (N < 1 || n < 1) return 0;
    const int64_t s = gram_splits(N, n, sym != 0);
    return s > 1 ? (size_t)s * (size_t)n * (size_t)n * sizeof(float) : 0;
}

static int gram_launch(const uint16_t* Xa, const uint16_t* Xb, int64_t N, int64_t n, int64_t ldx, const float* w,
                       float scale, float* out, int64_t ldo, bool sym, void* ws, size_t ws_bytes, hipStream_t s)
{
    const int64_t nt = cdiv(n, HT);
    const int64_t tiles = sym ? nt * (nt + 1) / 2 : nt * nt;
    const int64_t splits = gram_splits(N, n, sym);
    const int64_t per = cdiv(cdiv(N, splits), KT) * KT;
    const int64_t nsplit = cdiv(N, per);
    const bool partial = nsplit > 1;
    const int64_t slab = n * n;
    if (partial && (!ws || ws_bytes < (size_t)nsplit * (size_t)slab * sizeof(float))) return LAMQ_EINVAL;
    float* dst = partial ? reinterpret_cast<float*>(ws) : out;
    const int64_t ldd = partial ? n : ldo;
    dim3 grid((unsigned)tiles, (unsigned)nsplit);
#define GRAM_LAUNCH(S, W) \
    hipLaunchKernelGGL((gram_kernel<S, W>), grid, dim3(256), 0, s, Xa, Xb, N, n, ldx, w, scale, dst, ldd, slab, partial ? 1 : 0, per)
    if (sym) {
        if (w) GRAM_LAUNCH(true, true); else GRAM_LAUNCH(true, false);
    } else {
        if (w) GRAM_LAUNCH(false, true); else GRAM_LAUNCH(false, false);
    }
#undef GRAM_LAUNCH
    LAMQ_LAUNCH_CHECK();
    if (partial) {
        hipLaunchKernelGGL(gram_reduce_kernel, dim3((unsigned)cdiv(n, 64), (unsigned)cdiv(n, 4)), dim3(256), 0, s, dst,
                           nsplit, slab, n, scale, out, ldo, sym ? 1 : 0);
        LAMQ_LAUNCH_CHECK();
    }
    return LAMQ_OK;
}

static bool gram_args_ok(const uint16_t* X, int64_t N, int64_t n, int64_t ldx)
{
    return X && N >= 0 && n >= 2 && ldx >= n && (n % 2) == 0 && (ldx % 2) == 0 && ((uintptr_t)X % 4) == 0;
}

extern "C" int lamq_hessian_accum(const uint16_t* X, int64_t N, int64_t n, int64_t ldx, const float* w, float scale,
                                  float* H, int64_t ldH, void* workspace, size_t workspace_bytes, void* stream)
{
    if (!gram_args_ok(X, N, n, ldx) || !H || ldH < n) return LAMQ_EINVAL;
    if (N == 0) return LAMQ_OK;
    return gram_launch(X, X, N, n, ldx, w, scale, H, ldH, true, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int lamq_cross_gram(const uint16_t* Xr, const uint16_t* Xq, int64_t N, int64_t n, int64_t ldx, const float* w,
                               float scale, float* D, int64_t ldD, void* workspace, size_t workspace_bytes, void* stream)
{
    if (!gram_args_ok(Xr, N, n, ldx) || !gram_args_ok(Xq, N, n, ldx) || !D || ldD < n) return LAMQ_EINVAL;
    if (N == 0) return LAMQ_OK;
    return gram_launch(Xr, Xq, N, n, ldx, w, scale, D, ldD, false, workspace, workspace_bytes, as_stream(stream));
}

// H32 (lower triangle accumulated) -> symmetric H32 / n_tok, and optionally its float64 copy
// (quantize.py:1470: (H / n_tok).cpu().double()).
__global__ void hessian_finalize_kernel(float* __restrict__ H, int64_t n, int64_t ldH, float ntok,
                                        double* __restrict__ H64, int64_t ldH64)
{
    const int64_t i = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6);
    const int64_t j = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
    if (i >= n || j >= n || j > i) return;
    const float v = H[i * ldH + j] / ntok;
    H[i * ldH + j] = v;
    if (j != i) H[j * ldH + i] = v;
    if (H64) {
        H64[i * ldH64 + j] = (double)v;
        H64[j * ldH64 + i] = (double)v;
    }
}

extern "C" int lamq_hessian_finalize(float* H, int64_t n, int64_t ldH, float ntok, double* H64, int64_t ldH64,
                                     void* stream)
{
    if (!H || n < 1 || ldH < n || !(ntok > 0.0f) || (H64 && ldH64 < n)) return LAMQ_EINVAL;
    hipLaunchKernelGGL(hessian_finalize_kernel, dim3((unsigned)cdiv(n, 64), (unsigned)cdiv(n, 4)), dim3(256), 0,
                       as_stream(stream), H, n, ldH, ntok, H64, ldH64);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
