// The causal softmax of the calibration forwards' attention, fused: bf16 scores in, bf16 probabilities out, one
// pass. Row r of the scores is query r % T of its (sequence, head); column c is kept where c <= r % T and masked to
// -inf past it. In float32, as the unfused chain computes it: s = float(score) * scale, m = the row's maximum,
// e = exp(s - m), p = e / sum(e), rounded to bf16 (nearest, ties to even). One wave per row: every lane holds T / 64
// of the row's values in registers (16-byte loads of eight consecutive scores), the maximum and the sum are wave
// reductions in a fixed order, so a row's result does not depend on anything else that runs. The row is read whole
// before it is written, so P may be S.
#include "common.h"

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;  // nearest, ties to even, for finite values of either sign
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// NC chunks of 512 columns (64 lanes x 8); T <= 512 * NC
template <int NC>
__global__ __launch_bounds__(256) void causal_softmax_bf16_kernel(const uint16_t* __restrict__ S,
                                                                  uint16_t* __restrict__ P, int64_t rows, int T,
                                                                  int64_t lds, int64_t ldp, float scale)
{
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // the whole wave
    const int lane = threadIdx.x & 63;
    const int qi = (int)(row % T);
    const uint16_t* s = S + row * lds;
    float v[NC][8];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int col0 = c * 512 + 8 * lane;
        uint4 u = make_uint4(0u, 0u, 0u, 0u);
        if (col0 < T) u = *reinterpret_cast<const uint4*>(s + col0);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int col = col0 + e;
            const float f = bf16_bits_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) * scale;
            v[c][e] = (col < T && col <= qi) ? f : -__builtin_inff();
        }
    }
    float m = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, v[c][e]);
    m = wave_max(m);  // finite: column 0 is never masked
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[c][e] = expf(v[c][e] - m);  // exp(-inf) = 0 for the masked columns
            sum += v[c][e];
        }
    sum = wave_sum(sum);
    uint16_t* p = P + row * ldp;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int col0 = c * 512 + 8 * lane;
        if (col0 >= T) continue;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = f32_to_bf16_bits(v[c][2 * e] / sum) | (f32_to_bf16_bits(v[c][2 * e + 1] / sum) << 16);
        *reinterpret_cast<uint4*>(p + col0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

extern "C" int lamq_causal_softmax_bf16(const uint16_t* S, uint16_t* P, int64_t rows, int T, int64_t lds, int64_t ldp,
                                        float scale, void* stream)
{
    if (!S || !P || rows < 0 || T < 1 || lds < T || ldp < T) return LAMQ_EINVAL;
    if (((uintptr_t)S % 16) != 0 || ((uintptr_t)P % 16) != 0 || lds % 8 != 0 || ldp % 8 != 0) return LAMQ_EINVAL;
    if (T % 8 != 0 || T > 4096) return LAMQ_EUNSUP;
    if (!(scale > 0.0f) || !(scale < 3.0e38f)) return LAMQ_EINVAL;
    if (P != S && ((P < S && P + rows * ldp > S) || (S < P && S + rows * lds > P))) return LAMQ_EINVAL;
    if (P == S && ldp != lds) return LAMQ_EINVAL;
    if (rows == 0) return LAMQ_OK;
    if (cdiv(rows, 4) > 0x7fffffff) return LAMQ_EUNSUP;
    const dim3 grid((unsigned)cdiv(rows, 4));
    hipStream_t s = as_stream(stream);
    if (T <= 512)
        hipLaunchKernelGGL(causal_softmax_bf16_kernel<1>, grid, dim3(256), 0, s, S, P, rows, T, lds, ldp, scale);
    else if (T <= 1024)
        hipLaunchKernelGGL(causal_softmax_bf16_kernel<2>, grid, dim3(256), 0, s, S, P, rows, T, lds, ldp, scale);
    else if (T <= 2048)
        hipLaunchKernelGGL(causal_softmax_bf16_kernel<4>, grid, dim3(256), 0, s, S, P, rows, T, lds, ldp, scale);
    else
        hipLaunchKernelGGL(causal_softmax_bf16_kernel<8>, grid, dim3(256), 0, s, S, P, rows, T, lds, ldp, scale);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

// RMSNorm of the forwards (Qwen3's RMSNorm as the calibration model computes it, in float32 and back):
//   y = bf16( float(bf16(x * rsqrt(mean(x^2) + eps))) * float(g) ),  x = float(X[r, :]).
// P lanes per row (P divides 64), C 16-byte chunks of eight values per lane: the row in registers, the sum of squares
// as a segmented wave reduction in a fixed order, one read and one write of the row.
template <int P, int C>
__global__ __launch_bounds__(256) void rms_norm_bf16_kernel(const uint16_t* __restrict__ X, int64_t rows, int n,
                                                            int64_t ldx, const uint16_t* __restrict__ g,
                                                            uint16_t* __restrict__ Y, int64_t ldy, float eps)
{
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t row = wave * (64 / P) + lane / P;
    const int sl = lane % P;
    const bool live = row < rows;  // lanes past the last row still take part in the reductions
    const uint16_t* x = X + (live ? row : 0) * ldx;
    float v[C][8];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int col0 = 8 * (sl + P * c);
        uint4 u = make_uint4(0u, 0u, 0u, 0u);
        if (live && col0 < n) u = *reinterpret_cast<const uint4*>(x + col0);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[c][e] = bf16_bits_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
            ss += v[c][e] * v[c][e];
        }
    }
#pragma unroll
    for (int off = P / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float r = rsqrtf(ss / (float)n + eps);
    if (!live) return;
    uint16_t* y = Y + row * ldy;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int col0 = 8 * (sl + P * c);
        if (col0 >= n) continue;
        const uint4 gu = *reinterpret_cast<const uint4*>(g + col0);
        const uint32_t gw[4] = {gu.x, gu.y, gu.z, gu.w};
        uint32_t out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t pair = 0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int k = 2 * e + h;
                const float t = bf16_bits_to_f32(f32_to_bf16_bits(v[c][k] * r));
                const float gv = bf16_bits_to_f32((gw[k >> 1] >> (16 * (k & 1))) & 0xFFFFu);
                pair |= f32_to_bf16_bits(t * gv) << (16 * h);
            }
            out[e] = pair;
        }
        *reinterpret_cast<uint4*>(y + col0) = make_uint4(out[0], out[1], out[2], out[3]);
    }
}

extern "C" int lamq_rms_norm_bf16(const uint16_t* X, int64_t rows, int64_t n, int64_t ldx, const uint16_t* g,
                                  uint16_t* Y, int64_t ldy, float eps, void* stream)
{
    if (!X || !g || !Y || rows < 0 || n < 1 || ldx < n || ldy < n || !(eps >= 0.0f)) return LAMQ_EINVAL;
    if (n % 8 || ldx % 8 || ldy % 8 || ((uintptr_t)X % 16) || ((uintptr_t)Y % 16) || ((uintptr_t)g % 16))
        return LAMQ_EINVAL;
    if (n > 8 * 64 * 20) return LAMQ_EUNSUP;
    if (rows == 0) return LAMQ_OK;
    hipStream_t s = as_stream(stream);
#define RMS_LAUNCH(P, C)                                                                                              \
    do {                                                                                                              \
        const int64_t waves = cdiv(rows, 64 / (P));                                                                   \
        if (cdiv(waves, 4) > 0x7fffffff) return LAMQ_EUNSUP;                                                          \
        hipLaunchKernelGGL((rms_norm_bf16_kernel<P, C>), dim3((unsigned)cdiv(waves, 4)), dim3(256), 0, s, X, rows,      \
                           (int)n, ldx, g, Y, ldy, eps);                                                              \
    } while (0)
    if (n <= 128) RMS_LAUNCH(16, 1);
    else if (n <= 512) RMS_LAUNCH(64, 1);
    else if (n <= 1024) RMS_LAUNCH(64, 2);
    else if (n <= 2048) RMS_LAUNCH(64, 4);
    else if (n <= 2560) RMS_LAUNCH(64, 5);
    else if (n <= 4096) RMS_LAUNCH(64, 8);
    else RMS_LAUNCH(64, 20);
#undef RMS_LAUNCH
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

// The per-head RMSNorm of q or k and the rotary embedding after it, in one pass over 128-wide rows:
//   y = bf16( float(bf16(x r)) g ),  r = rsqrt(mean(x^2) + eps)          (a row of lamq_rms_norm_bf16)
//   out[i] = bf16( float(bf16(y[i] cos[t][i])) + float(bf16(rot[i] sin[t][i])) ),
//   rot[i] = -y[i + 64] for i < 64, y[i - 64] for i >= 64,
// each product and the sum rounded to bf16 as the unfused chain (q * cos + rotate_half(q) * sin) rounds them.
// Sixteen lanes a row, eight elements a lane: the partner element i +- 64 sits in lane +- 8 of the row's sixteen,
// one exchange of the row's packed values. Rows are ordered (sequence, token, head): token t = (row / heads) % T.
__global__ __launch_bounds__(256) void rms_norm_rope_bf16_kernel(
    const uint16_t* __restrict__ X, int64_t rows, int64_t ldx, const uint16_t* __restrict__ g,
    const uint16_t* __restrict__ cosT, const uint16_t* __restrict__ sinT, int64_t ldcs, int heads, int T,
    uint16_t* __restrict__ Y, int64_t ldy, float eps)
{
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t row = wave * 4 + lane / 16;
    const int sl = lane % 16;
    const bool live = row < rows;  // lanes past the last row still take part in the reductions and the exchange
    uint4 u = make_uint4(0u, 0u, 0u, 0u);
    if (live) u = *reinterpret_cast<const uint4*>(X + row * ldx + 8 * sl);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    float v[8];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        v[e] = bf16_bits_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
        ss += v[e] * v[e];
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float r = rsqrtf(ss / 128.0f + eps);
    const uint4 gu = *reinterpret_cast<const uint4*>(g + 8 * sl);
    const uint32_t gw[4] = {gu.x, gu.y, gu.z, gu.w};
    uint32_t yb[4];  // y as packed bf16 pairs
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        uint32_t pair = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = 2 * e + h;
            const float t = bf16_bits_to_f32(f32_to_bf16_bits(v[k] * r));
            const float gv = bf16_bits_to_f32((gw[k >> 1] >> (16 * (k & 1))) & 0xFFFFu);
            pair |= f32_to_bf16_bits(t * gv) << (16 * h);
        }
        yb[e] = pair;
    }
    uint32_t pb[4];  // the partner lane's y (elements i +- 64)
#pragma unroll
    for (int e = 0; e < 4; ++e) pb[e] = (uint32_t)__shfl_xor((int)yb[e], 8);
    if (!live) return;
    const int64_t tok = (row / heads) % T;
    const uint4 cu = *reinterpret_cast<const uint4*>(cosT + tok * ldcs + 8 * sl);
    const uint4 su = *reinterpret_cast<const uint4*>(sinT + tok * ldcs + 8 * sl);
    const uint32_t cw[4] = {cu.x, cu.y, cu.z, cu.w}, sw[4] = {su.x, su.y, su.z, su.w};
    const float sgn = sl < 8 ? -1.0f : 1.0f;  // rot = -y[i + 64] in the first half, y[i - 64] in the second
    uint32_t out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        uint32_t pair = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int sh = 16 * h;
            const float y = bf16_bits_to_f32((yb[e] >> sh) & 0xFFFFu);
            const float rot = sgn * bf16_bits_to_f32((pb[e] >> sh) & 0xFFFFu);
            const float c = bf16_bits_to_f32((cw[e] >> sh) & 0xFFFFu), s = bf16_bits_to_f32((sw[e] >> sh) & 0xFFFFu);
            const float a = bf16_bits_to_f32(f32_to_bf16_bits(y * c));
            const float b = bf16_bits_to_f32(f32_to_bf16_bits(rot * s));
            pair |= f32_to_bf16_bits(a + b) << sh;
        }
        out[e] = pair;
    }
    *reinterpret_cast<uint4*>(Y + row * ldy + 8 * sl) = make_uint4(out[0], out[1], out[2], out[3]);
}

extern "C" int lamq_rms_norm_rope_bf16(const uint16_t* X, int64_t rows, int64_t n, int64_t ldx, const uint16_t* g,
                                       const uint16_t* cosT, const uint16_t* sinT, int64_t ldcs, int64_t heads,
                                       int64_t T, uint16_t* Y, int64_t ldy, float eps, void* stream)
{
    if (!X || !g || !cosT || !sinT || !Y || rows < 0 || n < 1 || heads < 1 || T < 1 || !(eps >= 0.0f))
        return LAMQ_EINVAL;
    if (n != 128) return LAMQ_EUNSUP;
    if (ldx < n || ldy < n || ldcs < n || ldx % 8 || ldy % 8 || ldcs % 8 || rows % (heads * T)) return LAMQ_EINVAL;
    if (((uintptr_t)X % 16) || ((uintptr_t)Y % 16) || ((uintptr_t)g % 16) || ((uintptr_t)cosT % 16) ||
        ((uintptr_t)sinT % 16))
        return LAMQ_EINVAL;
    if (heads > 0x7fffffff || T > 0x7fffffff) return LAMQ_EUNSUP;
    if (rows == 0) return LAMQ_OK;
    const int64_t blocks = cdiv(rows, 16);  // four waves of four rows
    if (blocks > 0x7fffffff) return LAMQ_EUNSUP;
    hipLaunchKernelGGL(rms_norm_rope_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), X, rows,
                       ldx, g, cosT, sinT, ldcs, (int)heads, (int)T, Y, ldy, eps);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

// The MLP's gate of the forwards, fused: Y = bf16( float(bf16(silu(a))) * float(b) ), silu(a) = a / (1 + exp(-a)) in
// float32, for bf16 a (the gate product) and b (the up product), eight elements a thread.
__global__ __launch_bounds__(256) void swiglu_bf16_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ Bm,
                                                          uint16_t* __restrict__ Y, int64_t n8)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const uint4 ua = reinterpret_cast<const uint4*>(A)[i], ub = reinterpret_cast<const uint4*>(Bm)[i];
    const uint32_t wa[4] = {ua.x, ua.y, ua.z, ua.w}, wb[4] = {ub.x, ub.y, ub.z, ub.w};
    uint32_t out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        uint32_t pair = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float a = bf16_bits_to_f32((wa[e] >> (16 * h)) & 0xFFFFu);
            const float b = bf16_bits_to_f32((wb[e] >> (16 * h)) & 0xFFFFu);
            const float s = bf16_bits_to_f32(f32_to_bf16_bits(a / (1.0f + expf(-a))));
            pair |= f32_to_bf16_bits(s * b) << (16 * h);
        }
        out[e] = pair;
    }
    reinterpret_cast<uint4*>(Y)[i] = make_uint4(out[0], out[1], out[2], out[3]);
}

extern "C" int lamq_swiglu_bf16(const uint16_t* a, const uint16_t* b, uint16_t* y, int64_t n, void* stream)
{
    if (!a || !b || !y || n < 0 || n % 8) return LAMQ_EINVAL;
    if (((uintptr_t)a % 16) || ((uintptr_t)b % 16) || ((uintptr_t)y % 16)) return LAMQ_EINVAL;
    if (n == 0) return LAMQ_OK;
    const int64_t n8 = n / 8;
    if (cdiv(n8, 256) > 0x7fffffff) return LAMQ_EUNSUP;
    hipLaunchKernelGGL(swiglu_bf16_kernel, dim3((unsigned)cdiv(n8, 256)), dim3(256), 0, as_stream(stream), a, b, y, n8);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
