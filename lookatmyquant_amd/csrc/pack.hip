// Row-trellis states -> opgraph-packed-1 code words (compiler_artifact.py:225-240, 261-284).
// The symbol of column c is state & (2^k - 1); each row is padded forward with zero symbols to a
// multiple of 32 (npad), reversed, and packed 32 symbols per group: reversed symbol i of group g
// (the forward column npad-1-32g-i) occupies bits [i*k, i*k+k) of the group's k little-endian
// 32-bit words.
#include "common.h"

__global__ __launch_bounds__(256) void pack_trellis_kernel(const int32_t* __restrict__ states, int64_t m, int64_t n,
                                                           int64_t lds, int k, int L, uint32_t* __restrict__ codes,
                                                           int64_t ldc, int32_t* __restrict__ bad)
{
    const int64_t groups = (n + 31) / 32;
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= m * groups) return;
    const int64_t row = id / groups, g = id - row * groups;
    const int64_t npad = groups * 32;
    const int32_t* s = states + row * lds;
    const uint32_t kmask = (1u << k) - 1u, lmask = (1u << L) - 1u, rmask = (1u << (L - k)) - 1u;
    uint64_t lo = 0, hi = 0;  // up to 128 bits: 32 symbols of at most 4 bits
    int ok = 1;
    for (int i = 0; i < 32; ++i) {
        const int64_t c = npad - 1 - 32 * g - i;
        uint32_t sym = 0;
        if (c < n) {
            const int32_t st = s[c];
            ok &= (st >= 0 && (uint32_t)st <= lmask) ? 1 : 0;
            if (c == 0)
                ok &= ((uint32_t)st >> k) == 0u ? 1 : 0;
            else
                ok &= (((uint32_t)st >> k) == ((uint32_t)s[c - 1] & rmask)) ? 1 : 0;
            sym = (uint32_t)st & kmask;
        }
        const int bit = i * k;
        if (bit < 64) {
            lo |= (uint64_t)sym << bit;
            if (bit + k > 64) hi |= (uint64_t)sym >> (64 - bit);
        } else {
            hi |= (uint64_t)sym << (bit - 64);
        }
    }
    uint32_t* out = codes + row * ldc + g * k;
    for (int wd = 0; wd < k; ++wd) out[wd] = wd < 2 ? (uint32_t)(lo >> (32 * wd)) : (uint32_t)(hi >> (32 * (wd - 2)));
    if (!ok) atomicOr(bad, 1);
}

extern "C" int lamq_pack_trellis(const int32_t* states, int64_t m, int64_t n, int64_t lds, int k, int L, uint32_t* codes,
                                 int64_t ldc, int32_t* bad, void* stream)
{
    if (!states || !codes || !bad || m < 0 || n < 1 || lds < n || k < 1 || k > 4 || L <= k || L > 16) return LAMQ_EINVAL;
    if (ldc < (n + 31) / 32 * k) return LAMQ_EINVAL;
    if (m == 0) return LAMQ_OK;
    const int64_t total = m * ((n + 31) / 32);
    hipLaunchKernelGGL(pack_trellis_kernel, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, as_stream(stream), states, m, n,
                       lds, k, L, codes, ldc, bad);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

extern "C" int lamq_abi_version(void) { return 100; }
