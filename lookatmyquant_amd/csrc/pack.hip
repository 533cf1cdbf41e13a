// Code arrays -> opgraph-packed-1 code words (compiler_artifact.py:225-240, 261-284, 346-353).
// A row of n symbols is padded with zero symbols to a multiple of 32 and packed 32 symbols per group: symbol i of a
// group occupies bits [i*k, i*k+k) of the group's k little-endian 32-bit words. Scalar codes are packed in column
// order. Row-trellis codes use the symbol state & (2^k - 1) of each state, and the padded row is reversed before
// packing: output group g holds forward group G-1-g, its symbol i being the forward column 32(G-1-g) + 31 - i.
//
// One thread per (row, output group): it reads its forward group's 32 entries (eight 16-byte loads when the group
// is whole and the rows are 16-byte aligned), validates them, and writes k words. Each row is read once from HBM
// and each code word written once; the kernel is HBM-bound at 4 bytes read and k/8 bytes written per symbol.
#include "common.h"

// item id = (row r of the group, output group g) of one group's m * ceil(n / 32) items
template <int K, bool TRELLIS, bool VEC>
__device__ __forceinline__ void pack_item(const int32_t* __restrict__ src, int64_t ld, int64_t src_rows,
                                          const int64_t* __restrict__ rows, int64_t n, int32_t base, int L,
                                          uint32_t* __restrict__ codes, int64_t ldc, int32_t* __restrict__ bad,
                                          int64_t id)
{
    const int64_t G = (n + 31) / 32;
    const int64_t r = id / G, g = id - r * G;
    const int64_t fg = TRELLIS ? G - 1 - g : g;  // the forward group this output group holds
    const int64_t c0 = fg * 32;
    uint32_t* out = codes + r * ldc + g * K;
    const int64_t sr = rows ? rows[r] : r;
    if (sr < 0 || sr >= src_rows) {  // a row index outside the source: flagged, its words zero, nothing read
#pragma unroll
        for (int j = 0; j < K; ++j) out[j] = 0u;
        atomicOr(bad, 2);
        return;
    }
    const int32_t* s = src + sr * ld;
    const int nv = (int)(n - c0 < 32 ? n - c0 : 32);  // valid entries of the group
    int32_t v[32];
    if (VEC && nv == 32) {
        const int4* p = reinterpret_cast<const int4*>(s + c0);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int4 q = p[j];
            v[4 * j] = q.x; v[4 * j + 1] = q.y; v[4 * j + 2] = q.z; v[4 * j + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = j < nv ? s[c0 + j] : base;
    }
    const uint32_t kmask = (1u << K) - 1u;
    bool ok = true;
    if constexpr (TRELLIS) {
        // every state lies in [0, 2^L), the first column's state is a symbol shifted in from state 0, and each later
        // state's high L-k bits are its predecessor's low L-k bits
        const uint32_t lmask = (1u << L) - 1u, rmask = (1u << (L - K)) - 1u;
        uint32_t prev = c0 > 0 ? (uint32_t)s[c0 - 1] - (uint32_t)base : 0u;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            if (j < nv) {
                const uint32_t st = ((uint32_t)v[j] - (uint32_t)base);
                ok = ok && st <= lmask && (st >> K) == (prev & rmask);
                prev = st;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) ok = ok && ((uint32_t)v[j] - (uint32_t)base) <= kmask;
    }
    uint32_t w[K];
#pragma unroll
    for (int j = 0; j < K; ++j) w[j] = 0u;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int j = TRELLIS ? 31 - i : i;  // the entry that output symbol i takes
        const uint32_t sym = j < nv ? (((uint32_t)v[j] - (uint32_t)base) & kmask) : 0u;
        const int bit = i * K, wd = bit >> 5, sh = bit & 31;
        w[wd] |= sym << sh;
        if (sh + K > 32) w[wd + 1] |= sym >> (32 - sh);
    }
#pragma unroll
    for (int j = 0; j < K; ++j) out[j] = w[j];
    if (!ok) atomicOr(bad, 1);
}

template <int K, bool TRELLIS, bool VEC>
__global__ __launch_bounds__(256) void pack_codes_kernel(const int32_t* __restrict__ src, int64_t ld,
                                                         int64_t src_rows, const int64_t* __restrict__ rows, int64_t m,
                                                         int64_t n, int32_t base, int L, uint32_t* __restrict__ codes,
                                                         int64_t ldc, int32_t* __restrict__ bad)
{
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= m * ((n + 31) / 32)) return;
    pack_item<K, TRELLIS, VEC>(src, ld, src_rows, rows, n, base, L, codes, ldc, bad, id);
}

template <int K>
static int launch_pack(const int32_t* src, int64_t ld, int64_t src_rows, const int64_t* rows, int64_t m, int64_t n,
                       int32_t base, int L, int trellis, uint32_t* codes, int64_t ldc, int32_t* bad, hipStream_t st)
{
    const int64_t total = m * ((n + 31) / 32);
    const dim3 grid((unsigned)cdiv(total, 256)), block(256);
    const bool vec = (ld % 4) == 0 && ((uintptr_t)src & 15) == 0;
    if (trellis) {
        if (vec)
            hipLaunchKernelGGL((pack_codes_kernel<K, true, true>), grid, block, 0, st, src, ld, src_rows, rows, m, n, base, L, codes, ldc, bad);
        else
            hipLaunchKernelGGL((pack_codes_kernel<K, true, false>), grid, block, 0, st, src, ld, src_rows, rows, m, n, base, L, codes, ldc, bad);
    } else {
        if (vec)
            hipLaunchKernelGGL((pack_codes_kernel<K, false, true>), grid, block, 0, st, src, ld, src_rows, rows, m, n, base, L, codes, ldc, bad);
        else
            hipLaunchKernelGGL((pack_codes_kernel<K, false, false>), grid, block, 0, st, src, ld, src_rows, rows, m, n, base, L, codes, ldc, bad);
    }
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

extern "C" int lamq_pack_codes(const int32_t* src, int64_t ld, int64_t src_rows, const int64_t* rows, int64_t m, int64_t n,
                               int32_t base, int k, int L, int trellis, uint32_t* codes, int64_t ldc, int32_t* bad,
                               void* stream)
{
    if (!src || !codes || !bad || m < 0 || n < 1 || ld < n || src_rows < 0 || k < 1 || k > 8) return LAMQ_EINVAL;
    if (!rows && m > src_rows) return LAMQ_EINVAL;
    if (trellis && (L <= k || L > 16)) return LAMQ_EINVAL;
    if (ldc < (n + 31) / 32 * k) return LAMQ_EINVAL;
    if (m == 0) return LAMQ_OK;
    if (m * ((n + 31) / 32) > (int64_t)256 * 0x7fffffff) return LAMQ_EUNSUP;
    hipStream_t st = as_stream(stream);
    switch (k) {
        case 1: return launch_pack<1>(src, ld, src_rows, rows, m, n, base, L, trellis, codes, ldc, bad, st);
        case 2: return launch_pack<2>(src, ld, src_rows, rows, m, n, base, L, trellis, codes, ldc, bad, st);
        case 3: return launch_pack<3>(src, ld, src_rows, rows, m, n, base, L, trellis, codes, ldc, bad, st);
        case 4: return launch_pack<4>(src, ld, src_rows, rows, m, n, base, L, trellis, codes, ldc, bad, st);
        case 5: return launch_pack<5>(src, ld, src_rows, rows, m, n, base, L, trellis, codes, ldc, bad, st);
        case 6: return launch_pack<6>(src, ld, src_rows, rows, m, n, base, L, trellis, codes, ldc, bad, st);
        case 7: return launch_pack<7>(src, ld, src_rows, rows, m, n, base, L, trellis, codes, ldc, bad, st);
        default: return launch_pack<8>(src, ld, src_rows, rows, m, n, base, L, trellis, codes, ldc, bad, st);
    }
}

// ------------------------------------------------------------------------------------------------ many groups at once
// Workgroup b takes 256 consecutive items of one group: the groups' workgroup ranges are laid end to end, and a
// uniform scan over at most PACK_GROUPS_PER_LAUNCH entries finds b's group. The arithmetic is pack_item's, so every
// group's words and flags are those of lamq_pack_codes on that group alone.
#define PACK_GROUPS_PER_LAUNCH 32
struct PackGroupArg {
    const int32_t* src;
    const int64_t* rows;
    uint32_t* codes;
    int64_t ld, src_rows, m, ldc;
    int32_t base;
    int k, vec;
};
struct PackGroupArgs {
    PackGroupArg g[PACK_GROUPS_PER_LAUNCH];
    int64_t first[PACK_GROUPS_PER_LAUNCH + 1];  // first workgroup of each group; first[count] is the grid
    int count;
};

template <bool TRELLIS, bool VEC>
__device__ __forceinline__ void pack_item_k(const PackGroupArg& a, int64_t n, int L, int32_t* bad, int64_t id)
{
    switch (a.k) {
    case 1: pack_item<1, TRELLIS, VEC>(a.src, a.ld, a.src_rows, a.rows, n, a.base, L, a.codes, a.ldc, bad, id); break;
    case 2: pack_item<2, TRELLIS, VEC>(a.src, a.ld, a.src_rows, a.rows, n, a.base, L, a.codes, a.ldc, bad, id); break;
    case 3: pack_item<3, TRELLIS, VEC>(a.src, a.ld, a.src_rows, a.rows, n, a.base, L, a.codes, a.ldc, bad, id); break;
    case 4: pack_item<4, TRELLIS, VEC>(a.src, a.ld, a.src_rows, a.rows, n, a.base, L, a.codes, a.ldc, bad, id); break;
    case 5: pack_item<5, TRELLIS, VEC>(a.src, a.ld, a.src_rows, a.rows, n, a.base, L, a.codes, a.ldc, bad, id); break;
    case 6: pack_item<6, TRELLIS, VEC>(a.src, a.ld, a.src_rows, a.rows, n, a.base, L, a.codes, a.ldc, bad, id); break;
    case 7: pack_item<7, TRELLIS, VEC>(a.src, a.ld, a.src_rows, a.rows, n, a.base, L, a.codes, a.ldc, bad, id); break;
    default: pack_item<8, TRELLIS, VEC>(a.src, a.ld, a.src_rows, a.rows, n, a.base, L, a.codes, a.ldc, bad, id); break;
    }
}

template <bool TRELLIS>
__global__ __launch_bounds__(256) void pack_codes_groups_kernel(PackGroupArgs args, int64_t n, int L,
                                                                int32_t* __restrict__ bad)
{
    const int64_t b = blockIdx.x;
    int i = 0;
    while (i + 1 < args.count && b >= args.first[i + 1]) ++i;
    const PackGroupArg& a = args.g[i];
    const int64_t id = (b - args.first[i]) * 256 + threadIdx.x;
    if (id >= a.m * ((n + 31) / 32)) return;
    if (a.vec)
        pack_item_k<TRELLIS, true>(a, n, L, bad, id);
    else
        pack_item_k<TRELLIS, false>(a, n, L, bad, id);
}

extern "C" int lamq_pack_codes_groups(const lamq_pack_group* groups, int ngroups, int64_t n, int L, int trellis,
                                      int32_t* bad, void* stream)
{
    if ((!groups && ngroups > 0) || ngroups < 0 || n < 1 || !bad) return LAMQ_EINVAL;
    const int64_t G = (n + 31) / 32;
    for (int i = 0; i < ngroups; ++i) {  // every group checked before anything is launched
        const lamq_pack_group& g = groups[i];
        if (!g.src || !g.codes || g.m < 0 || g.ld < n || g.src_rows < 0 || g.k < 1 || g.k > 8) return LAMQ_EINVAL;
        if (!g.rows && g.m > g.src_rows) return LAMQ_EINVAL;
        if (trellis && (L <= g.k || L > 16)) return LAMQ_EINVAL;
        if (g.ldc < G * g.k) return LAMQ_EINVAL;
        if (g.m * G > (int64_t)256 * 0x7fffffff) return LAMQ_EUNSUP;
    }
    hipStream_t st = as_stream(stream);
    for (int i0 = 0; i0 < ngroups;) {
        PackGroupArgs args{};
        int64_t blocks = 0;
        int c = 0;
        for (; i0 < ngroups && c < PACK_GROUPS_PER_LAUNCH; ++i0) {
            const lamq_pack_group& g = groups[i0];
            const int64_t nb = cdiv(g.m * G, 256);
            if (nb == 0) continue;
            if (blocks + nb > 0x7fffffff) break;  // the next launch takes it
            args.g[c] = PackGroupArg{g.src, g.rows, g.codes, g.ld, g.src_rows, g.m, g.ldc, g.base, g.k,
                                     (g.ld % 4) == 0 && ((uintptr_t)g.src & 15) == 0 ? 1 : 0};
            args.first[c] = blocks;
            blocks += nb;
            ++c;
        }
        if (c == 0) continue;
        args.first[c] = blocks;
        args.count = c;
        if (trellis)
            hipLaunchKernelGGL((pack_codes_groups_kernel<true>), dim3((unsigned)blocks), dim3(256), 0, st, args, n, L, bad);
        else
            hipLaunchKernelGGL((pack_codes_groups_kernel<false>), dim3((unsigned)blocks), dim3(256), 0, st, args, n, L, bad);
        LAMQ_LAUNCH_CHECK();
    }
    return LAMQ_OK;
}

extern "C" int lamq_pack_trellis(const int32_t* states, int64_t m, int64_t n, int64_t lds, int k, int L, uint32_t* codes,
                                 int64_t ldc, int32_t* bad, void* stream)
{
    return lamq_pack_codes(states, lds, m, nullptr, m, n, 0, k, L, 1, codes, ldc, bad, stream);
}

extern "C" int lamq_abi_version(void) { return 101; }
