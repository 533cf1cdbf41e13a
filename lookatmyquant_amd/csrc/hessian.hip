// Token-weighted Gram matrices on bf16 MFMA (v_mfma_f32_32x32x16_bf16) with fp32 accumulation:
//   H += scale * X^T diag(w) X   (lower triangle; quantize.py:1465, compiler.py:244, frame.py:498-505)
//   D += scale * Xr^T diag(w) Xq (all of D; quantize.py:1457)
// bf16 x bf16 products are exact in fp32. With per-token weights the weighted operand w*x (fp32) is
// split into bf16 hi + lo parts (hi = bf16(w*x), lo = bf16(w*x - hi), exact up to 2^-16 relative)
// and both are multiplied, so the products keep the precision of the reference's fp32 w*x.
#include "common.h"
#include <type_traits>

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

// ------------------------------------------------------------------------------------------------
// The unweighted Gram on 256x256 output tiles (the weighted case reaches it class by class: a weight
// shared by a set of tokens scales that set's product, see lamq_hessian_accum_rows).
//
// One workgroup of four waves per tile (features I x features J); wave (wi, wj) owns the 128x128
// quarter of 4x4 MFMA tiles of 32x32 (v_mfma_f32_32x32x16_bf16), its 256 accumulators in AGPRs.
// Tokens advance in stages of GK = 32 through GNS LDS stage buffers filled by direct global->LDS loads
// (global_load_lds_dwordx4, 16 bytes per lane, no registers): GNS - 1 stages are in flight while one is
// consumed, and one barrier per stage both publishes the landed stage and frees the buffer of the
// previous one. The loads of the next stage are issued between the MFMAs, one per four. The LDS keeps
// the activations as they lie in memory, [token][feature] with 512-byte rows (256 features) whose
// 16-byte chunks are XOR-swizzled by 4 * (token & 3); the MFMA fragments (8 consecutive tokens of one
// feature per lane) come from two ds_read_b64_tr_b16 each: within a 16-lane group, lane s points at
// token k0 + s/4, features m0 + 4*(s%4), and lane i receives tokens k0..k0+3 of feature m0 + i. The LDS
// serves 32 lanes (two groups: 4 tokens x 2 feature pairs) at once, and the swizzle puts their eight
// 32-byte pieces in eight different bank windows. Tokens past the range and features past n load a zero
// row (a stale token in LDS would reach every output).
// ------------------------------------------------------------------------------------------------
#define GT 256
#define GK 32
#define GNS 5                      // LDS stages (5 x 32 KB: all of a CU's LDS)
#define GSTAGE (2 * GK * GT * 2)   // bytes per stage: operands A and B, GK rows of 512 bytes each

typedef short lamq_i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) lamq_i16x4 lamq_lds_i16x4;

__device__ uint4 lamq_zero_row[GT / 8];  // 512 zero bytes: the source of masked loads

__device__ __forceinline__ uint32_t gsw(int token, int chunk)
{
    return (uint32_t)(token * (GT * 2) + ((chunk ^ (4 * (token & 3))) << 4));
}

// Tile order: logical tiles run through panels of GP tile columns, row by row, so the workgroups resident
// at one time work on a compact block of tiles and share feature blocks of the activations. Logical
// workgroup b (xcd_remap of the grid index: the 32 workgroups one XCD holds at a time are neighbours) takes
// split b / tiles, tile b % tiles.
#define GP 8
__device__ __forceinline__ void gram_tile(int64_t t, int64_t nt, bool sym, int64_t& I, int64_t& J)
{
    for (int64_t c0 = 0; c0 < nt; c0 += GP) {
        const int64_t c1 = c0 + GP < nt ? c0 + GP : nt;
        const int64_t r0 = sym ? c0 : 0;
        int64_t count;
        if (sym) {
            const int64_t tri = c1 - c0;  // rows c0 .. c1-1 hold 1 .. tri tiles, the rows below tri each
            count = tri * (tri + 1) / 2 + (nt - c1) * tri;
        } else {
            count = nt * (c1 - c0);
        }
        if (t >= count) {
            t -= count;
            continue;
        }
        for (int64_t r = r0; r < nt; ++r) {
            const int64_t w = sym ? ((r < c1 ? r : c1 - 1) - c0 + 1) : (c1 - c0);
            if (t < w) {
                I = r;
                J = c0 + t;
                return;
            }
            t -= w;
        }
    }
    I = J = 0;  // not reached for t < the tile count
}

// ROWS: the tokens are rows tok[kb..ke) of X (else rows kb..ke).
template <bool SYM, bool ROWS>
__global__ __launch_bounds__(256) void gram256_kernel(const uint16_t* __restrict__ Xa, const uint16_t* __restrict__ Xb,
                                                      int64_t N, int64_t n, int64_t ldx, const int32_t* __restrict__ tok,
                                                      float scale, float* __restrict__ out, int64_t ldo, int64_t slab,
                                                      int partial, int64_t tokens_per_split, int64_t tiles)
{
    __shared__ __align__(16) uint8_t lds[GNS * GSTAGE];
    const int64_t b = xcd_remap(blockIdx.x, gridDim.x);
    const int64_t split = b / tiles;
    int64_t I, J;
    gram_tile(b - split * tiles, cdiv(n, GT), SYM, I, J);
    const int64_t kb = split * tokens_per_split;
    const int64_t ke = kb + tokens_per_split < N ? kb + tokens_per_split : N;
    const int64_t span = ke - kb;
    const int nst = (int)cdiv(span, GK);
    const bool diag = SYM && I == J;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wi = wave >> 1, wj = wave & 1;
    const int wv = __builtin_amdgcn_readfirstlane(wave);

    // Loads. Wave w, instruction q (0..3) covers rows 2*(4w + q) and +1 of a stage, for operand A and for
    // operand B (a diagonal tile loads A twice: 8 loads per wave and stage keep the vmcnt bookkeeping fixed);
    // lane l fills slot l%32 of row 2*(4w + q) + l/32 with the chunk slot ^ 4*(row & 3), and row & 3 =
    // 2*(q & 1) + l/32. The loads are issued from asm, so the compiler's wait insertion leaves them to the
    // explicit vmcnt waits and the barrier.
    const int lrow = lane >> 5, slot = lane & 31;
    const int64_t fA = I * GT, fB = diag ? I * GT : J * GT;
    const uint16_t* XB = diag ? Xa : Xb;
    const uint16_t* zrow = reinterpret_cast<const uint16_t*>(lamq_zero_row);
    asm volatile("" : "+s"(zrow));  // computed once, not rebuilt at every load
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    int64_t loff[2];  // element offset of this lane's chunk from the pair's first row (contiguous tokens)
    int coff[2];      // element offset of this lane's chunk within its row
    bool fok[2][2];   // [operand][q parity]: the chunk lies within n
#pragma unroll
    for (int par = 0; par < 2; ++par) {
        const int c = slot ^ (4 * (2 * par + lrow));
        coff[par] = 8 * c;
        loff[par] = lrow * ldx + 8 * c;
        fok[0][par] = fA + 8 * c < n;
        fok[1][par] = fB + 8 * c < n;
    }
    // with a row list, the wave's 8 rows of a stage (tokens kb + st*GK + 8w + k) are read one stage early and
    // turned into element offsets row * ldx (uniform: scalar arithmetic)
    auto load_idx = [&](int st, int64_t (&ix)[8]) {
        if (!ROWS) return;
        const int64_t tb = kb + (int64_t)st * GK + 8 * wv;
        int32_t r[8];
        if (tb + 8 <= ke) {
#pragma unroll
            for (int k = 0; k < 8; ++k) r[k] = tok[tb + k];
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) r[k] = tb + k < ke ? tok[tb + k] : 0;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) ix[k] = (int64_t)__builtin_amdgcn_readfirstlane(r[k]) * ldx;
    };
    auto piece = [&](int st, int q, int op, const int64_t (&ix)[8]) {
        const int rp = 2 * (4 * wv + q);  // first row of the pair (uniform)
        const bool ok = ((int64_t)st * GK + rp + lrow < span) && fok[op][q & 1];
        const uint16_t* X = op ? XB : Xa;
        const int64_t f0 = op ? fB : fA;
        const uint16_t* src;
        if (ROWS) {
            // both offsets as scalars first: selecting between two array elements by lane would become an
            // indexed (scratch) access
            const int64_t oa = ix[2 * q], ob = ix[2 * q + 1];
            src = X + (lrow ? ob : oa) + f0 + coff[q & 1];
        } else {
            src = X + (kb + (int64_t)st * GK + rp) * ldx + f0 + loff[q & 1];
        }
        const uint32_t m = lds_base + (uint32_t)((st % GNS) * GSTAGE + op * GK * 512 + rp * 512);
        load_lds16(ok ? (const void*)src : (const void*)zrow, m);
    };

    // fragment read offsets within a stage: group g = lane/16, i = lane%16; token 8*(g/2) + i/4 (+4 for the
    // second read, +16 per k-step), feature 16*(g%2) + 4*(i%4) + 32*t within the wave's 128 features
    const int g = lane >> 4, li = lane & 15;
    const int tk = 8 * (g >> 1) + (li >> 2);
    uint32_t offA[4], offB[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int fa = wi * 128 + 32 * t + 16 * (g & 1) + 4 * (li & 3);
        const int fb = wj * 128 + 32 * t + 16 * (g & 1) + 4 * (li & 3);
        offA[t] = gsw(tk, fa >> 3) + ((fa >> 2) & 1) * 8;
        offB[t] = GK * 512 + gsw(tk, fb >> 3) + ((fb >> 2) & 1) * 8;
    }
    // The fragment reads are issued from asm with immediate offsets (+2048 for the second read of a fragment,
    // +8192 per k-step) off one address per fragment and stage; asm reads are invisible to the compiler's wait
    // insertion, so frag_wait takes the fragments as operands: nothing that uses them can move above it. The outputs
    // are early-clobber: the second read takes its address after the first has been issued, and a first read whose
    // destination shared the address register could return into it before the second read leaves the wave.
    using v2u = uint32_t __attribute__((ext_vector_type(2)));
    auto tr_read = [&](uint32_t addr, v2u& lo, v2u& hi, auto ks_tag) {
        constexpr int ks = decltype(ks_tag)::value;
        asm volatile("ds_read_b64_tr_b16 %0, %2 offset:%3\n\tds_read_b64_tr_b16 %1, %2 offset:%4"
                     : "=&v"(lo), "=&v"(hi)
                     : "v"(addr), "n"(ks * 16 * 512), "n"(ks * 16 * 512 + 4 * 512)
                     : "memory");
    };
    auto as_frag = [](v2u lo, v2u hi) {
        const uint32_t __attribute__((ext_vector_type(4))) v = {lo[0], lo[1], hi[0], hi[1]};
        return __builtin_bit_cast(lamq_bf16x8, v);
    };
    auto frags = [&](uint32_t S, auto ks_tag, lamq_bf16x8 (&af)[4], lamq_bf16x8 (&bf)[4]) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            v2u a0, a1, b0, b1;
            tr_read(S + offA[t], a0, a1, ks_tag);
            tr_read(S + offB[t], b0, b1, ks_tag);
            af[t] = as_frag(a0, a1);
            bf[t] = as_frag(b0, b1);
        }
    };
    // s_waitcnt lgkmcnt(N) tied to the fragments it guards
    auto frag_wait = [](auto n_tag, lamq_bf16x8 (&af)[4], lamq_bf16x8 (&bf)[4]) {
        constexpr int N = decltype(n_tag)::value;
        asm volatile("s_waitcnt lgkmcnt(%8)"
                     : "+v"(af[0]), "+v"(af[1]), "+v"(af[2]), "+v"(af[3]), "+v"(bf[0]), "+v"(bf[1]), "+v"(bf[2]), "+v"(bf[3])
                     : "n"(N)
                     : "memory");
    };

    lamq_f32x16 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    int64_t ix[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int st = 0; st < GNS - 1; ++st) {
        load_idx(st, ix);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            piece(st, q, 0, ix);
            piece(st, q, 1, ix);
        }
    }
    load_idx(GNS - 1, ix);
    for (int st = 0; st < nst; ++st) {
        wait_vm<8 * (GNS - 2)>();  // stage st has landed (this wave's part)
        __syncthreads();           // every wave's part; the buffer of stage st - 1 is free
        const uint32_t S = lds_base + (uint32_t)((st % GNS) * GSTAGE);
        const int sn = st + GNS - 1;  // the stage loaded during this one, into the freed buffer
        lamq_bf16x8 af[2][4], bf[2][4];
        frags(S, std::integral_constant<int, 0>{}, af[0], bf[0]);
        frags(S, std::integral_constant<int, 1>{}, af[1], bf[1]);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int ti = 0; ti < 4; ++ti) {
                if (ti == 0) {  // 16 reads per k-step, issued in order: the first k-step's are done at 15 outstanding
                    if (ks == 0)  // (the counter field holds at most 15)
                        frag_wait(std::integral_constant<int, 15>{}, af[0], bf[0]);
                    else
                        frag_wait(std::integral_constant<int, 0>{}, af[1], bf[1]);
                }
#pragma unroll
                for (int tj = 0; tj < 4; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][ti], bf[ks][tj], acc[ti][tj], 0, 0, 0);
                const int p = ks * 4 + ti;  // one load of the next stage in the shadow of every four MFMAs
                piece(sn, p >> 1, p & 1, ix);
            }
        load_idx(sn + 1, ix);
    }
    wait_vm<0>();  // no load may still be writing this workgroup's LDS when it ends
    // result layout (32x32): lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, column l%32. Per row of MFMA
    // tiles, the 64 outputs of this lane are read before any is written (interleaved, every read would wait for
    // the write before it).
    float* o = out + (partial ? split * slab : 0);
    const int64_t fi = I * GT, fj = J * GT;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
        float hv[4][16];
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t i = fi + wi * 128 + ti * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const int64_t j = fj + wj * 128 + tj * 32 + (lane & 31);
                hv[tj][v] = (!partial && i < n && j < n && (!SYM || j <= i)) ? o[i * ldo + j] : 0.0f;
            }
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t i = fi + wi * 128 + ti * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const int64_t j = fj + wj * 128 + tj * 32 + (lane & 31);
                if (i < n && j < n && (!SYM || j <= i))
                    o[i * ldo + j] = partial ? acc[ti][tj][v] : hv[tj][v] + scale * acc[ti][tj][v];
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

// The 256-tile kernel needs 16-byte rows: n and the row stride multiples of 8 bf16, a 16-byte aligned base.
static bool gram256_ok(const uint16_t* X, int64_t n, int64_t ldx)
{
    return (n % 8) == 0 && (ldx % 8) == 0 && ((uintptr_t)X % 16) == 0;
}

// Token splits: enough workgroups to fill the chip, at least 1024 tokens per split. The 128 tiles aim at about
// four workgroups per CU; the 256 tiles (one workgroup per CU) at one round of at most 256 workgroups, since a
// short second round would cost as much as the first.
// Token splits of a Gram launch. The 128-tile kernel: enough splits for about 1024 workgroups. The 256-tile kernel
// (one workgroup per CU): 256 / tiles splits (one round) when those fill at least 85% of the CUs; otherwise the split
// count whose workgroups fill the 256 CUs' rounds best (tiles * s / (rounds * 256)), the smallest such count when
// several come within 2%, with at most max(8, 512 / tiles) splits and 512 MB of partial slabs (more splits cost a
// larger reduction and more pipeline fills). Always at least 1024 tokens per split. At n = 4,096 (136
// lower-triangle tiles) one split would leave 47% of the chip idle; seven fill 93% of four rounds.
static int64_t gram_splits(int64_t N, int64_t n, bool sym, int64_t edge)
{
    const int64_t nt = cdiv(n, edge);
    const int64_t tiles = sym ? nt * (nt + 1) / 2 : nt * nt;
    const int64_t maxs = N / 1024 > 1 ? N / 1024 : 1;
    if (edge != GT) {
        int64_t s = cdiv(1024, tiles);
        if (s > maxs) s = maxs;
        return s < 1 ? 1 : s;
    }
    int64_t s0 = 256 / tiles;
    if (s0 > maxs) s0 = maxs;
    if (s0 < 1) s0 = 1;
    if ((double)(tiles * s0) / (double)(cdiv(tiles * s0, 256) * 256) >= 0.85) return s0;
    int64_t smax = cdiv(512, tiles) > 8 ? cdiv(512, tiles) : 8;
    const int64_t slab_cap = ((int64_t)512 << 20) / (n * n * (int64_t)sizeof(float));
    if (smax > maxs) smax = maxs;
    if (smax > slab_cap) smax = slab_cap;
    int64_t best = 1;
    double best_eff = 0.0;
    for (int64_t s = 1; s <= smax; ++s) {
        const int64_t wg = tiles * s, rounds = cdiv(wg, 256);
        const double eff = (double)wg / (double)(rounds * 256);
        if (eff > best_eff + 0.02) {
            best = s;
            best_eff = eff;
        }
    }
    return best;
}

extern "C" size_t lamq_gram_workspace_size(int64_t N, int64_t n, int sym)
{
    if (N < 1 || n < 1) return 0;
    int64_t s = gram_splits(N, n, sym != 0, HT);
    const int64_t s2 = gram_splits(N, n, sym != 0, GT);
    if (s2 > s) s = s2;
    return s > 1 ? (size_t)s * (size_t)n * (size_t)n * sizeof(float) : 0;
}

static int gram_reduce(float* parts, int64_t nsplit, int64_t n, float scale, float* out, int64_t ldo, bool sym,
                       hipStream_t s)
{
    hipLaunchKernelGGL(gram_reduce_kernel, dim3((unsigned)cdiv(n, 64), (unsigned)cdiv(n, 4)), dim3(256), 0, s, parts,
                       nsplit, n * n, n, scale, out, ldo, sym ? 1 : 0);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}

// The unweighted Gram of the tokens tok[0..N) (or 0..N) on the 256-tile kernel.
static int gram256_launch(const uint16_t* Xa, const uint16_t* Xb, int64_t N, int64_t n, int64_t ldx, const int32_t* tok,
                          float scale, float* out, int64_t ldo, bool sym, void* ws, size_t ws_bytes, hipStream_t s)
{
    const int64_t nt = cdiv(n, GT);
    const int64_t tiles = sym ? nt * (nt + 1) / 2 : nt * nt;
    const int64_t splits = gram_splits(N, n, sym, GT);
    const int64_t per = cdiv(cdiv(N, splits), GK) * GK;
    const int64_t nsplit = cdiv(N, per);
    const bool partial = nsplit > 1;
    const int64_t slab = n * n;
    if (partial && (!ws || ws_bytes < (size_t)nsplit * (size_t)slab * sizeof(float))) return LAMQ_EINVAL;
    float* dst = partial ? reinterpret_cast<float*>(ws) : out;
    const int64_t ldd = partial ? n : ldo;
    dim3 grid((unsigned)(tiles * nsplit));
#define GRAM256(S, R)                                                                                               \
    hipLaunchKernelGGL((gram256_kernel<S, R>), grid, dim3(256), 0, s, Xa, Xb, N, n, ldx, tok, scale, dst, ldd, slab, \
                       partial ? 1 : 0, per, tiles)
    if (sym) {
        if (tok) GRAM256(true, true); else GRAM256(true, false);
    } else {
        if (tok) GRAM256(false, true); else GRAM256(false, false);
    }
#undef GRAM256
    LAMQ_LAUNCH_CHECK();
    return partial ? gram_reduce(dst, nsplit, n, scale, out, ldo, sym, s) : LAMQ_OK;
}

static int gram_launch(const uint16_t* Xa, const uint16_t* Xb, int64_t N, int64_t n, int64_t ldx, const float* w,
                       float scale, float* out, int64_t ldo, bool sym, void* ws, size_t ws_bytes, hipStream_t s)
{
    if (!w && gram256_ok(Xa, n, ldx) && gram256_ok(Xb, n, ldx))
        return gram256_launch(Xa, Xb, N, n, ldx, nullptr, scale, out, ldo, sym, ws, ws_bytes, s);
    const int64_t nt = cdiv(n, HT);
    const int64_t tiles = sym ? nt * (nt + 1) / 2 : nt * nt;
    const int64_t splits = gram_splits(N, n, sym, HT);
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
    return partial ? gram_reduce(dst, nsplit, n, scale, out, ldo, sym, s) : LAMQ_OK;
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

extern "C" int lamq_hessian_accum_rows(const uint16_t* X, const int32_t* rows, int64_t nrows, int64_t n, int64_t ldx,
                                       float scale, float* H, int64_t ldH, void* workspace, size_t workspace_bytes,
                                       void* stream)
{
    if (!gram_args_ok(X, nrows, n, ldx) || !rows || !H || ldH < n) return LAMQ_EINVAL;
    if (!gram256_ok(X, n, ldx)) return LAMQ_EUNSUP;
    if (nrows == 0) return LAMQ_OK;
    return gram256_launch(X, X, nrows, n, ldx, rows, scale, H, ldH, true, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int lamq_cross_gram_rows(const uint16_t* Xr, const uint16_t* Xq, const int32_t* rows, int64_t nrows, int64_t n,
                                    int64_t ldx, float scale, float* D, int64_t ldD, void* workspace, size_t workspace_bytes,
                                    void* stream)
{
    if (!gram_args_ok(Xr, nrows, n, ldx) || !gram_args_ok(Xq, nrows, n, ldx) || !rows || !D || ldD < n) return LAMQ_EINVAL;
    if (!gram256_ok(Xr, n, ldx) || !gram256_ok(Xq, n, ldx)) return LAMQ_EUNSUP;
    if (nrows == 0) return LAMQ_OK;
    return gram256_launch(Xr, Xq, nrows, n, ldx, rows, scale, D, ldD, false, workspace, workspace_bytes, as_stream(stream));
}
