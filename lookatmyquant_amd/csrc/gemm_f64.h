// C -= A @ op(B) on fp64 MFMA (v_mfma_f64_16x16x4f64), the update shape shared by the lazy trailing
// refit of the sweep and by the blocked factorizations.
#pragma once
#include "common.h"

typedef double lamq_d4 __attribute__((ext_vector_type(4)));

// Workgroup tile 64x64, four waves as 2x2 wave tiles of 32x32, each 2x2 MFMA tiles of 16x16.
// MFMA operand layout (16x16x4 f64): lane l holds A[l%16][l/16], B[l/16][l%16]; the result
// lane l, register v holds D[4*v + l/16][l%16]. Each output is the sum over k as a chain of
// MFMAs from zero, then subtracted from C once: C = C - sum.
// TRANSB: op(B)[k][j] = B[j*ldb + k]; otherwise B[k*ldb + j].
// LOWER: C is a square diagonal block; tiles wholly above the diagonal are skipped and only
// entries with col <= row are written.
// OVERWRITE: C = A @ op(B) instead of C -= A @ op(B). C may then alias A (a workgroup's output rows are the rows
// it reads, when N fits one tile column) or B (its output columns are the columns it reads, when M fits one tile
// row): every wave finishes its reads before any wave writes.
template <bool TRANSB, bool LOWER, bool OVERWRITE = false>
__global__ __launch_bounds__(256) void gemm_sub_f64_kernel(double* C, int64_t ldc, const double* A, int64_t lda,
                                                           const double* B, int64_t ldb, int64_t M, int64_t N,
                                                           int64_t K, const int32_t* __restrict__ info)
{
    if (info && *info != 0) return;
    const int64_t tr = (int64_t)blockIdx.y * 64, tc = (int64_t)blockIdx.x * 64;
    if (LOWER && tc > tr + 63) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t wr = tr + (wave >> 1) * 32, wc = tc + (wave & 1) * 32;
    const int li = lane & 15, lk = lane >> 4;
    lamq_d4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = lamq_d4{0.0, 0.0, 0.0, 0.0};
    const int64_t r0 = wr + li, r1 = wr + 16 + li, c0 = wc + li, c1 = wc + 16 + li;
    const bool vr0 = r0 < M, vr1 = r1 < M, vc0 = c0 < N, vc1 = c1 < N;
    // k advances in chunks of KC = 16 (four MFMA steps); the next chunk's operands are loaded into registers
    // while the current chunk's MFMAs run, so one memory latency is paid per chunk, overlapped.
    constexpr int KC = 16;
    double pa0[4], pa1[4], pb0[4], pb1[4];
    auto load = [&](int64_t kb) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int64_t kk = kb + 4 * s + lk;
            const bool vk = kk < K;
            pa0[s] = (vr0 && vk) ? A[r0 * lda + kk] : 0.0;
            pa1[s] = (vr1 && vk) ? A[r1 * lda + kk] : 0.0;
            if (TRANSB) {
                pb0[s] = (vc0 && vk) ? B[c0 * ldb + kk] : 0.0;
                pb1[s] = (vc1 && vk) ? B[c1 * ldb + kk] : 0.0;
            } else {
                pb0[s] = (vc0 && vk) ? B[kk * ldb + c0] : 0.0;
                pb1[s] = (vc1 && vk) ? B[kk * ldb + c1] : 0.0;
            }
        }
    };
    load(0);
    for (int64_t k0 = 0; k0 < K; k0 += KC) {
        double a0[4], a1[4], b0[4], b1[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            a0[s] = pa0[s];
            a1[s] = pa1[s];
            b0[s] = pb0[s];
            b1[s] = pb1[s];
        }
        if (k0 + KC < K) load(k0 + KC);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0[s], b0[s], acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0[s], b1[s], acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1[s], b0[s], acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1[s], b1[s], acc[1][1], 0, 0, 0);
        }
    }
    if (OVERWRITE) __syncthreads();
    // all reads of C before any write (see gemm128_f64_kernel)
    double cv[2][2][4];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t row = wr + ti * 16 + 4 * v + lk;
                const int64_t col = wc + tj * 16 + li;
                cv[ti][tj][v] = (!OVERWRITE && row < M && col < N && (!LOWER || col <= row)) ? C[row * ldc + col] : 0.0;
            }
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t row = wr + ti * 16 + 4 * v + lk;
                const int64_t col = wc + tj * 16 + li;
                if (row < M && col < N && (!LOWER || col <= row))
                    C[row * ldc + col] = OVERWRITE ? acc[ti][tj][v] : cv[ti][tj][v] - acc[ti][tj][v];
            }
}

// The same C -= A op(B) (no OVERWRITE) for large products: workgroup tile 128x128, four waves of 64x64 = 4x4
// MFMA tiles (64 accumulators per lane, VGPR-form). Operands go straight from memory into LDS (global_load_lds,
// 16 bytes = two doubles per lane, no registers), BK deep in k, two stage buffers: one barrier per stage
// publishes the stage and frees the other buffer for the next stage's loads, which are issued between the
// MFMAs. With BK = 16 a workgroup holds 64 KB of LDS and at most 256 VGPRs per lane, so two workgroups share a
// CU and each SIMD runs two waves that cover each other's stage barriers and epilogue (measured: 53-57 TF/s at
// K = 512 against 45-47 for BK = 32 with one workgroup per CU). LDS keeps the operands as they lie in memory, in
// 16-byte chunks XOR-swizzled so that the fragment reads (one double per lane) are bank-conflict-free:
//   [row][k] operands (A; B when TRANSB): rows of BK doubles, chunk c of row r at c ^ (r & 15) for 16 chunks a
//     row (BK = 32), c ^ ((r >> 1) & 7) for 8 (BK = 16: rows 2m and 2m + 1 sit 128 bytes apart in the banks):
//     the 16 rows of a fragment read hit 16 different 16-byte bank windows;
//   [k][col] operands (B): 1 KB rows of 128 columns, chunk c of row k at c ^ 8*(k & LAMQ_KSW_MASK): the four k-rows
//     of a fragment read sit 128 bytes apart in the banks.
// Rows past M / N and k past K load zero chunks. Needs even leading dimensions, even K (and even N for a
// [k][col] B) and 16-byte aligned operands (gemm_sub_f64 checks; other shapes take the kernel above).
#define G8_BM 128
#define G8_BK 16
#ifndef LAMQ_PANEL_MAX_TILES128
#define LAMQ_PANEL_MAX_TILES128 1024  // short products with fewer 128-tiles than this take the 64-tile panel kernel
#endif
#ifndef LAMQ_KSW_MASK
#define LAMQ_KSW_MASK 3  // [k][col] B operands: k-row k's 16-byte chunks XOR 8*(k & LAMQ_KSW_MASK)
#endif
#define LAMQ_TRI_KGE 1
#define LAMQ_TRI_KLE 2

__device__ double lamq_zero_chunk[2];

// TRI: the k-range of a tile column when op(B) is triangular, stages wholly in its zero part skipped:
// LAMQ_TRI_KGE (op(B)[k][j] = 0 for k < j, a lower op(B)): k from the tile's first column on;
// LAMQ_TRI_KLE (op(B)[k][j] = 0 for k > j, an upper op(B)): k up to the tile's last column.
template <bool TRANSB, bool LOWER, int BK, int TRI = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BK == 16 ? 2 : 1, BK == 16 ? 2 : 1))) void
gemm128_f64_kernel(double* __restrict__ C, int64_t ldc, const double* __restrict__ A, int64_t lda,
                   const double* __restrict__ B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                   const int32_t* __restrict__ info)
{
    constexpr int ASZ = G8_BM * BK * 8;  // bytes of one operand stage
    constexpr int RB = BK * 8;           // bytes of a [row][k] row
    constexpr int CPR = RB / 16;         // 16-byte chunks per [row][k] row
    constexpr int RPI = 64 / CPR;        // [row][k] rows per 1 KB load instruction
    constexpr int IPW = BK / 4;          // load instructions per wave, operand and stage
    __shared__ __align__(16) uint8_t lds[2][2][ASZ];  // [buffer][operand]
    if (info && *info != 0) return;
    int64_t tr = (int64_t)blockIdx.y * G8_BM, tc = (int64_t)blockIdx.x * G8_BM;
    if (TRI != 0) {
        // a triangular op(B) gives each tile column its own k-range: the tiles go out column by column, the longest
        // k-ranges first (workgroups start in the order of their linear index), so that the last round holds the
        // shortest tiles rather than a full-depth one that starts late
        const int64_t gx = gridDim.x, gy = gridDim.y, lin = (int64_t)blockIdx.y * gx + blockIdx.x;
        const int64_t cr = lin / gy;
        tr = (lin % gy) * G8_BM;
        tc = (TRI == LAMQ_TRI_KGE ? cr : gx - 1 - cr) * G8_BM;
    }
    if (LOWER && tc > tr + G8_BM - 1) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    const double* zc = lamq_zero_chunk;
    asm volatile("" : "+s"(zc));
    // chunk swizzle of [row][k] rows: the 16 rows of a fragment land in 16 different 16-byte windows of the 64 banks
    auto rsw = [](int r) { return CPR == 16 ? (r & 15) : ((r >> 1) & 7); };

    // loads: BK instructions of 1 KB per operand and stage, IPW per wave (instruction q of wave w is IPW*w + q)
    //   [row][k]: instruction i covers rows RPI*i .. RPI*i + RPI-1, lane l row RPI*i + l/CPR, slot l%CPR,
    //             chunk (l%CPR) ^ rsw(row)
    //   [k][col]: instruction i covers k-row i, lane l slot l, chunk l ^ 8*(i & 1)
    auto load_rowk = [&](const double* X, int64_t ldx, int64_t r0, int64_t R, int64_t k0, int i, uint32_t m) {
        const int r = RPI * i + lane / CPR;
        const int c = (lane % CPR) ^ rsw(r);
        const int64_t row = r0 + r, k = k0 + 2 * c;
        const bool ok = row < R && k < K;
        const double* g = ok ? X + row * ldx + k : zc;
        load_lds16(g, m);
    };
    auto load_kcol = [&](const double* X, int64_t ldx, int64_t c0, int64_t k0, int i, uint32_t m) {
        const int c = lane ^ (8 * (i & LAMQ_KSW_MASK));
        const int64_t k = k0 + i, col = c0 + 2 * c;
        const bool ok = k < K && col < N;
        const double* g = ok ? X + k * ldx + col : zc;
        load_lds16(g, m);
    };
    auto piece = [&](int64_t k0, int buf, int q, int op) {
        const int i = IPW * wv + q;
        const uint32_t m = lds_base + (uint32_t)((buf * 2 + op) * ASZ + i * 1024);
        if (op == 0)
            load_rowk(A, lda, tr, M, k0, i, m);
        else if (TRANSB)
            load_rowk(B, ldb, tc, N, k0, i, m);
        else
            load_kcol(B, ldb, tc, k0, i, m);
    };

    lamq_d4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = lamq_d4{0.0, 0.0, 0.0, 0.0};
    const int li = lane & 15, lk = lane >> 4;
    // fragment addresses (bytes within an operand stage) for k = k4 + lk
    auto aaddr = [&](int row, int k) -> uint32_t { return (uint32_t)(row * RB + (((k >> 1) ^ rsw(row)) << 4) + (k & 1) * 8); };
    auto baddr = [&](int col, int k) -> uint32_t {
        return TRANSB ? aaddr(col, k) : (uint32_t)(k * 1024 + (((col >> 1) ^ (8 * (k & LAMQ_KSW_MASK))) << 4) + (col & 1) * 8);
    };

    int st0 = 0, nst = (int)cdiv(K, BK);
    if (TRI == LAMQ_TRI_KGE) st0 = (int)(tc / BK);
    if (TRI == LAMQ_TRI_KLE && tc + G8_BM < K) nst = (int)cdiv(tc + G8_BM, BK);
    if (st0 >= nst) st0 = nst;  // an empty range: no loads, C - 0 written back
#pragma unroll
    for (int q = 0; q < IPW; ++q) {
        piece((int64_t)st0 * BK, st0 & 1, q, 0);
        piece((int64_t)st0 * BK, st0 & 1, q, 1);
    }
    // D layout (16x16): lane l, register v -> row 4*v + l/16, column l%16. C is read two row-groups of 16 ahead of
    // its writes: one wait counter covers loads and stores alike, so a read issued after a write would wait for it.
    auto cload = [&](int i, double(&g)[4][4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t row = tr + wr + 16 * i + 4 * v + lk;
                const int64_t col = tc + wc + 16 * j + li;
                g[j][v] = (row < M && col < N && (!LOWER || col <= row)) ? C[row * ldc + col] : 0.0;
            }
    };
    double g0[4][4], g1[4][4];
    for (int st = st0; st < nst; ++st) {
        wait_vm<0>();     // this wave's loads of stage st have landed
        __syncthreads();  // everyone's; the other buffer (stage st - 1) is free
        // the first row-group of C is read during the last stage's MFMAs
        if (st == nst - 1) cload(0, g0);
        const int buf = st & 1;
        const uint8_t* As = lds[buf][0];
        const uint8_t* Bs = lds[buf][1];
#pragma unroll
        for (int k4 = 0; k4 < BK; k4 += 4) {
            double a[4], b[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                a[t] = *reinterpret_cast<const double*>(As + aaddr(wr + 16 * t + li, k4 + lk));
                b[t] = *reinterpret_cast<const double*>(Bs + baddr(wc + 16 * t + li, k4 + lk));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
                // the next stage's 2*IPW loads, one per four MFMAs over the stage's first k-steps (after the
                // last stage they load zero chunks into the buffer no one reads: no branch in the loop)
                {
                    const int p = (k4 / 4) * 4 + i;
                    if (p < 2 * IPW) piece((int64_t)(st + 1) * BK, buf ^ 1, p >> 1, p & 1);
                }
            }
        }
    }
    if (st0 >= nst) cload(0, g0);  // no stage ran
    cload(1, g1);
    wait_vm<0>();
    auto cstore = [&](int i, const double(&g)[4][4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t row = tr + wr + 16 * i + 4 * v + lk;
                const int64_t col = tc + wc + 16 * j + li;
                if (row < M && col < N && (!LOWER || col <= row)) C[row * ldc + col] = g[j][v] - acc[i][j][v];
            }
    };
    cstore(0, g0);
    cload(2, g0);
    cstore(1, g1);
    cload(3, g1);
    cstore(2, g0);
    cstore(3, g1);
}

// Short products (K <= 128: the narrow refits of the sweep, the factor's panel products): the same C -= A op(B) (or
// C = A op(B) with OVERWRITE) on 64x64 tiles whose whole k-range stays in LDS, in up to four stages of 32: every load
// of every stage is issued at once (global_load_lds, 16 bytes a lane), and stage s is computed as soon as its own
// loads have landed, while the later stages' loads are still in flight; C is read before them. Four waves of 32x32
// (2x2 MFMA tiles). LDS layout per stage: [row][k] operands (A; B when TRANSB) 256 bytes a row, chunk c of row r at
// c ^ (r & 15) (the 16 rows of a fragment read fall in 16 different 16-byte bank windows); [k][col] B 512 bytes a
// k-row, chunk c of k-row k at c ^ 8*(k & LAMQ_KSW_MASK) (the four k-rows of a fragment read 128 bytes apart). Needs
// even K, lda, ldb (and N for a [k][col] B) and 16-byte aligned A and B, like the 128-tile kernel.
#define GP_BK 32
// NS: the most stages, K <= NS GP_BK (the whole k-range sits in LDS, 32 NS KB: two stages for the factor's depth-64
// products give two workgroups a CU, four 128 KB and one)
template <bool TRANSB, bool LOWER, bool OVERWRITE, int NS = 128 / GP_BK>
__global__ __launch_bounds__(256) void gemm64_panel_f64_kernel(double* C, int64_t ldc, const double* A, int64_t lda,
                                                               const double* B, int64_t ldb, int64_t M, int64_t N,
                                                               int64_t K, const int32_t* __restrict__ info)
{
    constexpr int SB = 64 * GP_BK * 8;  // bytes of one operand stage (A: 64 rows x 256 B; B: 32 k-rows x 512 B)
    __shared__ __align__(16) uint8_t lds[NS][2][SB];
    if (info && *info != 0) return;
    const int64_t tr = (int64_t)blockIdx.y * 64, tc = (int64_t)blockIdx.x * 64;
    if (LOWER && tc > tr + 63) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    const double* zc = lamq_zero_chunk;
    asm volatile("" : "+s"(zc));
    const int nst = (int)cdiv(K, GP_BK);
    const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
    const int li = lane & 15, lk = lane >> 4;
    // C first: its loads are the oldest, so each stage's wait below also covers them
    double cv[2][2][4];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t row = tr + wr + ti * 16 + 4 * v + lk;
                const int64_t col = tc + wc + tj * 16 + li;
                cv[ti][tj][v] = (!OVERWRITE && row < M && col < N && (!LOWER || col <= row)) ? C[row * ldc + col] : 0.0;
            }
    // stage st, operand op: 16 instructions of 1 KB, four a wave (instruction i = 4 wv + q)
    //   [row][k]: rows 4i .. 4i + 3, lane l row 4i + l/16, slot l%16 holding chunk (l%16) ^ (row & 15)
    //   [k][col]: k-rows 2i and 2i + 1, lane l k-row 2i + l/32, columns 2 (l%32), 2 (l%32) + 1
    for (int st = 0; st < nst; ++st) {
        const int64_t k0 = (int64_t)st * GP_BK;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 4 * wv + q;
            {
                const int r = 4 * i + lane / 16, c = (lane % 16) ^ (r & 15);
                const int64_t row = tr + r, k = k0 + 2 * c;
                load_lds16((row < M && k < K) ? A + row * lda + k : zc, base + (uint32_t)((st * 2 + 0) * SB + i * 1024));
            }
            if (TRANSB) {
                const int r = 4 * i + lane / 16, c = (lane % 16) ^ (r & 15);
                const int64_t col = tc + r, k = k0 + 2 * c;
                load_lds16((col < N && k < K) ? B + col * ldb + k : zc, base + (uint32_t)((st * 2 + 1) * SB + i * 1024));
            } else {
                const int kr = 2 * i + lane / 32;
                const int64_t k = k0 + kr, col = tc + 2 * ((lane % 32) ^ (8 * (kr & LAMQ_KSW_MASK)));
                load_lds16((k < K && col < N) ? B + k * ldb + col : zc, base + (uint32_t)((st * 2 + 1) * SB + i * 1024));
            }
        }
    }
    auto aaddr = [](int r, int kk) -> uint32_t { return (uint32_t)(r * 256 + (((kk >> 1) ^ (r & 15)) << 4) + (kk & 1) * 8); };
    auto kbaddr = [](int col, int kk) -> uint32_t {
        return (uint32_t)(kk * 512 + (((col >> 1) ^ (8 * (kk & LAMQ_KSW_MASK))) << 4) + (col & 1) * 8);
    };
    lamq_d4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = lamq_d4{0.0, 0.0, 0.0, 0.0};
    for (int st = 0; st < nst; ++st) {
        // this wave's loads of stages 0..st have landed when at most 8 (nst - 1 - st) of its loads are outstanding
        switch (nst - 1 - st) {
            case 0: wait_vm<0>(); break;
            case 1: wait_vm<8>(); break;
            case 2: wait_vm<16>(); break;
            default: wait_vm<24>(); break;
        }
        __syncthreads();
        const uint8_t* As = lds[st][0];
        const uint8_t* Bs = lds[st][1];
#pragma unroll
        for (int k4 = 0; k4 < GP_BK; k4 += 4) {
            const int kk = k4 + lk;
            double a[2], b[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                a[t] = *reinterpret_cast<const double*>(As + aaddr(wr + 16 * t + li, kk));
                b[t] = TRANSB ? *reinterpret_cast<const double*>(Bs + aaddr(wc + 16 * t + li, kk))
                              : *reinterpret_cast<const double*>(Bs + kbaddr(wc + 16 * t + li, kk));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
    if (OVERWRITE) __syncthreads();
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t row = tr + wr + ti * 16 + 4 * v + lk;
                const int64_t col = tc + wc + tj * 16 + li;
                if (row < M && col < N && (!LOWER || col <= row))
                    C[row * ldc + col] = OVERWRITE ? acc[ti][tj][v] : cv[ti][tj][v] - acc[ti][tj][v];
            }
}

// Short products with B as [k][col] (the sweep's narrow refits, K <= 128 by default): C -= A B on TM x TN tiles whose
// four waves split K instead of the tile. The k-range is cut into chunks of 8 and each wave takes a quarter of the
// chunks; it accumulates the whole tile over its quarter with its operands loaded straight into registers, one chunk
// ahead of its MFMAs: lane l (group g = l/16, i = l%16) loads A[row i][k0 + 2g .. k0 + 2g + 1] as one 16-byte load and
// B[k0 + 2g][col i], B[k0 + 2g + 1][col i], and the chunk is two MFMA k-steps over the k-sets {k0 + 2g} and
// {k0 + 2g + 1}. No wave waits for another until the end, where the four partial tiles meet in LDS and are summed in
// a fixed order, (w0 + w1) + (w2 + w3), and subtracted from C once. A workgroup's operands are read once, with no
// LDS staging, so a CU holds several workgroups (LDS 4 TM TN doubles each), and small tiles give a product of a few
// thousand rows enough workgroups to fill the chip, where the 64-tile kernel's one workgroup per CU (its k-range in
// LDS) left most CUs idle. Needs even K and lda and a 16-byte aligned A.
#ifndef LAMQ_SPLITK_DEPTH
#define LAMQ_SPLITK_DEPTH 2  // chunks of 8 k in flight per wave (measured: 2 beats 4 and 8)
#endif
template <int TM, int TN>
__global__ __launch_bounds__(256) void gemm_splitk_f64_kernel(double* __restrict__ C, int64_t ldc,
                                                              const double* __restrict__ A, int64_t lda,
                                                              const double* __restrict__ B, int64_t ldb, int64_t M,
                                                              int64_t N, int64_t K, const int32_t* __restrict__ info)
{
    constexpr int MT = TM / 16, NT = TN / 16;
    constexpr int PV = MT * NT * 4;  // partial values per lane
    __shared__ double part[4][PV * 64];
    if (info && *info != 0) return;
    const int64_t tr = (int64_t)blockIdx.y * TM, tc = (int64_t)blockIdx.x * TN;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int li = lane & 15, lg = lane >> 4;
    const int64_t nch = (K + 7) >> 3, per = (nch + 3) >> 2;
    const int64_t ch0 = wave * per, ch1 = ch0 + per < nch ? ch0 + per : nch;
    lamq_d4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = lamq_d4{0.0, 0.0, 0.0, 0.0};
    typedef double lamq_d2 __attribute__((ext_vector_type(2)));
    const double* arow[MT];
    bool aok[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int64_t row = tr + 16 * i + li;
        aok[i] = row < M;
        arow[i] = A + (aok[i] ? row : 0) * lda;
    }
    bool bok[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) bok[j] = tc + 16 * j + li < N;
    // one chunk's operands: a[i] = A[row][k, k + 1], b[j][e] = B[k + e][col] with k = 8 ch + 2 g (K even: k < K holds
    // for both or neither of the pair)
    auto load = [&](int64_t ch, lamq_d2 (&a)[MT], double (&b)[NT][2]) {
        const int64_t k = 8 * ch + 2 * lg;
        const bool kok = k < K;
#pragma unroll
        for (int i = 0; i < MT; ++i)
            a[i] = (aok[i] && kok) ? *reinterpret_cast<const lamq_d2*>(arow[i] + k) : lamq_d2{0.0, 0.0};
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int64_t col = tc + 16 * j + li;
            b[j][0] = (bok[j] && kok) ? B[k * ldb + col] : 0.0;
            b[j][1] = (bok[j] && kok) ? B[(k + 1) * ldb + col] : 0.0;
        }
    };
    // this thread's outputs of C, read now so that their latency overlaps the k-loop (TM TN / 256 per thread, columns
    // fastest across threads, as the epilogue writes them)
    constexpr int QO = TM * TN / 256;
    double cpre[QO];
#pragma unroll
    for (int q = 0; q < QO; ++q) {
        const int o = q * 256 + (int)threadIdx.x;
        const int64_t row = tr + o / TN, col = tc + o % TN;
        cpre[q] = (row < M && col < N) ? C[row * ldc + col] : 0.0;
    }
    // a ring of LAMQ_SPLITK_DEPTH chunks in flight: chunk c lives in slot (c - ch0) % D, reloaded with chunk c + D as
    // soon as its MFMAs are issued
    constexpr int D = LAMQ_SPLITK_DEPTH;
    lamq_d2 a[D][MT];
    double b[D][NT][2];
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (ch0 + d < ch1) load(ch0 + d, a[d], b[d]);
    for (int64_t ch = ch0; ch < ch1; ch += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (ch + d < ch1) {
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int i = 0; i < MT; ++i)
#pragma unroll
                        for (int j = 0; j < NT; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[d][i][e], b[d][j][e], acc[i][j], 0, 0, 0);
                if (ch + d + D < ch1) load(ch + d + D, a[d], b[d]);
            }
        }
    }
    // partials in LDS, value p of lane l at p * 64 + l (p = (i NT + j) 4 + v)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) part[wave][((i * NT + j) * 4 + v) * 64 + lane] = acc[i][j][v];
    __syncthreads();
    // each thread sums the four partials of TM TN / 256 outputs, columns fastest across threads; output (r, c) is
    // value ((r/16) NT + c/16) 4 + (r%16)/4 of lane 16 (r%4) + c%16 (the 16x16 MFMA result layout)
#pragma unroll
    for (int q = 0; q < QO; ++q) {
        const int o = q * 256 + (int)threadIdx.x;
        const int r = o / TN, c = o % TN;
        const int idx = (((r >> 4) * NT + (c >> 4)) * 4 + ((r & 15) >> 2)) * 64 + ((r & 3) << 4) + (c & 15);
        const double s = (part[0][idx] + part[1][idx]) + (part[2][idx] + part[3][idx]);
        const int64_t row = tr + r, col = tc + c;
        if (row < M && col < N) C[row * ldc + col] = cpre[q] - s;
    }
}

#ifndef LAMQ_SPLITK_MAXK
#define LAMQ_SPLITK_MAXK 128  // [k][col] products up to this K (not LOWER, not OVERWRITE) take the split-K kernel
#endif
// Deeper [k][col] products (K <= LAMQ_SPLITK_DEEPK) take it too where the 128-tile kernel's workgroups would fill the
// chip's 512 slots (two a CU) poorly: fewer than LAMQ_SPLITK_TILES128 tiles, or a second round holding under 64 of
// them. Measured at K = 512 (the sweep's deep products): 20-80 tiles 5.7-17 -> 19-35 TFLOP/s, 300-320 tiles 35-38 ->
// 44-46, 560 tiles 43 -> 47; at 384-480 and 608 tiles the two kernels are even or the 128-tile one is ahead.
#ifndef LAMQ_SPLITK_TILES128
#define LAMQ_SPLITK_TILES128 384
#endif
#ifndef LAMQ_SPLITK_DEEPK
#define LAMQ_SPLITK_DEEPK 1024
#endif

// TRI (LAMQ_TRI_KGE, LAMQ_TRI_KLE): op(B) is triangular and the 128-tile kernel skips the stages of its zero part (the
// other kernels read the zeros).
template <bool TRANSB, bool LOWER, bool OVERWRITE = false, int TRI = 0>
static int gemm_sub_f64(double* C, int64_t ldc, const double* A, int64_t lda, const double* B, int64_t ldb, int64_t M,
                        int64_t N, int64_t K, const int32_t* info, hipStream_t s)
{
    if (M <= 0 || N <= 0 || K <= 0) return LAMQ_OK;
    // the 128 tiles once there are enough of them to fill most of the chip, for operands it can load in 16-byte
    // chunks
    // (a [k][col] B chunk holds columns col, col + 1: N even keeps the pair inside the row)
    const bool chunks = (lda % 2) == 0 && (ldb % 2) == 0 && (K % 2) == 0 && (TRANSB || (N % 2) == 0) &&
                        ((uintptr_t)A % 16) == 0 && ((uintptr_t)B % 16) == 0;
    const int64_t tiles128 = cdiv(M, G8_BM) * cdiv(N, G8_BM);
    dim3 grid((unsigned)cdiv(N, 64), (unsigned)cdiv(M, 64));
    // the split-K kernel loads A in 16-byte pairs (even lda and K, a 16-byte aligned A) and B element by element
    const bool pairs = (lda % 2) == 0 && (K % 2) == 0 && ((uintptr_t)A % 16) == 0;
    const bool thin = tiles128 < LAMQ_SPLITK_TILES128 || (tiles128 > 512 && tiles128 < 1024 && tiles128 % 512 < 64);
    if (!TRANSB && !LOWER && !OVERWRITE && TRI == 0 && pairs && cdiv(M, 32) <= 65535 &&
        (K <= LAMQ_SPLITK_MAXK || (K <= LAMQ_SPLITK_DEEPK && thin))) {
        hipLaunchKernelGGL((gemm_splitk_f64_kernel<32, 32>), dim3((unsigned)cdiv(N, 32), (unsigned)cdiv(M, 32)), dim3(256),
                           0, s, C, ldc, A, lda, B, ldb, M, N, K, info);
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
    if (chunks && K <= 128 && (OVERWRITE || tiles128 < LAMQ_PANEL_MAX_TILES128)) {
        if (K <= 2 * GP_BK)
            hipLaunchKernelGGL((gemm64_panel_f64_kernel<TRANSB, LOWER, OVERWRITE, 2>), grid, dim3(256), 0, s, C, ldc, A,
                               lda, B, ldb, M, N, K, info);
        else
            hipLaunchKernelGGL((gemm64_panel_f64_kernel<TRANSB, LOWER, OVERWRITE>), grid, dim3(256), 0, s, C, ldc, A, lda,
                               B, ldb, M, N, K, info);
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
    if (!OVERWRITE && chunks && tiles128 >= 128) {
        dim3 grid128((unsigned)cdiv(N, G8_BM), (unsigned)cdiv(M, G8_BM));
        hipLaunchKernelGGL((gemm128_f64_kernel<TRANSB, LOWER, G8_BK, TRI>), grid128, dim3(256), 0, s, C, ldc, A, lda, B,
                           ldb, M, N, K, info);
        LAMQ_LAUNCH_CHECK();
        return LAMQ_OK;
    }
    hipLaunchKernelGGL((gemm_sub_f64_kernel<TRANSB, LOWER, OVERWRITE>), grid, dim3(256), 0, s, C, ldc, A, lda, B, ldb, M, N,
                       K, info);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
