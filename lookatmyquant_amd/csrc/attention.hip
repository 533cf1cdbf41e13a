// Causal grouped-query attention of the calibration forwards, fused: the score matrix never reaches memory.
//
// One workgroup per (sequence, head, block of 128 queries); its four waves take 32 queries each. The workgroup walks
// the key blocks of 64 up to its last query: each block's K and V rows (16 KB each) go straight from memory into LDS
// (global_load_lds, 16 bytes a lane, no registers), double-buffered, the next block's loads issued as soon as the
// current one is published (one barrier a block), so the four waves share one copy and no wave waits on a global
// load. Per 32-key half of a block a wave forms S^T = K Q^T (32 keys x 32 queries: the head dim, 128, as eight
// 16-deep steps of v_mfma_f32_32x32x16_bf16, float32 sums), masks it causally, updates each query's running maximum
// and sum (the online softmax: exp2 with the scale and log2(e) folded into the scores), rounds the probabilities to
// bf16 and accumulates O^T += V^T P^T (128 x 32, float32) with the earlier sums rescaled; a wave past its own last
// query skips the half (its key blocks still arrive for the others). At the end O = O^T / sum, rounded to bf16
// (nearest, ties to even).
//
// Operand layouts (32x32x16 bf16 MFMA): A[m][k] has lane l holding m = l % 32 and k = 8 (l / 32) .. + 7; B[k][n]
// has lane l holding n = l % 32 and the same k; the result has lane l holding column l % 32 and rows
// 8 (v / 4) + 4 (l / 32) + v % 4 of register v. So S^T's result is P^T's B operand as it stands, with its k order
// (keys {0-3, 8-11} in lanes 0-31 and {4-7, 12-15} in lanes 32-63 for the first 16 keys, +16 for the second): the
// V^T operand takes the same order, as two transposing LDS reads (ds_read_b64_tr_b16: a 16-lane group reads a 4 x 16
// block, lane i receiving the four rows of column i) of four consecutive keys each. Q's fragments (B of S^T: eight
// consecutive head-dim values of one query) stay in registers; K's (A of S^T: eight consecutive head-dim values of
// one key) are 16-byte LDS reads. LDS rows are 256 bytes; K's 16-byte chunks are XOR-swizzled by (row & 15), so the
// 16 keys a fragment read serves at once touch 16 different chunks (all 64 banks once); V's by 4 (row & 3), so the
// 32 lanes a transposing read serves at once touch 16 different chunks of four rows. The loads place each chunk where
// the swizzle puts it (a lane fetches the chunk that belongs in its 16-byte slot).
#include "common.h"

typedef __bf16 lamq_at_bf16x8 __attribute__((ext_vector_type(8)));
typedef float lamq_at_f32x16 __attribute__((ext_vector_type(16)));

#define AT_D 128                        // head dim
#define AT_QW 32                        // queries per wave
#define AT_KB 32                        // keys per half block (one S^T tile)
#define AT_KB2 64                       // keys per block in LDS
#define AT_QB 128                       // queries per workgroup
#define AT_OPB (AT_KB2 * AT_D * 2)      // bytes of one operand's block (16 KB)

// byte offset of 16-byte chunk `chunk` (0..15) of row `row` in a V block, and in a K block
__device__ __forceinline__ uint32_t at_sw(int row, int chunk)
{
    return (uint32_t)(row * (AT_D * 2) + ((chunk ^ (4 * (row & 3))) << 4));
}
__device__ __forceinline__ uint32_t at_ksw(int row, int chunk)
{
    return (uint32_t)(row * (AT_D * 2) + ((chunk ^ (row & 15)) << 4));
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_causal_kernel(
    const uint16_t* __restrict__ Q, int64_t sqb, int64_t sqh, int64_t sqt, const uint16_t* __restrict__ K,
    int64_t skb, int64_t skh, int64_t skt, const uint16_t* __restrict__ V, int64_t svb, int64_t svh, int64_t svt,
    uint16_t* __restrict__ O, int64_t sob, int64_t soh, int64_t sot, int rep, int T, float scale_log2)
{
    __shared__ __align__(16) uint8_t lds[2][2][AT_OPB];  // [buffer][K, V]
    const int nqb = (T + AT_QB - 1) / AT_QB;
    const int qb = nqb - 1 - (int)blockIdx.x;  // the longest query blocks first
    const int h = (int)blockIdx.y, b = (int)blockIdx.z;
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int q0 = qb * AT_QB + AT_QW * wave;
    const int li = lane & 31, hi = lane >> 5, g = lane >> 4, i16 = lane & 15;
    const uint16_t* Qp = Q + b * sqb + (int64_t)h * sqh;
    const uint16_t* Kp = K + b * skb + (int64_t)(h / rep) * skh;
    const uint16_t* Vp = V + b * svb + (int64_t)(h / rep) * svh;
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    // every wave takes part in the loads and barriers up to the workgroup's last query; a wave's own work ends at its
    // last query (none for a wave wholly past T)
    const int wg_last = (qb * AT_QB + AT_QB < T ? qb * AT_QB + AT_QB : T) - 1;
    const int nblk = wg_last / AT_KB2 + 1;
    const int my_last = q0 < T ? (q0 + AT_QW < T ? q0 + AT_QW : T) - 1 : -1;
    // block kb's rows (keys past T read row T - 1: finite values that meet zero probabilities) into buffer kb & 1:
    // instruction i (four a wave and operand) covers rows 4i .. 4i + 3, lane l row 4i + l / 16, slot l % 16
    auto load_block = [&](int kb) {
        const int k0 = kb * AT_KB2;
        const uint32_t kbuf = base + (uint32_t)((kb & 1) * 2 * AT_OPB), vbuf = kbuf + AT_OPB;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 4 * wv + q;
            const int row = 4 * i + (lane >> 4), slot = lane & 15;
            const int64_t key = k0 + row < T ? k0 + row : T - 1;
            load_lds16(Kp + key * skt + 8 * (slot ^ (row & 15)), kbuf + (uint32_t)(i * 1024));
            load_lds16(Vp + key * svt + 8 * (slot ^ (4 * (row & 3))), vbuf + (uint32_t)(i * 1024));
        }
    };
    load_block(0);
    const int myq = q0 + li;  // this lane's query (past T: computed, not stored)
    const int qrow = myq < T ? myq : T - 1;
    lamq_at_bf16x8 qf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) qf[j] = *reinterpret_cast<const lamq_at_bf16x8*>(Qp + qrow * sqt + 16 * j + 8 * hi);
    // the Q fragments as operands of an empty asm: the compiler waits for their loads here, before the loop. The
    // loop's own waits are asm, invisible to it, so without this it would wait on the Q loads inside the loop, where
    // its counts would cover the next block's loads as well and stall their prefetch
    asm volatile("" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]), "+v"(qf[4]), "+v"(qf[5]), "+v"(qf[6]),
                 "+v"(qf[7]));
    lamq_at_f32x16 o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[t][v] = 0.0f;
    float mrun = -__builtin_inff(), lrun = 0.0f;
    using v2u = uint32_t __attribute__((ext_vector_type(2)));
    for (int kb = 0; kb < nblk; ++kb) {
        wait_vm<0>();     // this wave's loads of block kb have landed
        __syncthreads();  // everyone's; the other buffer (block kb - 1) is free
        if (kb + 1 < nblk) load_block(kb + 1);
        const uint8_t* kl = lds[kb & 1][0];
        const uint32_t vbase = base + (uint32_t)(((kb & 1) * 2 + 1) * AT_OPB);
        for (int hf = 0; hf < 2; ++hf) {
            const int k0 = kb * AT_KB2 + AT_KB * hf;
            if (k0 > my_last) break;  // uniform: this wave's queries end before these keys
            // K fragments (A of S^T): key 32 hf + li of the block, head dims 16 j + 8 hi .. + 7 (chunk 2 j + hi)
            lamq_at_bf16x8 kf[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                kf[j] = *reinterpret_cast<const lamq_at_bf16x8*>(kl + at_ksw(AT_KB * hf + li, 2 * j + hi));
            lamq_at_f32x16 s;
#pragma unroll
            for (int v = 0; v < 16; ++v) s[v] = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[j], qf[j], s, 0, 0, 0);
            // causal mask, scale, the running maximum of each query (its 32 keys: 16 here, 16 in lane l ^ 32)
            float mx = -__builtin_inff();
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int key = k0 + 8 * (v >> 2) + 4 * hi + (v & 3);
                const float x = (key <= myq && key < T) ? s[v] * scale_log2 : -__builtin_inff();
                s[v] = x;
                mx = fmaxf(mx, x);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mnew = fmaxf(mrun, mx);  // finite from the first half on: key 0 is never masked
            const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);  // 0 on the first half
            float ps = 0.0f;
            lamq_at_bf16x8 pf[2];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float p = __builtin_amdgcn_exp2f(s[v] - mnew);  // masked: exp2(-inf) = 0
                ps += p;
                pf[v >> 3][v & 7] = (__bf16)p;
            }
            ps += __shfl_xor(ps, 32);
            lrun = lrun * alpha + ps;
            mrun = mnew;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[t][v] *= alpha;
            // all sixteen transposing reads first, one wait, then the eight MFMAs. Lane: head dim 32 t + li; keys
            // 16 mi + 4 hi + {0..3} and + 8 of the half (the P^T order); the group's lane i16 points at row
            // 32 hf + 16 mi + 4 hi + i16 / 4, columns 32 t + 16 (g & 1) + 4 (i16 % 4) .. + 3
            v2u lo[4][2], hi2[4][2];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int mi = 0; mi < 2; ++mi) {
                    const int row = AT_KB * hf + 16 * mi + 4 * hi + (i16 >> 2);
                    const int col = 32 * t + 16 * (g & 1) + 4 * (i16 & 3);
                    const uint32_t a0 = vbase + at_sw(row, col >> 3) + 8 * ((col >> 2) & 1);
                    const uint32_t a1 = vbase + at_sw(row + 8, col >> 3) + 8 * ((col >> 2) & 1);
                    // early-clobber outputs: the first read's destination may not share the second's address
                    // register (the first can return into it before the second read leaves the wave)
                    asm volatile("ds_read_b64_tr_b16 %0, %2\n\tds_read_b64_tr_b16 %1, %3"
                                 : "=&v"(lo[t][mi]), "=&v"(hi2[t][mi])
                                 : "v"(a0), "v"(a1)
                                 : "memory");
                }
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(lo[0][0]), "+v"(lo[0][1]), "+v"(lo[1][0]), "+v"(lo[1][1]), "+v"(lo[2][0]),
                           "+v"(lo[2][1]), "+v"(lo[3][0]), "+v"(lo[3][1]), "+v"(hi2[0][0]), "+v"(hi2[0][1]),
                           "+v"(hi2[1][0]), "+v"(hi2[1][1]), "+v"(hi2[2][0]), "+v"(hi2[2][1]), "+v"(hi2[3][0]),
                           "+v"(hi2[3][1])
                         :
                         : "memory");
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int mi = 0; mi < 2; ++mi) {
                    const uint32_t __attribute__((ext_vector_type(4))) w = {lo[t][mi][0], lo[t][mi][1], hi2[t][mi][0],
                                                                            hi2[t][mi][1]};
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(lamq_at_bf16x8, w), pf[mi], o[t], 0,
                                                                   0, 0);
                }
        }
        // the next iteration's barrier comes after every wave's reads of this buffer (their results are used above)
    }
    if (myq >= T) return;
    const float inv = 1.0f / lrun;
    uint16_t* Op = O + b * sob + (int64_t)h * soh + (int64_t)myq * sot;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            // registers 4 r .. 4 r + 3: head dims 32 t + 8 r + 4 hi + {0..3}
            uint32_t w2[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const __bf16 x0 = (__bf16)(o[t][4 * r + 2 * e] * inv), x1 = (__bf16)(o[t][4 * r + 2 * e + 1] * inv);
                w2[e] = (uint32_t)__builtin_bit_cast(uint16_t, x0) | ((uint32_t)__builtin_bit_cast(uint16_t, x1) << 16);
            }
            *reinterpret_cast<uint2*>(Op + 32 * t + 8 * r + 4 * hi) = make_uint2(w2[0], w2[1]);
        }
}

// out[b, t, h, :] = softmax(q[b, h, t, :] k[b, h / rep, :t + 1, :]^T * scale) v[b, h / rep, :t + 1, :], bf16 in and out;
// every tensor's head dim (128) contiguous, the other strides in elements.
extern "C" int lamq_attention_causal_bf16(const uint16_t* q, int64_t sqb, int64_t sqh, int64_t sqt, const uint16_t* k,
                                          int64_t skb, int64_t skh, int64_t skt, const uint16_t* v, int64_t svb,
                                          int64_t svh, int64_t svt, uint16_t* out, int64_t sob, int64_t soh,
                                          int64_t sot, int64_t B, int64_t H, int64_t Hkv, int64_t T, int64_t D,
                                          float scale, void* stream)
{
    if (!q || !k || !v || !out || B < 0 || H < 1 || Hkv < 1 || T < 0 || H % Hkv != 0) return LAMQ_EINVAL;
    if (D != AT_D) return LAMQ_EUNSUP;
    if (!(scale > 0.0f) || !(scale < 3.0e38f)) return LAMQ_EINVAL;
    const int64_t strides[12] = {sqb, sqh, sqt, skb, skh, skt, svb, svh, svt, sob, soh, sot};
    for (int64_t s : strides)
        if (s < 0 || s % 8 != 0) return LAMQ_EINVAL;  // 16-byte rows of eight bf16
    if (((uintptr_t)q % 16) || ((uintptr_t)k % 16) || ((uintptr_t)v % 16) || ((uintptr_t)out % 8)) return LAMQ_EINVAL;
    if (B == 0 || T == 0) return LAMQ_OK;
    if (B > 65535 || H > 65535 || T > 0x7fffff) return LAMQ_EUNSUP;
    const dim3 grid((unsigned)cdiv(T, AT_QB), (unsigned)H, (unsigned)B);
    hipLaunchKernelGGL(attention_causal_kernel, grid, dim3(256), 0, as_stream(stream), q, sqb, sqh, sqt, k, skb, skh, skt,
                       v, svb, svh, svt, out, sob, soh, sot, (int)(H / Hkv), (int)T, scale * 1.4426950408889634f);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
