// Bitshift-trellis search (opgraph/codes.py:151-181) shared by the standalone kernels and the fused
// block-LDLQ kernels, and the in-block refit of the fused kernels (opgraph/syntax.py:109-121).
//
// Layout. The 2^L states fall into R = 2^(L-K) groups of NB = 2^K: group r collects the states h*R + r
// (h < NB), which are the possible predecessors of the states r*NB + b. One step of the reference
// (codes.py:170-172) is best(r) = min_h cost(h*R + r) with the lowest h on ties, then
// cost'(r*NB + b) = best(r) + (x_t - C[r*NB + b])^2. Thread t of NT owns the G groups r = G*t + g and keeps
// the values of their NB*G member states h*R + G*t + g in registers. Between steps only the group minima
// B (R floats) travel through LDS: member h*R + r has the path cost B((h*R + r) >> K) + (x - C)^2, which
// its group's owner forms itself with the reference's three rounded operations (difference, square, sum),
// hence the same float32 value. Per step a thread reads the B entries of its members, forms the NB costs
// of each of its groups, keeps the minimum and its h (strict comparison in increasing h: the lowest h wins
// a tie, as torch's min does) and writes its G new minima: R floats written and R read per step, a
// quarter of the full cost vector.
#pragma once
#include "common.h"

#define LAMQ_WMAX 16      // widest block the fused kernels settle at once
#ifndef LAMQ_RAMP_LOG_STATES
#define LAMQ_RAMP_LOG_STATES 13  // L > 12: the ramp of a fixed start ends at the last position reaching <= 2^this states
#endif
#define LAMQ_PRE_MAX 1024  // most earlier columns of a run whose updates a block takes itself (pre)

template <int L, int K, int NT>
struct VX {
    static constexpr int NS = 1 << L;
    static constexpr int R = 1 << (L - K);
    static constexpr int NB = 1 << K;
    static constexpr int ACT = R >= NT ? NT : R;   // threads that own groups
    static constexpr int G = R >= NT ? R / NT : 1;  // groups per thread
    static constexpr int SPT = G * NB;              // member states per thread
    // G >= NB: the B entries of a thread's members are NB runs of M consecutive entries, run h starting at
    // h*(R >> K) + M*t. G < NB: one entry per h, (h*R + G*t) >> K, shared by NB/G neighbouring threads.
    static constexpr bool RUN = G >= NB;
    static constexpr int M = RUN ? G / NB : 1;
};

// s_waitcnt lgkmcnt(0) + s_barrier: orders this workgroup's LDS traffic without waiting for its
// outstanding global loads (prefetches stay in flight across the search's barriers).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float h2f_lo(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(u & 0xFFFFu)); }
__device__ __forceinline__ float h2f_hi(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(u >> 16)); }

// x - C as fma(C, -1, x) with C read in place from its fp16 half of a register (v_fma_mix_f32): one rounding of
// the exact difference, the value of the float32 subtraction x - float(C). Written as asm because the compiler
// turns fma(c, -1, x) back into a conversion and a subtraction.
__device__ __forceinline__ float xmc_lo(float x, uint32_t c)
{
    float d;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(c), "v"(x));
    return d;
}
__device__ __forceinline__ float xmc_hi(float x, uint32_t c)
{
    float d;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(c), "v"(x));
    return d;
}

// 2 v + (this lane's bit of mask): one v_addc_co_u32 with the mask as its carry-in
__device__ __forceinline__ uint32_t shift_in(uint32_t v, uint64_t mask)
{
    uint32_t r;
    uint64_t carry;
    asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(r), "=s"(carry) : "v"(v), "s"(mask));
    return r;
}

// The member state values of thread t: member i = h*G + g is state h*R + G*t + g.
template <class V>
struct TabF32 {
    float v[V::SPT];
    __device__ __forceinline__ void load(const float* __restrict__ C, int t)
    {
        src = C;
#pragma unroll
        for (int h = 0; h < V::NB; ++h)
#pragma unroll
            for (int g = 0; g < V::G; ++g) v[h * V::G + g] = C[h * V::R + V::G * t + g];
    }
    const float* src;  // the whole table (the ramp of a fixed start reads other threads' states there)
    __device__ __forceinline__ void hold() {}
    __device__ __forceinline__ float dsq(float x, int i) const
    {
        const float d = x - v[i];
        return d * d;
    }
    // (x - C[s])^2 of state s, and of the states s, s + 1 (s even), read from memory
    __device__ __forceinline__ float dsq_at(float x, uint32_t s) const
    {
        const float d = x - src[s];
        return d * d;
    }
    __device__ __forceinline__ void dsq_at2(float x, uint32_t s, float& q0, float& q1) const
    {
        const float2 c = *reinterpret_cast<const float2*>(src + s);
        const float d0 = x - c.x, d1 = x - c.y;
        q0 = d0 * d0;
        q1 = d1 * d1;
    }
};

// fp16 values packed two per register (tables whose values fp16 holds exactly).
template <class V>
struct TabF16 {
    static_assert(V::G % 2 == 0, "members in pairs");
    uint32_t v[V::SPT / 2];
    const uint16_t* src;  // the whole table (the ramp of a fixed start reads other threads' states there)
    __device__ __forceinline__ void load(const uint16_t* __restrict__ C16, int t)
    {
        src = C16;
#pragma unroll
        for (int h = 0; h < V::NB; ++h)
#pragma unroll
            for (int g = 0; g < V::G; g += 2)
                v[(h * V::G + g) / 2] = *reinterpret_cast<const uint32_t*>(C16 + h * V::R + V::G * t + g);
    }
    // keeps the compiler from unpacking the table out of the step loop (twice the registers)
    __device__ __forceinline__ void hold()
    {
#pragma unroll
        for (int i = 0; i < V::SPT / 2; ++i) asm volatile("" : "+v"(v[i]));
    }
    __device__ __forceinline__ float dsq(float x, int i) const
    {
        const float d = (i & 1) ? xmc_hi(x, v[i >> 1]) : xmc_lo(x, v[i >> 1]);
        return d * d;
    }
    __device__ __forceinline__ float dsq_at(float x, uint32_t s) const
    {
        const float d = xmc_lo(x, (uint32_t)src[s]);
        return d * d;
    }
    __device__ __forceinline__ void dsq_at2(float x, uint32_t s, float& q0, float& q1) const
    {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(src + s);
        const float d0 = xmc_lo(x, w), d1 = xmc_hi(x, w);
        q0 = d0 * d0;
        q1 = d1 * d1;
    }
};

// f(IntC<v>{}) for the uniform v in [I, N): a chain of scalar branches, so that f indexes registers statically
template <int I>
struct IntC {
    static constexpr int value = I;
};
template <int I, int N, class F>
__device__ __forceinline__ void uniform_switch(int v, F& f)
{
    if constexpr (I < N) {
        if (v == I)
            f(IntC<I>{});
        else
            uniform_switch<I + 1, N>(v, f);
    }
}

// f(IntC<I>{}), f(IntC<I + 1>{}), ..., f(IntC<N - 1>{})
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F& f)
{
    if constexpr (I < N) {
        f(IntC<I>{});
        static_for<I + 1, N>(f);
    }
}

// Search one path of TV steps; path[0..TV) is complete when this returns (it ends with a barrier).
//   xs: TV float32 targets (LDS or global). start < 0 leaves the first state free, else only the states
//   (start << K | b) & (2^L - 1) may begin (codes.py:164-167). buf: DBL ? 2R : R floats of LDS (with one
//   buffer each step takes a second barrier, between the reads of the old minima and the writes of the new).
//   back: (TV-1) * ACT entries (LDS or global), entry t*ACT + owner holding the winning h of each of the
//   owner's groups for the step that produced B_{t+1}. red: 2*(NT/64) words of LDS.
//   Final state: the lowest among the minimal costs (codes.py:173); traceback codes.py:176-179.
struct NoHook {
    __device__ __forceinline__ void operator()() const {}
};

// hook() runs once the forward pass is done (the caller's chance to issue loads that the final argmin and the
// traceback then cover). BACK_GLOBAL: back-pointers in global memory, published to the tracing thread by a full
// barrier (otherwise only LDS is ordered, and the caller's outstanding loads stay in flight).
// lexicographic (v, i) minimum of the wave through DPP moves (no LDS): quad swaps, half-row and row mirrors, then the
// row broadcasts; lane 63 ends up with the minimum of all 64 lanes.
template <int CTRL, int ROWS>
__device__ __forceinline__ void argmin_dpp(float& v, int& i)
{
    const float ov = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS, 0xF, false));
    const int oi = __builtin_amdgcn_update_dpp(i, i, CTRL, ROWS, 0xF, false);
    if (ov < v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__device__ __forceinline__ void wave_argmin(float& v, int& i)
{
    argmin_dpp<0xB1, 0xF>(v, i);   // quad_perm [1,0,3,2]
    argmin_dpp<0x4E, 0xF>(v, i);   // quad_perm [2,3,0,1]
    argmin_dpp<0x141, 0xF>(v, i);  // row_half_mirror
    argmin_dpp<0x140, 0xF>(v, i);  // row_mirror
    argmin_dpp<0x142, 0xA>(v, i);  // row_bcast15 into rows 1 and 3
    argmin_dpp<0x143, 0xC>(v, i);  // row_bcast31 into rows 2 and 3
}

// the minimum of the wave (float or int) by the same DPP moves; lane 63 ends up with it
template <int CTRL, int ROWS>
__device__ __forceinline__ float fmin_dpp(float v)
{
    return fminf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS, 0xF, false)));
}
__device__ __forceinline__ float wave_min(float v)
{
    v = fmin_dpp<0xB1, 0xF>(v);
    v = fmin_dpp<0x4E, 0xF>(v);
    v = fmin_dpp<0x141, 0xF>(v);
    v = fmin_dpp<0x140, 0xF>(v);
    v = fmin_dpp<0x142, 0xA>(v);
    return fmin_dpp<0x143, 0xC>(v);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ int imin_dpp(int v)
{
    return min(v, __builtin_amdgcn_update_dpp(v, v, CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ int wave_imin(int v)
{
    v = imin_dpp<0xB1, 0xF>(v);
    v = imin_dpp<0x4E, 0xF>(v);
    v = imin_dpp<0x141, 0xF>(v);
    v = imin_dpp<0x140, 0xF>(v);
    v = imin_dpp<0x142, 0xA>(v);
    return imin_dpp<0x143, 0xC>(v);
}

// Search one path of TV steps. With PATHREG (TV <= 64) the path comes back in a register of wave 0, lane c holding
// path[c] (the return value), and is also stored to path[0..TV) (LDS or global); otherwise lane 0 of wave 0 stores
// path[] as the traceback goes and the return value is 0. Ends with a barrier after which path[] is complete.
//   xs: TV float32 targets (LDS or global). start < 0 leaves the first state free, else only the states
//   (start << K | b) & (2^L - 1) may begin (codes.py:164-167). buf: DBL ? 2R : R floats of LDS (with one
//   buffer each step takes a second barrier, between the reads of the old minima and the writes of the new).
//   back: (TV-1) * ACT entries (LDS or global), entry t*ACT + owner holding the winning h of each of the
//   owner's groups for the step that produced B_{t+1}. red: 2*(NT/64) words of LDS.
//   Final state: the lowest among the minimal costs (codes.py:173); traceback codes.py:176-179.
// hook() runs once the forward pass is done (the caller's chance to issue loads that the end of the final argmin and
// the traceback then cover; at L > 12 after the argmin's two passes over the states). BACK_GLOBAL: back-pointers in
// global memory, published to the tracing wave by a full barrier (otherwise only LDS is ordered, and the caller's
// outstanding loads stay in flight).
template <int L, int K, int NT, bool DBL, bool BACK_GLOBAL = false, bool PATHREG = false, typename BackT, class Tab,
          class Hook = NoHook>
__device__ int viterbi_gx(const float* xs, int TV, Tab& tab, int start, float* buf, BackT* back, int* path, float* red,
                          Hook hook = Hook())
{
    using V = VX<L, K, NT>;
    constexpr int G = V::G, NB = V::NB, M = V::M, R = V::R;
    static_assert(G * K <= 8 * (int)sizeof(BackT), "one back-pointer entry per thread and step");
    const int tid = threadIdx.x;
    // every thread owns groups when there are at least NT of them (the kernels launch exactly NT threads): a
    // compile-time true then, and the step loop carries no exec-mask branches
    const bool act = V::ACT >= NT || tid < V::ACT;
    int ent[NB];
#pragma unroll
    for (int h = 0; h < NB; ++h) ent[h] = V::RUN ? h * (R >> K) + M * tid : (h * R + G * tid) >> K;
    float bv[NB][M];
    // ent[h] = ent[0] + h (R >> K); where that stride is a multiple of 256 the swizzle keeps it (swz(x + 256 i) =
    // swz(x) + 256 i), so every h reads at one swizzled index plus a constant offset (one register, not NB)
    constexpr bool EOFF = (R >> K) % 256 == 0;
    const auto load_minima = [&](const float* b, int h) {
        if constexpr (EOFF)
            lds_load_swz<M>(b + h * (R >> K), ent[0], bv[h]);
        else
            lds_load_swz<M>(b, ent[h], bv[h]);
    };
    // the group minima before position 0: 0 for the start's group (every group with a free start), else +inf
    const auto start_minima = [&]() {
        const int rs = start >= 0 ? (start & (R - 1)) : -1;
        const int d = rs - ent[0];  // ent[h] + e == rs exactly when d == h (R >> K) + e
#pragma unroll
        for (int h = 0; h < NB; ++h)
#pragma unroll
            for (int e = 0; e < M; ++e) bv[h][e] = (rs < 0 || d == h * (R >> K) + e) ? 0.0f : __builtin_inff();
    };
    int cur = 0;
    float x = xs[0];
    // From a given start state, position t reaches only the 2^(K (t+1)) states of one aligned range,
    // [(start << K (t+1)) mod 2^L, + 2^(K (t+1))); every other state's cost is +inf there, and so is the group minimum
    // in bv of each of them (a state is reachable exactly when a state of its predecessor group is). Two savings follow,
    // both giving the values the full computation gives. A wave none of whose member states h*R + r lies in the range
    // only stores +inf minima for its groups, and no back-pointers (a traced path never reads a group whose minimum
    // is +inf). While the range spans at most R states (K (t+1) <= L - K) it lies in the slab of one h, hl: every
    // other member of a group is +inf, so the group's minimum is its member hl's cost, bv[hl] + (x - C)^2 (+inf for
    // the groups outside the range, as bv is there), and hl is the winner wherever that is finite. Only for L >= 16:
    // at L = 12 a step is short enough that the wave test costs more than the skipped waves save.
    constexpr bool SKIP = L >= 16;
    constexpr uint32_t REP = [] {  // hl in every group's K-bit field of a back-pointer word
        uint32_t r = 0;
        for (int g = 0; g < G; ++g) r |= 1u << (g * K);
        return r;
    }();
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int st0 = __builtin_amdgcn_readfirstlane(start);
    // whether some member state of this wave is reachable at position p (always, once every state is)
    const auto wave_live = [&](int p) {
        if (!SKIP || st0 < 0 || K * (p + 1) >= L) return true;
        const int span = 1 << (K * (p + 1));
        const int base = (int)(((uint32_t)st0 << (K * (p + 1))) & (uint32_t)(V::NS - 1));
        const int w0 = wv * 64 * G;  // the wave's first group
        bool lv = false;
#pragma unroll
        for (int h = 0; h < NB; ++h) {
            const int lo = h * R + w0;
            lv = lv || (lo < base + span && base < lo + 64 * G);
        }
        return lv;
    };
    // A wave none of whose members is reachable stores +inf minima only where its groups' entries in the target buffer
    // may hold finite values: stale from an earlier search (both buffers at the start) or written at an earlier
    // position. dirty0/1 track that per buffer, so a wave that stays unreachable stores its +inf once per buffer; and a
    // wave unreachable at the next position skips the loads of its members' minima (it computes nothing there).
    bool dirty0 = true, dirty1 = true;
    bool live = wave_live(0);
    // one step of the search, position t, reading minima buffer cur (written into cur ^ 1 with two buffers)
    const auto step = [&](const int t, int& cur) {
        const float xn = xs[t + 1];
        const int base = (SKIP && st0 >= 0 && K * (t + 1) < L)
                             ? (int)(((uint32_t)st0 << (K * (t + 1))) & (uint32_t)(V::NS - 1)) : 0;
        const bool one_h = SKIP && st0 >= 0 && K * (t + 1) <= L - K;
        const bool tgt1 = DBL && cur == 0;  // the buffer this step writes: cur ^ 1 (DBL), else the only one
        if (act && !live && (tgt1 ? dirty1 : dirty0)) {
            constexpr int CKI = V::RUN ? NB : G;
            float* dst = buf + (DBL ? (cur ^ 1) * R : 0);
            float infs[CKI];
#pragma unroll
            for (int i = 0; i < CKI; ++i) infs[i] = __builtin_inff();
#pragma unroll
            for (int e = 0; e < G / CKI; ++e) lds_store_swz<CKI>(dst, G * tid + e * CKI, infs);
        }
        if (tgt1)
            dirty1 = live;
        else
            dirty0 = live;
        if (act && live && one_h) {
            tab.hold();
            float* dst = buf + (DBL ? (cur ^ 1) * R : 0);
            auto step1 = [&](auto hc) {
                constexpr int HL = decltype(hc)::value;
                constexpr int CK = V::RUN ? NB : G;
#pragma unroll
                for (int e = 0; e < G / CK; ++e) {
                    float best[CK];
#pragma unroll
                    for (int gg = 0; gg < CK; ++gg) best[gg] = bv[HL][e] + tab.dsq(x, HL * G + e * CK + gg);
                    lds_store_swz<CK>(dst, G * tid + e * CK, best);
                }
                back[t * V::ACT + tid] = (BackT)((uint32_t)HL * REP);
            };
            uniform_switch<0, NB>(base >> (L - K), step1);
        }
        if (act && live && !one_h) {
            tab.hold();
            uint32_t bits = 0;
            float* dst = buf + (DBL ? (cur ^ 1) * R : 0);
            // groups in chunks of CK sharing one B entry per h (RUN) or all of them; each chunk stored when done
            constexpr int CK = V::RUN ? NB : G;
            // with the tournament below (K = 2 in the 16-bit-state kernels) the groups are visited from the last to the
            // first, so that the winning h can be shifted in bit by bit
            constexpr bool TOUR = NB == 2 || (NB == 4 && L > 12);
#pragma unroll
            for (int ei = 0; ei < G / CK; ++ei) {
                const int e = TOUR ? G / CK - 1 - ei : ei;
                float best[CK];
#pragma unroll
                for (int gi = 0; gi < CK; ++gi) {
                    const int gg = TOUR ? CK - 1 - gi : gi;
                    const int g = e * CK + gg;
                    float c[NB];
#pragma unroll
                    for (int h = 0; h < NB; ++h) c[h] = bv[h][e] + tab.dsq(x, h * G + g);
                    // the minimum, then the lowest h attaining it (costs are never NaN: finite or +inf)
                    if constexpr (NB == 2) {
                        // the second state wins only if strictly lower; its bit enters as a carry-in
                        const uint64_t lo = __builtin_amdgcn_ballot_w64(c[1] < c[0]);
                        best[gg] = fminf(c[0], c[1]);
                        bits = shift_in(bits, lo);
                    } else if constexpr (TOUR) {
                        // (at L <= 12 the extra register it takes would cost the kernel a wave of occupancy)
                        // a two-level tournament with strict comparisons (a tie keeps the left, lower, side): the
                        // winning pair hi = (min(c2,c3) < min(c0,c1)), then within it lo; h = 2 hi + lo enters bits
                        // [2g, 2g+2) as two carry-ins (bits = 2 bits + bit), the comparisons staying lane masks
                        // (the minimum as one v_min3 of m01, c2, c3; the right pair wins exactly when it is below m01)
                        const float m01 = fminf(c[0], c[1]);
                        const float mb = fminf(m01, fminf(c[2], c[3]));
                        const uint64_t hi = __builtin_amdgcn_ballot_w64(mb < m01);
                        const uint64_t lo = (hi & __builtin_amdgcn_ballot_w64(c[3] < c[2])) |
                                            (~hi & __builtin_amdgcn_ballot_w64(c[1] < c[0]));
                        best[gg] = mb;
                        bits = shift_in(bits, hi);
                        bits = shift_in(bits, lo);
                    } else {
                        float b = c[0];
#pragma unroll
                        for (int h = 1; h < NB; ++h) b = fminf(b, c[h]);
                        uint32_t hs = NB - 1;
#pragma unroll
                        for (int h = NB - 2; h >= 0; --h) hs = c[h] == b ? (uint32_t)h : hs;
                        best[gg] = b;
                        asm volatile("" : "+v"(hs));  // keeps h a small integer: one shift-or per group, no wide constants
                        bits |= hs << (g * K);
                    }
                }
                lds_store_swz<CK>(dst, G * tid + e * CK, best);
            }
            back[t * V::ACT + tid] = (BackT)bits;
        }
        lds_barrier();
        cur ^= 1;
        x = xn;
        live = wave_live(t + 1);
        if (act && live) {
#pragma unroll
            for (int h = 0; h < NB; ++h) load_minima(buf + (DBL ? cur * R : 0), h);
        }
        if (!DBL) lds_barrier();
    };
    // The ramp of a fixed start. Position t reaches only the 2^(K (t+1)) states base_t + i (i < 2^(K (t+1))),
    // base_t = (start << K (t+1)) mod 2^L, each with exactly one reachable predecessor, base_(t-1) + (i >> K), while
    // the range lies in the slab of one h (K (t+1) <= L - K). The path cost of base_t + i is then that predecessor's
    // cost plus (x_t - C)^2, the value the full step forms (the minimum over one finite member is that member, and
    // 0 + (x_0 - C)^2 at position 0). Positions 0 .. T1 are therefore taken by every thread at once with no exchange
    // and no barrier: thread tid follows the ancestors of the states i0 .. i0 + Q - 1 of T1's range (i0 = Q tid; at
    // position t the distinct ancestors ((i0 + j) >> K (T1 - t)), j < Q), reading the table from memory, and stores
    // their costs as the minima of their groups rb + i (T1's range covers groups rb .. rb + SPAN - 1); the owners of
    // the groups outside it store +inf. Each thread also writes its back-pointer word of every position its groups
    // reach (winner hl = base_t >> (L - K) in every field, as the one-slab step writes them). Minima buffer 0 then holds
    // exactly the minima of position T1 and the steps go on from T1 + 1. T1 is the last position whose range fits the
    // slab (T0) where the table is small (L <= 12: float32, 16 KB), and at most the one whose range holds one state per
    // thread at L = 16: there a wider ramp reads more of the 128 KB fp16 table from memory than the one-slab steps
    // (register-held table, one barrier each) that take the positions up to T0 cost.
    constexpr int LNT = LAMQ_RAMP_LOG_STATES;
    constexpr int T0 = (L - K) / K - 1;  // the last position whose range fits one slab
    constexpr int T1 = L <= 12 ? T0 : (LNT / K - 1 < T0 ? LNT / K - 1 : T0);
    constexpr int LS = K * (T1 + 1);  // log2 of T1's range
    constexpr bool RAMP = V::R >= NT && T1 >= 1;
    int tb = 0;
    if constexpr (RAMP) {
        if (st0 >= 0 && T1 <= TV - 2) {
            constexpr int SPAN = 1 << LS;
            constexpr int Q = SPAN > NT ? SPAN / NT : 1;  // states a thread takes
            constexpr int CK4 = G < 4 ? G : 4;
            static_assert(SPAN >= G && SPAN % Q == 0, "T1's range: whole blocks of G groups, Q states a thread");
            const uint32_t su = (uint32_t)st0;
            const int rb = (int)((su << LS) & (uint32_t)(R - 1));
            if (G * tid < rb || G * tid >= rb + SPAN) {
                float infs[CK4];
#pragma unroll
                for (int i = 0; i < CK4; ++i) infs[i] = __builtin_inff();
#pragma unroll
                for (int e = 0; e < G / CK4; ++e) lds_store_swz<CK4>(buf, G * tid + e * CK4, infs);
            }
            if (Q * tid < SPAN) {
                // the offset through an opaque move: the addresses below are formed here, not hoisted out of the
                // caller's loop over searches (held across it, they would take registers the steps need)
                uint32_t ii = (uint32_t)(Q * tid);
                asm volatile("" : "+v"(ii));
                // depth first, to keep few costs live: positions 0 .. TC, where all of this thread's states share one
                // ancestor, once; then the states in chunks of CH, each chunk's ancestors at TC + 1 .. T1 (at
                // position t the chunk's distinct ancestors ((i0 + CH c) >> K (T1 - t)) + j)
                constexpr int LGQ = __builtin_ctz(Q);
                constexpr int TC = T1 - ((LGQ + K - 1) / K > 1 ? (LGQ + K - 1) / K : 1);  // (T1 itself is a chunk's)
                constexpr int CH = Q < 8 ? Q : 8;
                constexpr int CPN = (CH >> K) > 0 ? (CH >> K) : 1;  // a chunk's ancestors at T1 - 1
                float c0 = 0.0f;  // the start's group minimum
                const auto common = [&](auto tc) {
                    constexpr int t = decltype(tc)::value;
                    const uint32_t idx = ((su << (K * (t + 1))) & (uint32_t)(V::NS - 1)) + (ii >> (K * (T1 - t)));
                    c0 = c0 + tab.dsq_at(xs[t], idx);
                };
                static_for<0, TC + 1>(common);
#pragma unroll
                for (int cc = 0; cc < Q / CH; ++cc) {
                    // one chunk's table loads at a time (issued all at once they take a register each)
                    __builtin_amdgcn_sched_barrier(0);
                    const uint32_t ic = ii + (uint32_t)(CH * cc);
                    float cp[CPN];
                    cp[0] = c0;
                    const auto pos = [&](auto tc) {
                        constexpr int t = decltype(tc)::value;
                        constexpr int SH = K * (T1 - t);
                        constexpr int NTS = (CH >> SH) > 0 ? (CH >> SH) : 1;
                        const uint32_t idx = ((su << (K * (t + 1))) & (uint32_t)(V::NS - 1)) + (ic >> SH);
                        const float xt = xs[t];
                        float cn[NTS];
                        if constexpr (NTS == 1) {
                            cn[0] = cp[0] + tab.dsq_at(xt, idx);
                        } else {
#pragma unroll
                            for (int j = 0; j < NTS; j += 2) {
                                float q0, q1;
                                tab.dsq_at2(xt, idx + j, q0, q1);
                                cn[j] = cp[j >> K] + q0;
                                cn[j + 1] = cp[(j + 1) >> K] + q1;
                            }
                        }
                        if constexpr (t < T1) {
#pragma unroll
                            for (int j = 0; j < NTS; ++j) cp[j] = cn[j];
                        } else {
                            lds_store_swz<CH>(buf, rb + (int)ic, cn);
                        }
                    };
                    static_for<TC + 1, T1 + 1>(pos);
                }
            }
            // the back-pointer words of positions 0 .. T1: thread tid's, where its groups are reached (the word's address
            // formed from an opaque copy of tid, so that the T1 + 1 addresses are not hoisted out of the caller's loop
            // over searches and held across it)
            int to = tid;
            asm volatile("" : "+v"(to));
            BackT* const bw = back + to;
            const auto words = [&](auto tc) {
                constexpr int t = decltype(tc)::value;
                constexpr int span = 1 << (K * (t + 1));
                constexpr int no = span >= G ? span / G : 1;
                const uint32_t base = (su << (K * (t + 1))) & (uint32_t)(V::NS - 1);
                const int olo = (int)(base & (uint32_t)(R - 1)) / G;
                if (tid >= olo && tid < olo + no) bw[t * V::ACT] = (BackT)((base >> (L - K)) * REP);
            };
            static_for<0, T1 + 1>(words);
            lds_barrier();
            dirty0 = wave_live(T1);
            dirty1 = true;
            cur = 0;
            x = xs[T1 + 1];
            live = wave_live(T1 + 1);
            if (act && live) {
#pragma unroll
                for (int h = 0; h < NB; ++h) load_minima(buf, h);
            }
            if (!DBL) lds_barrier();
            tb = T1 + 1;
        }
    }
    if (tb == 0) start_minima();
    if constexpr (L <= 12 && DBL) {
        // a step at L <= 12 is short: two steps per iteration, each with its buffer a constant (immediate LDS offsets
        // instead of addresses formed every step); step t reads buffer (t - tb) & 1
        int t = tb;
        for (; t + 1 < TV - 1; t += 2) {
            int c0 = 0, c1 = 1;
            step(t, c0);
            step(t + 1, c1);
        }
        if (t < TV - 1) {
            int c0 = 0;
            step(t, c0);
        }
        cur = (TV - 1 - tb) & 1;
    } else {
        for (int t = tb; t < TV - 1; ++t) step(t, cur);
    }
    int* redi = reinterpret_cast<int*>(red + NT / 64);
    constexpr bool TWOPASS = L > 12;  // (at L <= 12 a thread holds at most 16 states: one pass with the index)
    if constexpr (TWOPASS) {
        // final costs in two passes: the minimum of this thread's states (a v_min3 tree per h; a wave with no reachable
        // member there keeps +inf) and the block's minimum M, then the lowest state attaining M, looked for only in the
        // threads whose own minimum is M (typically one) and there only under the h whose minimum is M (NB <= 8)
        constexpr bool KEEPH = NB <= 8;
        float mh[KEEPH ? NB : 1];
        float mine = __builtin_inff();
        if (act && live) {
            tab.hold();
#pragma unroll
            for (int h = 0; h < NB; ++h) {
                float m = __builtin_inff();
#pragma unroll
                for (int g = 0; g < G; ++g) m = fminf(m, bv[h][V::RUN ? (g >> K) : 0] + tab.dsq(x, h * G + g));
                if constexpr (KEEPH) mh[h] = m;
                mine = fminf(mine, m);
            }
        }
        const float wmin = wave_min(mine);
        if ((tid & 63) == 63) red[tid >> 6] = wmin;
        lds_barrier();
        float mb = red[0];
#pragma unroll
        for (int wv = 1; wv < NT / 64; ++wv) mb = fminf(mb, red[wv]);
        int bi = 0x7fffffff;
        if (act && live && mine == mb) {
            tab.hold();
            // x through an opaque move: the costs are formed again here, not kept from the first pass (64 registers)
            float xo = x;
            asm volatile("" : "+v"(xo));
#pragma unroll
            for (int h = 0; h < NB; ++h) {
                if (bi == 0x7fffffff && (!KEEPH || mh[KEEPH ? h : 0] == mb)) {
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const float c = bv[h][V::RUN ? (g >> K) : 0] + tab.dsq(xo, h * G + g);
                        bi = (c == mb && bi == 0x7fffffff) ? h * R + G * tid + g : bi;
                    }
                }
            }
        }
        hook();  // (after both passes, whose registers the caller's loads would otherwise share)
        const int wbi = wave_imin(bi);
        if ((tid & 63) == 63) redi[tid >> 6] = wbi;
    } else {
        hook();
        // final costs, the lowest state on ties (a thread's states increase with (h, g)); a wave with no reachable
        // member there keeps +inf
        float bvv = __builtin_inff();
        int bi = 0x7fffffff;
        if (act && live) {
            tab.hold();
#pragma unroll
            for (int h = 0; h < NB; ++h)
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float c = bv[h][V::RUN ? (g >> K) : 0] + tab.dsq(x, h * G + g);
                    if ((h == 0 && g == 0) || c < bvv) {
                        bvv = c;
                        bi = h * R + G * tid + g;
                    }
                }
        }
        wave_argmin(bvv, bi);
        if ((tid & 63) == 63) {
            red[tid >> 6] = bvv;
            redi[tid >> 6] = bi;
        }
    }
    if (BACK_GLOBAL)
        __syncthreads();
    else
        lds_barrier();
    int pathv = 0;
    if (tid < 64) {
        // wave 0 traces back; every lane combines the waves' results, so s is uniform
        int s = redi[0];
        if constexpr (TWOPASS) {
#pragma unroll
            for (int wv = 1; wv < NT / 64; ++wv) s = min(s, redi[wv]);
        } else {
            float v = red[0];
#pragma unroll
            for (int wv = 1; wv < NT / 64; ++wv)
                if (red[wv] < v || (red[wv] == v && redi[wv] < s)) {
                    v = red[wv];
                    s = redi[wv];
                }
        }
        // no state attains the minimum only when every final cost is NaN (a NaN target: each cost of that position and
        // every later one is NaN; in one pass the result may then come from a thread that owns no states); the
        // reference's argmin then returns the first entry, state 0, and the traceback below stays inside the
        // back-pointers
        s = (uint32_t)s < (uint32_t)V::NS ? s : 0;
        s = __builtin_amdgcn_readfirstlane(s);
        const auto emit = [&](int c, int sc) {
            if (PATHREG)
                pathv = tid == c ? sc : pathv;
            else if (tid == 0)
                path[c] = sc;
        };
        emit(TV - 1, s);
        // D steps per round trip to the back-pointers: lane 0 reads the word of s's group for step t; lanes 1..NB
        // the words of the groups step t-1 continues from (one per h that step t may pick); with D = 3, lanes
        // NB+1 .. NB+NB^2 those of step t-2 (one per pair of picks). Then the picks resolve through readlane.
        constexpr int D = (1 + NB + NB * NB <= 64) ? 3 : 2;
        constexpr int LG = __builtin_ctz(G);
        const int lane = tid;
        const int level = lane == 0 ? 0 : (lane <= NB ? 1 : ((D == 3 && lane <= NB + NB * NB) ? 2 : 0));
        const uint32_t sp1 = (uint32_t)(level == 1 ? lane - 1 : (level == 2 ? (lane - 1 - NB) / NB : 0)) * R;
        const uint32_t sp2 = (uint32_t)(level == 2 ? (lane - 1 - NB) % NB : 0) * R;
        const auto pick = [&](uint32_t word, uint32_t r) {  // the state before r's group at that step
            return r + ((word >> ((r & (G - 1)) * K)) & (uint32_t)(NB - 1)) * (uint32_t)R;
        };
        int t = TV - 1;
        for (; t >= D; t -= D) {
            const uint32_t r = (uint32_t)s >> K;
            uint32_t grp = r;
            if (level >= 1) grp = (grp + sp1) >> K;
            if (level >= 2) grp = (grp + sp2) >> K;
            const uint32_t wd = (uint32_t)back[(t - 1 - level) * V::ACT + (grp >> LG)];
            const uint32_t s1 = pick((uint32_t)__builtin_amdgcn_readfirstlane((int)wd), r);
            const uint32_t h1 = s1 >> (L - K);
            const uint32_t s2 = pick((uint32_t)__builtin_amdgcn_readlane((int)wd, 1 + h1), s1 >> K);
            emit(t - 1, (int)s1);
            emit(t - 2, (int)s2);
            if (D == 3) {
                const uint32_t h2 = s2 >> (L - K);
                const uint32_t s3 = pick((uint32_t)__builtin_amdgcn_readlane((int)wd, 1 + NB + h1 * NB + h2), s2 >> K);
                emit(t - 3, (int)s3);
                s = (int)s3;
            } else {
                s = (int)s2;
            }
        }
        for (; t >= 1; --t) {
            const uint32_t r = (uint32_t)s >> K;
            s = (int)pick((uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)back[(t - 1) * V::ACT + (r >> LG)]), r);
            emit(t - 1, s);
        }
        if (PATHREG && tid < TV) path[tid] = pathv;
    }
    lds_barrier();
    return pathv;
}

// ------------------------------------------------------------------------------------------------ block row
// The block's columns of one row as the lazy sweep sees them when the block starts: trow[c] = Tr[b0 + c] for
// c < nplain (T holds every earlier update there), and for nplain <= c < nc (the look-ahead past the caller's run, at
// most LAMQ_WMAX + 8 columns) trow[c] = Tr[b0 + c] - sum_{l < pre} Zr[l] U[b0 - pre + l][b0 + c]: those columns still
// lack the trailing updates (syntax.py:123) of the run's pre earlier columns, which the caller applies past the run
// in one product only after the run. Zr: the row's coefficients of those columns. The first wave takes the updated
// columns, its lanes as 4 column pairs x 16 slices of l (lane = 4 * slice + pair): slice s sums l = s, s + 16, ... as
// an fma chain in increasing l, and four butterfly steps add the slices in a fixed order (every lane ends with the
// same bits).
template <int NT>
__device__ __forceinline__ void load_block_row(double* trow, const double* __restrict__ Tr, int64_t b0, int nplain,
                                               int nc, const double* __restrict__ Zr, int pre,
                                               const double* __restrict__ U, int64_t ldU)
{
    const int tid = threadIdx.x;
    const int plain = pre > 0 ? nplain : nc;
    for (int c = tid; c < plain; c += NT) trow[c] = Tr[b0 + c];
    if (pre <= 0 || tid >= 64) return;
    constexpr int SL = 16;
    const int pr = tid & 3, sl = tid >> 2;
    const double* Ub = U + (b0 - pre) * ldU + b0;
    for (int c0 = nplain; c0 < nc; c0 += 8) {
        const int c = c0 + 2 * pr;
        const bool in0 = c < nc, in1 = c + 1 < nc;
        double a0 = 0.0, a1 = 0.0;
        if (in0) {
#pragma unroll 4
            for (int l = sl; l < pre; l += SL) {
                const double* p = Ub + (int64_t)l * ldU + c;
                const double z = Zr[l];
                a0 = fma(z, p[0], a0);
                a1 = fma(z, in1 ? p[1] : 0.0, a1);
            }
        }
#pragma unroll
        for (int o = 4; o < 64; o <<= 1) {
            a0 += __shfl_xor(a0, o);
            a1 += __shfl_xor(a1, o);
        }
        if (sl == 0) {
            if (in0) trow[c] = Tr[b0 + c] - a0;
            if (in1) trow[c + 1] = Tr[b0 + c + 1] - a1;
        }
    }
}

// ------------------------------------------------------------------------------------------------ refit
// One block step of the fused sweep settles w <= 16 columns j..j+w of a row (syntax.py:109-121):
//   E = T[j+c] - table64[path[c]] * S
//   z = E U_BB^-1: z[c] = (E[c] - sum_{l<c} z[l] U[j+l][j+c]) / U[j+c][j+c], an fma chain in l (one wave)
//   T[col] = T[col] - sum_l z[l] U[j+l][col] for col in [j+w, b1), the sum an fma chain from l = 0
// The U operands do not depend on the row's search, so they are fetched before it and arrive while it runs.

// E (lanes c < w of wave 0, which also store the states) and the forward substitution by wave 0 given ucol[l] =
// U[j+l][j+c] for lane c = tid % 16. Writes z to zs (LDS) and Zj.
// E (lanes c < w of wave 0, which also store the states) and the forward substitution by wave 0 given ucolf(l) =
// U[j+l][j+c] for lane c = tid % 16 and q = table64[path[c]] (lanes c < w). The diagonal enters through its
// reciprocal, as BLAS trsm kernels apply it: z[c] = acc * (1 / U[j+c][j+c]). Writes z to zs (LDS) and Zj.
template <class UCol>
__device__ __forceinline__ void refit_solve(UCol ucolf, double* trow, int jo, int w, double q, double Sr, double* Zj,
                                            double* zs)
{
    const int tid = threadIdx.x;
    const int c = tid & (LAMQ_WMAX - 1);
    const double rinv = 1.0 / ucolf(c);
    double e = 0.0;
    if (tid < w) {
        const double qs = q * Sr;
        e = trow[jo + tid] - qs;
    }
    double acc = e, zme = 0.0;
    // U_BB's column in two halves of eight rows (the second fetched only after the first is used)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        double ucol[LAMQ_WMAX / 2];
#pragma unroll
        for (int i = 0; i < LAMQ_WMAX / 2; ++i) ucol[i] = ucolf(half * (LAMQ_WMAX / 2) + i);
#pragma unroll
        for (int i = 0; i < LAMQ_WMAX / 2; ++i) {
            const int l = half * (LAMQ_WMAX / 2) + i;
            if (l < w) {
                const double zl = readlane_f64(acc * rinv, l);
                if (tid == l) zme = zl;
                if (tid > l && tid < w) acc = fma(-zl, ucol[i], acc);
            }
        }
        asm volatile("" ::: "memory");
    }
    if (tid < w) {
        zs[tid] = zme;
        Zj[tid] = zme;
    }
}

// U staged in LDS (the fused kernels with room for it): rows j..j+w of U from column j to b1, fetched by direct
// global->LDS loads before the search (wave v of NT/64 takes rows v, v + NT/64, ...; four 64-dword pieces per
// row), urows[l][c] = U[j+l][j+c]. No registers are held across the search.
template <int NT, int LAZY>
__device__ __forceinline__ void refit_fetch_lds(double (*urows)[LAZY], const double* __restrict__ U, int64_t ldU,
                                                int64_t j, int w, int64_t b1)
{
    static_assert(LAZY * 2 == 4 * 64, "four 64-dword pieces per row");
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int len = 2 * (int)(b1 - j);  // dwords from column j to b1 (<= 2 * LAZY)
    for (int l = wv; l < w; l += NT / 64) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(U + (j + l) * ldU + j);
        const uint32_t dst = lds_addr(&urows[l][0]);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            if (p * 64 < len) {
                const int d = p * 64 + lane;
                load_lds4(src + (d < len ? d : 0), dst + p * 256);  // lanes past b1 fill the row's padding
            }
        }
    }
}

// pv: the path register of the search (wave 0, lane c = path[c]).
template <int NT, int LAZY>
__device__ void refit_apply_lds(double (*urows)[LAZY], double* trow, int jo, int w, int nc, int pv,
                                const double* __restrict__ table64, double Sr, int32_t* states_j, double* Zj,
                                double* zs)
{
    const int tid = threadIdx.x;
    wait_vm<0>();
    double qset = 0.0;
    if (tid < w) {
        qset = table64[pv];
        states_j[tid] = pv;
    }
    lds_barrier();
    if (tid < 64) {
        const int c = tid & (LAMQ_WMAX - 1);
        refit_solve([&](int l) { return urows[l][c]; }, trow, jo, w, qset, Sr, Zj, zs);
    }
    lds_barrier();
    if (tid < nc) {
        double acc = 0.0;
#pragma unroll
        for (int l = 0; l < LAMQ_WMAX; ++l)
            if (l < w) acc = fma(zs[l], urows[l][w + tid], acc);
        trow[jo + w + tid] = trow[jo + w + tid] - acc;
    }
    lds_barrier();
}

// U held in registers (the kernels whose LDS is full): ub, entry (tid/16, tid%16) of the upper triangle of U_BB
// (first 256 threads), staged into LDS (ubb) after the search; uc, CH consecutive terms of one column of the update
// (16/CH threads per column, the chain passed along them in order).
template <int CH>
struct RefitRegs {
    double ub;
    double uc[CH];
};

template <int NT, int CH>
__device__ __forceinline__ void refit_fetch_regs(RefitRegs<CH>& o, const double* __restrict__ U, int64_t ldU, int64_t j,
                                                 int w, int nc)
{
    constexpr int TPC = LAMQ_WMAX / CH;
    static_assert(NT >= LAMQ_WMAX * LAMQ_WMAX, "one U_BB entry per thread");
    const int tid = threadIdx.x;
    o.ub = 0.0;
    if (tid < LAMQ_WMAX * LAMQ_WMAX) {
        const int l = tid / LAMQ_WMAX, c = tid % LAMQ_WMAX;
        if (l <= c && c < w) o.ub = U[(j + l) * ldU + j + c];
    }
    const int col = tid / TPC, q = tid % TPC;
#pragma unroll
    for (int i = 0; i < CH; ++i) o.uc[i] = 0.0;
    if (col < nc) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int l = q * CH + i;
            if (l < w) o.uc[i] = U[(j + l) * ldU + j + w + col];
        }
    }
}

template <int NT, int CH>
__device__ void refit_apply_regs(const RefitRegs<CH>& o, double* trow, int jo, int w, int nc, int pv,
                                 const double* __restrict__ table64, double Sr, int32_t* states_j, double* Zj,
                                 double* ubb, double* zs)
{
    constexpr int TPC = LAMQ_WMAX / CH;
    const int tid = threadIdx.x;
    double qset = 0.0;
    if (tid < w) {
        qset = table64[pv];
        states_j[tid] = pv;
    }
    if (tid < LAMQ_WMAX * LAMQ_WMAX) ubb[tid] = o.ub;
    lds_barrier();
    if (tid < 64) {
        const int c = tid & (LAMQ_WMAX - 1);
        refit_solve([&](int l) { return ubb[l * LAMQ_WMAX + c]; }, trow, jo, w, qset, Sr, Zj, zs);
    }
    lds_barrier();
    const int col = tid / TPC, q = tid % TPC;
    double acc = 0.0;
#pragma unroll
    for (int p = 0; p < TPC; ++p) {
        if (q == p && col < nc) {
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int l = p * CH + i;
                if (l < w) acc = fma(zs[l], o.uc[i], acc);
            }
        }
        if (p + 1 < TPC) acc = __shfl_up(acc, 1, TPC);
    }
    if (q == TPC - 1 && col < nc) trow[jo + w + col] = trow[jo + w + col] - acc;
    lds_barrier();
}
