// Per-token KL(p_ref || p_q) of bf16 or float32 logits in one streaming pass (compiler.py:177-188).
//
// For a token with logits r (reference) and q (quantized):
//   KL = sum_v p_v ((r_v - lse_r) - (q_v - lse_q)) = (sum_v e^(r_v - m_r) (r_v - q_v)) / s_r - lse_r + lse_q
// with s_r = sum_v e^(r_v - m_r), lse_r = m_r + log s_r and likewise for q. Each thread keeps running
// maxima and sums over its share of the row (16-byte loads of 8 logits, rescaled when a chunk raises
// the maximum); chunk sums are float32 and the running sums float64. The workgroup merges the
// partials in a fixed order, so the result does not depend on scheduling.
#include "common.h"

#include <mutex>

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }

struct KLPart {
    float mr, mq;
    double sr, ar, sq;
};

__device__ __forceinline__ void kl_chunk(KLPart& p, const float (&r)[8], const float (&q)[8], int cnt)
{
    float cr = r[0], cq = q[0];
#pragma unroll
    for (int e = 1; e < 8; ++e)
        if (e < cnt) { cr = fmaxf(cr, r[e]); cq = fmaxf(cq, q[e]); }
    if (cr > p.mr) {
        const double f = (double)__expf(p.mr - cr);
        p.sr *= f;
        p.ar *= f;
        p.mr = cr;
    }
    if (cq > p.mq) {
        p.sq *= (double)__expf(p.mq - cq);
        p.mq = cq;
    }
    // e^(v - m) = 2^(v log2(e) - m log2(e)): one fma and the hardware 2^x per term
    const float l2e = 1.4426950408889634f;
    const float mr2 = p.mr * l2e, mq2 = p.mq * l2e;
    float sr = 0.0f, ar = 0.0f, sq = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        if (e < cnt) {
            const float er = __builtin_amdgcn_exp2f(fmaf(r[e], l2e, -mr2));
            sr += er;
            ar = fmaf(er, r[e] - q[e], ar);
            sq += __builtin_amdgcn_exp2f(fmaf(q[e], l2e, -mq2));
        }
    p.sr += (double)sr;
    p.ar += (double)ar;
    p.sq += (double)sq;
}

__device__ __forceinline__ void kl_merge(KLPart& a, const KLPart& b)
{
    const float mr = fmaxf(a.mr, b.mr), mq = fmaxf(a.mq, b.mq);
    const double fa = a.mr == -__builtin_inff() ? 0.0 : exp((double)a.mr - (double)mr);
    const double fb = b.mr == -__builtin_inff() ? 0.0 : exp((double)b.mr - (double)mr);
    const double ga = a.mq == -__builtin_inff() ? 0.0 : exp((double)a.mq - (double)mq);
    const double gb = b.mq == -__builtin_inff() ? 0.0 : exp((double)b.mq - (double)mq);
    a.sr = a.sr * fa + b.sr * fb;
    a.ar = a.ar * fa + b.ar * fb;
    a.sq = a.sq * ga + b.sq * gb;
    a.mr = mr;
    a.mq = mq;
}

// Eight logits from 16-byte loads (chunk i of the row, whose start is 16-byte aligned), and one logit, as float32:
// a bf16 logit widens exactly, so both element types feed the same float32 arithmetic.
__device__ __forceinline__ void load8(const uint16_t* row, int64_t i, float (&v)[8])
{
    const uint4 x = reinterpret_cast<const uint4*>(row)[i];
    v[0] = bf_lo(x.x); v[1] = bf_hi(x.x); v[2] = bf_lo(x.y); v[3] = bf_hi(x.y);
    v[4] = bf_lo(x.z); v[5] = bf_hi(x.z); v[6] = bf_lo(x.w); v[7] = bf_hi(x.w);
}
__device__ __forceinline__ void load8(const float* row, int64_t i, float (&v)[8])
{
    const float4* p = reinterpret_cast<const float4*>(row) + 2 * i;
    const float4 x = p[0], y = p[1];
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
}
__device__ __forceinline__ float load1(const uint16_t* row, int64_t i) { return __uint_as_float((uint32_t)row[i] << 16); }
__device__ __forceinline__ float load1(const float* row, int64_t i) { return row[i]; }

template <typename Elt>
__global__ __launch_bounds__(256) void kl_rows_kernel(const Elt* __restrict__ ref, const Elt* __restrict__ q,
                                                      int64_t V, int64_t ldr, int64_t ldq, const float* __restrict__ w,
                                                      float* __restrict__ kl, double* __restrict__ wkl,
                                                      double* __restrict__ wt, int vec)
{
    __shared__ KLPart parts[256];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const Elt* r = ref + row * ldr;
    const Elt* p = q + row * ldq;
    KLPart a;
    a.mr = -__builtin_inff();
    a.mq = -__builtin_inff();
    a.sr = a.ar = a.sq = 0.0;
    float rv[8], qv[8];
    int64_t done = 0;
    if (vec) {
        const int64_t nv = V / 8;
        for (int64_t i = tid; i < nv; i += 256) {
            load8(r, i, rv);
            load8(p, i, qv);
            kl_chunk(a, rv, qv, 8);
        }
        done = nv * 8;
    }
    for (int64_t i = done + (int64_t)tid * 8; i < V; i += 256 * 8) {
        int cnt = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const bool in = i + e < V;
            rv[e] = in ? load1(r, i + e) : 0.0f;
            qv[e] = in ? load1(p, i + e) : 0.0f;
            cnt += in ? 1 : 0;
        }
        kl_chunk(a, rv, qv, cnt);
    }
    parts[tid] = a;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) {
            KLPart b = parts[tid + s];
            KLPart c = parts[tid];
            kl_merge(c, b);
            parts[tid] = c;
        }
        __syncthreads();
    }
    if (tid == 0) {
        const KLPart f = parts[0];
        const double lse_r = (double)f.mr + log(f.sr), lse_q = (double)f.mq + log(f.sq);
        const double v = f.ar / f.sr - lse_r + lse_q;
        kl[row] = (float)v;
        const double wr = w ? (double)w[row] : 1.0;
        wkl[row] = wr * v;
        wt[row] = wr;
    }
}

// sums[0] = sum_t wkl[t], sums[1] = sum_t wt[t], in a fixed order.
__global__ __launch_bounds__(256) void kl_sum_kernel(const double* __restrict__ wkl, const double* __restrict__ wt,
                                                     int64_t T, double* __restrict__ sums)
{
    __shared__ double a[256], b[256];
    double x = 0.0, y = 0.0;
    for (int64_t i = threadIdx.x; i < T; i += 256) {
        x += wkl[i];
        y += wt[i];
    }
    a[threadIdx.x] = x;
    b[threadIdx.x] = y;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            a[threadIdx.x] += a[threadIdx.x + s];
            b[threadIdx.x] += b[threadIdx.x + s];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        sums[0] = a[0];
        sums[1] = b[0];
    }
}

extern "C" size_t lamq_kl_workspace_size(int64_t T) { return T > 0 ? (size_t)T * 2 * sizeof(double) : 0; }

// The two launches of both entry points: per-row KL into kl, w*kl and w into wkl[0..T), wkl[T..2T), then their sums.
template <typename Elt>
static int kl_launch(const Elt* ref, const Elt* q, int64_t T, int64_t V, int64_t ldr, int64_t ldq,
                     const float* w, float* kl, double* sums, double* wkl, hipStream_t s)
{
    // 16-byte loads where every row starts 16-byte aligned
    constexpr int64_t per16 = 16 / sizeof(Elt);
    const int vec = ((uintptr_t)ref % 16 == 0) && ((uintptr_t)q % 16 == 0) && (ldr % per16 == 0) && (ldq % per16 == 0);
    double* wt = wkl + T;
    hipLaunchKernelGGL(kl_rows_kernel<Elt>, dim3((unsigned)T), dim3(256), 0, s, ref, q, V, ldr, ldq, w, kl, wkl, wt,
                       vec);
    LAMQ_LAUNCH_CHECK();
    if (sums) {
        hipLaunchKernelGGL(kl_sum_kernel, dim3(1), dim3(256), 0, s, wkl, wt, T, sums);
        LAMQ_LAUNCH_CHECK();
    }
    return LAMQ_OK;
}

extern "C" int lamq_kl_rows(const uint16_t* ref, const uint16_t* q, int64_t T, int64_t V, int64_t ldr, int64_t ldq,
                            const float* w, float* kl, double* sums, void* workspace, size_t workspace_bytes, void* stream)
{
    if (!ref || !q || !kl || T < 0 || V < 1 || ldr < V || ldq < V) return LAMQ_EINVAL;
    if (T == 0) return LAMQ_OK;
    if (!workspace || workspace_bytes < lamq_kl_workspace_size(T)) return LAMQ_EINVAL;
    if (T > 0x7fffffff) return LAMQ_EUNSUP;
    return kl_launch(ref, q, T, V, ldr, ldq, w, kl, sums, reinterpret_cast<double*>(workspace), as_stream(stream));
}

extern "C" int lamq_kl_rows_f32(const float* ref, const float* q, int64_t T, int64_t V, int64_t ldr, int64_t ldq,
                                const float* w, float* kl, double* sums, void* workspace, size_t workspace_bytes,
                                void* stream)
{
    if (!ref || !q || !kl || T < 0 || V < 1 || ldr < V || ldq < V) return LAMQ_EINVAL;
    if (T == 0) return LAMQ_OK;
    if (!workspace || workspace_bytes < lamq_kl_workspace_size(T)) return LAMQ_EINVAL;
    if (T > 0x7fffffff) return LAMQ_EUNSUP;
    return kl_launch(ref, q, T, V, ldr, ldq, w, kl, sums, reinterpret_cast<double*>(workspace), as_stream(stream));
}

// The allocation-free variant's partials: one array per GPU, for the life of the process. In host code `scratch`
// names a host-side stand-in, not device memory; kernels get the device address hipGetSymbolAddress returns for the
// current device, looked up once per device and kept in kl_scratch_ptr.
static __device__ __align__(256) double scratch[2 * LAMQ_KL_NOALLOC_MAX_T];

#define LAMQ_MAX_DEVICES 64
static std::mutex kl_scratch_mu;
static void* kl_scratch_ptr[LAMQ_MAX_DEVICES];

// The device address of this GPU's scratch array (the current device, which must be the stream's).
static int kl_scratch(hipStream_t s, double** out)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= LAMQ_MAX_DEVICES) return LAMQ_EUNSUP;
    if (s) {
        hipDevice_t sdev = -1;
        e = hipStreamGetDevice(s, &sdev);
        if (e != hipSuccess) return (int)e;
        if (sdev != dev) return LAMQ_EINVAL;
    }
    std::lock_guard<std::mutex> lock(kl_scratch_mu);
    if (!kl_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return LAMQ_EINVAL;
        kl_scratch_ptr[dev] = p;
    }
    *out = static_cast<double*>(kl_scratch_ptr[dev]);
    return LAMQ_OK;
}

extern "C" int lamq_kl_rows_noalloc(const uint16_t* ref, const uint16_t* q, int64_t T, int64_t V, int64_t ldr,
                                    int64_t ldq, const float* w, float* kl, double* sums, void* stream)
{
    if (!ref || !q || !kl || T < 0 || V < 1 || ldr < V || ldq < V) return LAMQ_EINVAL;
    if (T > LAMQ_KL_NOALLOC_MAX_T) return LAMQ_EINVAL;
    if (T == 0) return LAMQ_OK;
    hipStream_t s = as_stream(stream);
    double* wkl = nullptr;
    const int rc = kl_scratch(s, &wkl);
    if (rc != LAMQ_OK) return rc;
    return kl_launch(ref, q, T, V, ldr, ldq, w, kl, sums, wkl, s);
}
