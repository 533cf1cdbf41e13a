// Measurement only (no counterpart in the reference): the L2-to-CU delivery ceiling of the direct global->LDS load path
// that the Gram kernels (hessian.hip) feed their MFMAs through. Each workgroup of four waves streams 32 KB stages
// (32 loads of 1 KB, global_load_lds_dwordx4, 16 bytes a lane) from an L2-resident region of its own XCD into a ring
// of LAMQ_PROBE_STAGES LDS buffers, one barrier a stage, as the Gram kernels' stage loop does, and nothing else: with
// five stages (160 KB) one workgroup fits a CU, the Gram kernels' occupancy. Bytes delivered = workgroups x stages x
// 32 KB; bench.py --workload l2 times it and rocprofv3's TCP_TCC_READ_REQ counts it.
#include "common.h"

#define LAMQ_PROBE_STAGES 5
#define LAMQ_PROBE_STAGE_BYTES 32768

__global__ __launch_bounds__(256) void l2_delivery_kernel(const uint8_t* __restrict__ buf, int64_t region_bytes,
                                                          int stages)
{
    __shared__ __align__(16) uint8_t lds[LAMQ_PROBE_STAGES * LAMQ_PROBE_STAGE_BYTES];
    const int64_t b = blockIdx.x;
    const uint8_t* base = buf + (b % LAMQ_XCDS) * region_bytes;  // workgroup b runs on XCD b % 8
    const int64_t nchunk = region_bytes / 1024;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    // load q (0..7) of wave w in stage st: 1 KB chunk (workgroup offset + 32 st + 8 w + q) mod the region's chunks
    auto piece = [&](int64_t st, int q) {
        const int64_t chunk = ((b / LAMQ_XCDS) * 131 + st * 32 + 8 * wv + q) % nchunk;
        const uint32_t m = lds_base + (uint32_t)((st % LAMQ_PROBE_STAGES) * LAMQ_PROBE_STAGE_BYTES + (8 * wv + q) * 1024);
        load_lds16(base + chunk * 1024 + lane * 16, m);
    };
#pragma unroll
    for (int st = 0; st < LAMQ_PROBE_STAGES - 1; ++st)
#pragma unroll
        for (int q = 0; q < 8; ++q) piece(st, q);
    for (int st = 0; st < stages; ++st) {
        wait_vm<8 * (LAMQ_PROBE_STAGES - 2)>();  // stage st has landed (this wave's part)
        __syncthreads();                        // everyone's; the buffer of stage st - 1 is free
#pragma unroll
        for (int q = 0; q < 8; ++q) piece(st + LAMQ_PROBE_STAGES - 1, q);
    }
    wait_vm<0>();  // no load may still be writing this workgroup's LDS when it ends
}

extern "C" int lamq_probe_l2_delivery(const void* buf, int64_t region_bytes, int stages, int workgroups, void* stream)
{
    if (!buf || region_bytes < 65536 || (region_bytes % 1024) != 0 || stages < 1 || workgroups < 1) return LAMQ_EINVAL;
    hipLaunchKernelGGL(l2_delivery_kernel, dim3((unsigned)workgroups), dim3(256), 0, as_stream(stream),
                       reinterpret_cast<const uint8_t*>(buf), region_bytes, stages);
    LAMQ_LAUNCH_CHECK();
    return LAMQ_OK;
}
