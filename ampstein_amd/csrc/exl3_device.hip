// Device-side helpers of the C-ABI layer:
//  - topology probe: which XCD (accelerator complex die, each with its own L2) runs each
//    workgroup.  The GEMV's XCD-local split-k hand-off relies on MI355X dispatching linear
//    workgroup b to XCD (b + c) % 8, c fixed per launch, so workgroups b and b + 8 share an XCD;
//    exl3_amd_init verifies that on the device before enabling it.
//  - word fill: re-zeroes the hand-off counters and owner words after the XCD hand-off check
//    trips (a kernel, not hipMemsetAsync, so that it may sit inside a captured graph).
//  - mgemm expert-range filter (quant/exl3_gemm_kernel.cuh:98-143): selections outside
//    [min_index, max_index) are removed (one token: compacted) or masked to -1 (several tokens),
//    retained indices rebased by min_index.
#include "exl3_common.cuh"
#include "exl3_kernels.h"

#include <algorithm>

namespace {

__global__ void xcd_probe_kernel(int* __restrict__ out)
{
    if (threadIdx.x == 0)
    {
        uint32_t v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
        out[blockIdx.y * gridDim.x + blockIdx.x] = (int) v;
    }
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t v, size_t n)
{
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t) gridDim.x * blockDim.x) p[i] = v;
}

__global__ void mgemm_filter_kernel(const int64_t* __restrict__ indices, const uint16_t* __restrict__ weights,
                                    int bszm, int min_index, int max_index, int num_tokens,
                                    int64_t* __restrict__ idx_out, uint16_t* __restrict__ w_out)
{
    if (threadIdx.x != 0) return;
    if (num_tokens > 1)
    {
        for (int i = 0; i < bszm; ++i)
        {
            const int64_t idx = indices[i];
            const bool keep = idx >= min_index && idx < max_index;
            idx_out[i] = keep ? idx - min_index : -1;
            if (weights) w_out[i] = keep ? weights[i] : (uint16_t) 0;
        }
        return;
    }
    int j = 0;
    for (int i = 0; i < bszm; ++i)
    {
        const int64_t idx = indices[i];
        if (idx >= min_index && idx < max_index)
        {
            idx_out[j] = idx - min_index;
            if (weights) w_out[j] = weights[i];
            ++j;
        }
    }
    for (; j < bszm; ++j) idx_out[j] = -1;
}

}  // namespace

int exl3k_xcd_probe(int* out, int blocks_x, int blocks_y, hipStream_t s)
{
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(blocks_x, blocks_y), dim3(64), 0, s, out);
    return (int) hipGetLastError();
}

int exl3k_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t s)
{
    if (n == 0) return 0;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned) blocks), dim3(256), 0, s, p, v, n);
    return (int) hipGetLastError();
}

int exl3k_mgemm_filter(const int64_t* indices, const uint16_t* weights, int bszm, int min_index,
                       int max_index, int num_tokens, int64_t* idx_out, uint16_t* w_out, hipStream_t s)
{
    hipLaunchKernelGGL(mgemm_filter_kernel, dim3(1), dim3(64), 0, s, indices, weights, bszm, min_index,
                       max_index, num_tokens, idx_out, w_out);
    return (int) hipGetLastError();
}
