// Device topology probe: which XCD (accelerator complex die, each with its own L2) runs each
// workgroup.  The GEMV's XCD-local split-k hand-off relies on MI355X dispatching workgroup b to
// XCD b % 8; exl3_amd_init verifies that on the device before enabling it.
#include "exl3_common.cuh"
#include "exl3_kernels.h"

namespace {

__global__ void xcd_probe_kernel(int* __restrict__ out)
{
    if (threadIdx.x == 0)
    {
        uint32_t v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
        out[blockIdx.x] = (int) v;
    }
}

}  // namespace

int exl3k_xcd_probe(int* out, int blocks, hipStream_t s)
{
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(blocks), dim3(64), 0, s, out);
    return (int) hipGetLastError();
}
