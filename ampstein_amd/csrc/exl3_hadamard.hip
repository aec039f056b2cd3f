// Standalone Hadamard-128 rotation (had_r_128, quant/hadamard.cu:125-210) for gfx950.
// y[r, 128c .. 128c+127] = H128(x[r, chunk] (o pre)) * scale / sqrt(128) (o post), one wave64
// per 128-element chunk (lane l holds elements 2l, 2l+1), in place allowed.
// fp16 data: had_hf_r_128_inner (pre/post scales are fp16 multiplies, fp32 butterfly);
// fp32 data: had_ff_r_128_inner (scales applied in fp32).
#include "exl3_common.cuh"
#include "exl3_kernels.h"

using namespace exl3;

namespace {

template <bool FP32>
__global__ __launch_bounds__(256)
void had128_kernel(const void* __restrict__ in, void* __restrict__ out, int rows, int cols,
                   const uint16_t* __restrict__ pre, const uint16_t* __restrict__ post, float r_scale)
{
    const int lane = threadIdx.x & 63;
    const int chunks = cols / 128;
    const long job = (long) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (job >= (long) rows * chunks) return;
    const int row = (int) (job / chunks), c = (int) (job % chunks);
    const int col = c * 128 + 2 * lane;
    const size_t idx = (size_t) row * cols + col;
    float v0, v1;
    if constexpr (FP32)
    {
        float2 v = *(const float2*) ((const float*) in + idx);
        v0 = v.x; v1 = v.y;
        if (pre)
        {
            f16x2 s = as_h2(*(const uint32_t*) (pre + col));
            v0 *= (float) s.x; v1 *= (float) s.y;
        }
    }
    else
    {
        f16x2 v = as_h2(*(const uint32_t*) ((const uint16_t*) in + idx));
        if (pre) v = v * as_h2(*(const uint32_t*) (pre + col));
        v0 = (float) v.x; v1 = (float) v.y;
    }
    fwht128_wave(v0, v1, lane);
    v0 *= r_scale;
    v1 *= r_scale;
    if constexpr (FP32)
    {
        if (post)
        {
            f16x2 s = as_h2(*(const uint32_t*) (post + col));
            v0 *= (float) s.x; v1 *= (float) s.y;
        }
        float2 o = { v0, v1 };
        *(float2*) ((float*) out + idx) = o;
    }
    else
    {
        f16x2 h = { (f16) v0, (f16) v1 };
        if (post) h = h * as_h2(*(const uint32_t*) (post + col));
        *(uint32_t*) ((uint16_t*) out + idx) = as_u32(h);
    }
}

}  // namespace

int exl3k_had128(const void* in, void* out, int rows, int cols, int fp32,
                 const uint16_t* pre, const uint16_t* post, float scale, hipStream_t s)
{
    const float r_scale = scale * 0.088388347648f;
    const long jobs = (long) rows * (cols / 128);
    if (jobs == 0) return 0;
    dim3 grid((unsigned) ((jobs + 3) / 4));
    if (fp32) hipLaunchKernelGGL(had128_kernel<true>, grid, dim3(256), 0, s, in, out, rows, cols, pre, post, r_scale);
    else      hipLaunchKernelGGL(had128_kernel<false>, grid, dim3(256), 0, s, in, out, rows, cols, pre, post, r_scale);
    return (int) hipGetLastError();
}
