// Standalone Hadamard-128 rotation (had_r_128, quant/hadamard.cu:125-210) for gfx950.
// y[r, 128c .. 128c+127] = H128(x[r, chunk] (o pre)) * scale / sqrt(128) (o post), 16 lanes per
// 128-element chunk, in place allowed (a chunk is read whole before it is written).
// fp16 data: had_hf_r_128_inner (pre/post scales are fp16 multiplies, fp32 butterfly);
// fp32 data: had_ff_r_128_inner (scales applied in fp32).
#include "exl3_common.cuh"
#include "exl3_kernels.h"

using namespace exl3;

namespace {

// Lane mapping: 16 lanes per 128-element chunk, lane g of the group holds elements 8g .. 8g+7
// (one 16-byte fp16 load, two for fp32), so a wave rotates 4 chunks per step with coalesced
// loads.  Butterfly stages in the reference's order, widths 1, 2, 4 in-lane and 8, 16, 32, 64
// across lanes (DPP xor 1, 2, 4, 8 inside the 16-lane row): every stage writes a + b / a - b with
// one fp32 rounding, so the result is bit-identical to any other placement of the same stages.
__device__ __forceinline__ void fwht8_inlane(float* e)
{
    #pragma unroll
    for (int w = 1; w < 8; w <<= 1)
    {
        #pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            if (i & w) continue;
            const float a = e[i], b = e[i + w];
            e[i] = a + b;
            e[i + w] = a - b;
        }
    }
}

template <int M>
__device__ __forceinline__ void fwht8_stage(float* e, int lane)
{
    const float sg = (lane & M) ? -1.0f : 1.0f;
    #pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        // partner through the LDS crossbar (ds_swizzle): fewer VALU ops than DPP, measured 4-13 %
        // faster on 2048 x {8192, 28672} and 16384 x 4096 rotations
        const float p = xor_partner_sw<M>(e[i]);
        e[i] = __builtin_fmaf(sg, e[i], p);
    }
}

// slab_rows > 0 (fp16 only): y is written in k slabs, [cols / 32][slab_rows][32] (the dense recon
// GEMM's operand layout), not row-major.
template <bool FP32>
__global__ __launch_bounds__(256)
void had128_kernel(const void* __restrict__ in, void* __restrict__ out, long jobs, int cols,
                   const uint16_t* __restrict__ pre, const uint16_t* __restrict__ post, float r_scale,
                   int slab_rows)
{
    const int lane = threadIdx.x & 63;
    const int g = lane & 15;
    const int chunks = cols / 128;
    const long step = (long) gridDim.x * 16;
    for (long base = ((long) blockIdx.x * 4 + (threadIdx.x >> 6)) * 4; base < jobs; base += step)
    {
        const long job = base + (lane >> 4);
        const bool valid = job < jobs;
        const long jc = valid ? job : jobs - 1;
        // jobs row-major over (row, chunk); for slab output chunk-major, so that the 4 consecutive
        // rows of a wave write 4 x 64 contiguous bytes per slab
        long row;
        int c;
        if (slab_rows)
        {
            c = (int) (jc / slab_rows);
            row = jc - (long) c * slab_rows;
        }
        else
        {
            row = jc / chunks;
            c = (int) (jc - row * chunks);
        }
        const int col = c * 128 + 8 * g;
        const size_t idx = (size_t) row * cols + col;
        float e[8];
        if constexpr (FP32)
        {
            const f32x4* src = (const f32x4*) ((const float*) in + idx);
            const f32x4 a = __builtin_nontemporal_load(to_global(src)), b = __builtin_nontemporal_load(to_global(src) + 1);
            e[0] = a.x; e[1] = a.y; e[2] = a.z; e[3] = a.w; e[4] = b.x; e[5] = b.y; e[6] = b.z; e[7] = b.w;
            if (pre)
            {
                const u32x4 sv = *to_global((const u32x4*) (pre + col));
                const uint32_t sw[4] = { sv.x, sv.y, sv.z, sv.w };
                #pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const f16x2 s2 = as_h2(sw[q]);
                    e[2 * q] *= (float) s2.x;
                    e[2 * q + 1] *= (float) s2.y;
                }
            }
        }
        else
        {
            const u32x4 v = __builtin_nontemporal_load(to_global((const u32x4*) ((const uint16_t*) in + idx)));
            uint32_t vw[4] = { v.x, v.y, v.z, v.w };
            if (pre)
            {
                const u32x4 sv = *to_global((const u32x4*) (pre + col));
                const uint32_t sw[4] = { sv.x, sv.y, sv.z, sv.w };
                #pragma unroll
                for (int q = 0; q < 4; ++q) vw[q] = as_u32(as_h2(vw[q]) * as_h2(sw[q]));    // fp16 multiply
            }
            #pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                const f16x2 h = as_h2(vw[q]);
                e[2 * q] = (float) h.x;
                e[2 * q + 1] = (float) h.y;
            }
        }
        fwht8_inlane(e);
        fwht8_stage<1>(e, lane);
        fwht8_stage<2>(e, lane);
        fwht8_stage<4>(e, lane);
        fwht8_stage<8>(e, lane);
        #pragma unroll
        for (int i = 0; i < 8; ++i) e[i] *= r_scale;
        if (!valid) continue;
        if constexpr (FP32)
        {
            if (post)
            {
                const u32x4 sv = *to_global((const u32x4*) (post + col));
                const uint32_t sw[4] = { sv.x, sv.y, sv.z, sv.w };
                #pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const f16x2 s2 = as_h2(sw[q]);
                    e[2 * q] *= (float) s2.x;
                    e[2 * q + 1] *= (float) s2.y;
                }
            }
            f32x4* dst = (f32x4*) ((float*) out + idx);
            __builtin_nontemporal_store((f32x4) { e[0], e[1], e[2], e[3] }, to_global_w(dst));
            __builtin_nontemporal_store((f32x4) { e[4], e[5], e[6], e[7] }, to_global_w(dst) + 1);
        }
        else
        {
            uint32_t ow[4];
            #pragma unroll
            for (int q = 0; q < 4; ++q) ow[q] = as_u32((f16x2) { (f16) e[2 * q], (f16) e[2 * q + 1] });
            if (post)
            {
                const u32x4 sv = *to_global((const u32x4*) (post + col));
                const uint32_t sw[4] = { sv.x, sv.y, sv.z, sv.w };
                #pragma unroll
                for (int q = 0; q < 4; ++q) ow[q] = as_u32(as_h2(ow[q]) * as_h2(sw[q]));  // fp16 multiply
            }
            const size_t oidx = slab_rows ? (size_t) (col >> 5) * slab_rows * 32 + (size_t) row * 32 + (col & 31) : idx;
            __builtin_nontemporal_store((u32x4) { ow[0], ow[1], ow[2], ow[3] },
                                        to_global_w((u32x4*) ((uint16_t*) out + oidx)));
        }
    }
}

// y (rows x cols fp16, k slabs [cols / 32][rows][32]) = x (row-major), with had128_kernel's slab
// mapping: 16 threads per 128-column chunk of a row (16 contiguous bytes each: the group reads
// 256 contiguous bytes), chunk-major over rows, so that the 4 consecutive rows of a wave write
// 4 x 64 contiguous bytes per slab.  Tail chunks of cols % 128 columns: threads past the row end
// do nothing.
__global__ __launch_bounds__(256)
void slab_copy_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int rows, int cols)
{
    const int chunks = (cols + 127) / 128;
    const long total = (long) rows * chunks * 16;
    for (long t = (long) blockIdx.x * 256 + threadIdx.x; t < total; t += (long) gridDim.x * 256)
    {
        const long job = t >> 4;
        const int c = (int) (job / rows);
        const long row = job - (long) c * rows;
        const int col = c * 128 + 8 * (int) (t & 15);
        if (col >= cols) continue;
        const u32x4 v = __builtin_nontemporal_load(to_global((const u32x4*) (x + (size_t) row * cols + col)));
        __builtin_nontemporal_store(v, to_global_w((u32x4*) (y + (size_t) (col >> 5) * rows * 32 + (size_t) row * 32 + (col & 31))));
    }
}

}  // namespace

int exl3k_slab_copy(const uint16_t* x, uint16_t* y, int rows, int cols, hipStream_t s)
{
    const long total = (long) rows * ((cols + 127) / 128) * 16;
    if (total == 0) return 0;
    const long want = (total + 255) / 256;
    hipLaunchKernelGGL(slab_copy_kernel, dim3((unsigned) (want < 4096 ? want : 4096)), dim3(256), 0, s, x, y, rows, cols);
    return (int) hipGetLastError();
}

int exl3k_had128(const void* in, void* out, int rows, int cols, int fp32,
                 const uint16_t* pre, const uint16_t* post, float scale, int slabs, hipStream_t s)
{
    const float r_scale = scale * 0.088388347648f;
    const long jobs = (long) rows * (cols / 128);
    if (jobs == 0) return 0;
    // 16 chunks per workgroup per step; at most 8 workgroups per CU (grid-stride beyond)
    const long want = (jobs + 15) / 16;
    dim3 grid((unsigned) (want < 2048 ? want : 2048));
    if (fp32) hipLaunchKernelGGL(had128_kernel<true>, grid, dim3(256), 0, s, in, out, jobs, cols, pre, post, r_scale, 0);
    else      hipLaunchKernelGGL(had128_kernel<false>, grid, dim3(256), 0, s, in, out, jobs, cols, pre, post, r_scale,
                                 slabs ? rows : 0);
    return (int) hipGetLastError();
}
