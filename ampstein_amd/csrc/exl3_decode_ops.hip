// Neighbours of the EXL3 linears in the decode step (graphdec.uc:151-230):
//   rms_norm_res  y = fp16(x + r); n = fp16(fp16(y * rsqrt(mean(y^2) + eps)) * w)
//                 (amp_rms_norm_res_kernel, src/torch/amp_kernels.cu:279-365)
//   silu_mul      out = fp16(silu(g) * u), fp32 math (amp_silu_mul_kernel, amp_kernels.cu:235-251)
// One workgroup per row for the norm: 8-byte chunks (4 halves) per thread, the sum of squares
// reduced within each wave by DPP (xor shuffles) and across waves in LDS.  y may alias x.
#include "exl3_common.cuh"
#include "exl3_kernels.h"

using namespace exl3;

namespace {

__device__ __forceinline__ float wave_sum64(float v)
{
    #pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Chunks per thread kept in registers between the two passes (dim <= 4 * 4 * 1024 = 16384);
// wider rows re-read the rest of y from memory.
constexpr int NORM_REG_CHUNKS = 4;

__global__ __launch_bounds__(1024)
void rms_norm_res_kernel(const uint16_t* x, const uint16_t* __restrict__ r, const uint16_t* __restrict__ w,
                         uint16_t* y, uint16_t* __restrict__ n, int dim, float eps)
{
    __shared__ float wsum[16];
    const int row = blockIdx.x, t = threadIdx.x, cnt = dim >> 2;
    const size_t off = (size_t) row * dim;
    float acc = 0.0f;
    u32x2 yk[NORM_REG_CHUNKS], wk[NORM_REG_CHUNKS];
    #pragma unroll
    for (int q = 0; q < NORM_REG_CHUNKS; ++q) { yk[q] = (u32x2) { 0u, 0u }; wk[q] = yk[q]; }
    int q = 0;
    for (int c = t; c < cnt; c += blockDim.x, ++q)
    {
        const u32x2 xv = *to_global((const u32x2*) (x + off) + c);
        const u32x2 rv = *to_global((const u32x2*) (r + off) + c);
        const f16x2 x0 = as_h2(xv.x), x1 = as_h2(xv.y), r0 = as_h2(rv.x), r1 = as_h2(rv.y);
        // fp32 add of two fp16 values rounded once: the fp16 sum exactly
        const f16x2 h0 = { (f16) ((float) x0.x + (float) r0.x), (f16) ((float) x0.y + (float) r0.y) };
        const f16x2 h1 = { (f16) ((float) x1.x + (float) r1.x), (f16) ((float) x1.y + (float) r1.y) };
        const u32x2 hv = { as_u32(h0), as_u32(h1) };
        *((u32x2*) (y + off) + c) = hv;
        #pragma unroll
        for (int j = 0; j < NORM_REG_CHUNKS; ++j)
            if (j == q)
            {
                yk[j] = hv;
                wk[j] = *to_global((const u32x2*) w + c);       // the weights, before the barrier
            }
        const float a = (float) h0.x, b = (float) h0.y, cc = (float) h1.x, d = (float) h1.y;
        acc += a * a + b * b;
        acc += cc * cc + d * d;
    }
    acc = wave_sum64(acc);
    if ((t & 63) == 0) wsum[t >> 6] = acc;
    __syncthreads();
    if (t == 0)
    {
        float total = 0.0f;
        for (int i = 0; i < (int) (blockDim.x >> 6); ++i) total += wsum[i];
        wsum[0] = 1.0f / sqrtf(total / (float) dim + eps);
    }
    __syncthreads();
    const float scale = wsum[0];
    q = 0;
    for (int c = t; c < cnt; c += blockDim.x, ++q)
    {
        u32x2 yv, wv;
        if (q < NORM_REG_CHUNKS)
        {
            #pragma unroll
            for (int j = 0; j < NORM_REG_CHUNKS; ++j)
                if (j == q) { yv = yk[j]; wv = wk[j]; }
        }
        else
        {
            yv = *((const u32x2*) (y + off) + c);
            wv = *to_global((const u32x2*) w + c);
        }
        const f16x2 y0 = as_h2(yv.x), y1 = as_h2(yv.y);
        // normalise in fp32, round to fp16, then the fp16 weight multiply
        const f16x2 n0 = (f16x2) { (f16) ((float) y0.x * scale), (f16) ((float) y0.y * scale) } * as_h2(wv.x);
        const f16x2 n1 = (f16x2) { (f16) ((float) y1.x * scale), (f16) ((float) y1.y * scale) } * as_h2(wv.y);
        *((u32x2*) (n + off) + c) = (u32x2) { as_u32(n0), as_u32(n1) };
    }
}

// Split residual norm, producer half on its own: one wave per (128-column chunk, row), the same
// res_pair_sq as the GEMV epilogue's.  c null adds (-0, -0): h exactly unchanged.
__global__ __launch_bounds__(64)
void res_sq_kernel(uint16_t* h, const uint16_t* __restrict__ c, float* __restrict__ sq, int n)
{
    const int lane = threadIdx.x, chunk = blockIdx.x, row = blockIdx.y;
    const size_t idx = (size_t) row * n + chunk * 128 + 2 * lane;
    const uint32_t cp = c ? *to_global((const uint32_t*) (c + idx)) : 0x80008000u;
    const float t = res_pair_sq(*to_global((const uint32_t*) (h + idx)), cp, h, idx, lane);
    if (lane == 0) sq[(size_t) row * (n / 128) + chunk] = t;
}

// Consumer half on its own: r = norm_pair(h, w, scale); every wave forms the row's scale with
// sq_scale, as the M = 1 stream kernel's waves do.  Grid (n / 512, rows), 4 waves of one chunk.
__global__ __launch_bounds__(256)
void norm_sq_kernel(const uint16_t* __restrict__ h, const float* __restrict__ sq, const uint16_t* __restrict__ w,
                    uint16_t* __restrict__ r, int n, float eps)
{
    const int lane = threadIdx.x & 63, row = blockIdx.y;
    const int chunk = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nch = n / 128;
    float sv[SQ_SCALE_MAX_PER_LANE];
    sq_load(sq + (size_t) row * nch, nch, lane, sv);
    const float scale = sq_scale(sv, n, eps, lane);
    if (chunk >= nch) return;
    const int col = chunk * 128 + 2 * lane;
    const uint32_t yv = *to_global((const uint32_t*) (h + (size_t) row * n + col));
    const uint32_t wv = *to_global((const uint32_t*) (w + col));
    *to_global_w((uint32_t*) (r + (size_t) row * n + col)) = norm_pair(yv, wv, scale);
}

__global__ __launch_bounds__(256)
void silu_mul_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u, uint16_t* __restrict__ out, long n)
{
    for (long i = (long) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long) gridDim.x * blockDim.x)
    {
        const float gf = (float) as_h(g[i]), uf = (float) as_h(u[i]);
        out[i] = h_bits((f16) (silu_f32(gf) * uf));
    }
}

}  // namespace

int exl3k_rms_norm_res(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* y, uint16_t* n,
                       long rows, int dim, float eps, hipStream_t s)
{
    int threads = ((dim / 4 + 63) / 64) * 64;
    threads = threads < 64 ? 64 : (threads > 1024 ? 1024 : threads);
    hipLaunchKernelGGL(rms_norm_res_kernel, dim3((unsigned) rows), dim3(threads), 0, s, x, r, w, y, n, dim, eps);
    return (int) hipGetLastError();
}

int exl3k_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, long n, hipStream_t s)
{
    long grid = (n + 255) / 256;
    if (grid > 2048) grid = 2048;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned) grid), dim3(256), 0, s, g, u, out, n);
    return (int) hipGetLastError();
}

int exl3k_res_sq(uint16_t* h, const uint16_t* c, float* sq, long rows, int n, hipStream_t s)
{
    hipLaunchKernelGGL(res_sq_kernel, dim3((unsigned) (n / 128), (unsigned) rows), dim3(64), 0, s, h, c, sq, n);
    return (int) hipGetLastError();
}

int exl3k_norm_sq(const uint16_t* h, const float* sq, const uint16_t* w, uint16_t* r, long rows, int n, float eps,
                  hipStream_t s)
{
    hipLaunchKernelGGL(norm_sq_kernel, dim3((unsigned) ((n / 128 + 3) / 4), (unsigned) rows), dim3(256), 0, s,
                       h, sq, w, r, n, eps);
    return (int) hipGetLastError();
}
