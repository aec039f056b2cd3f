// Decode-shaped EXL3 GEMV for gfx950: C = had(had(A o suh) @ W_hat) o svh, m = 1..8.
//
// Semantics of exl3_gemv_kernel / exl3_gemm (quant/exl3_gemv_kernel.cuh:186-482), built
// differently for CDNA4:
//   * no cooperative launch: each workgroup owns one 128-column output chunk and a range of
//     128-row input chunks; it recomputes the input rotation had(x o suh) for its own k range
//     from x (2 bytes per input element, negligible next to the weights) into LDS;
//   * split-k across workgroups writes fp32 partials; the last workgroup to arrive on a column
//     chunk (device-scope counter) sums them in split order -- deterministic -- and applies
//     the output rotation and svh, then re-arms the counter, so no memset is needed per call;
//   * trellis words are streamed with 64-lane coalesced non-temporal loads: one k-slice of a
//     128-column chunk (8 tiles, 256*K bytes) per wave instruction group, K words per lane;
//   * decode in registers (exl3_common.cuh), dot products with v_dot2_f32_f16 into fp32
//     accumulators: lane j of tile t owns output columns 16t+j and 16t+j+8, so no cross-lane
//     reduction is needed inside a wave.
//
// Compiled once per K (EXL3_INST_K) to keep build units small.
#include "exl3_common.cuh"
#include "exl3_kernels.h"

#ifndef EXL3_INST_K
#define EXL3_INST_K 4
#endif

using namespace exl3;

namespace {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = 4;

template <int K>
__device__ __forceinline__ void load_words(const uint32_t* __restrict__ p, uint32_t* w)
{
    if constexpr (K % 4 == 0)
    {
        #pragma unroll
        for (int i = 0; i < K / 4; ++i)
        {
            u32x4 v = __builtin_nontemporal_load((const u32x4*) p + i);
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    }
    else if constexpr (K % 2 == 0)
    {
        #pragma unroll
        for (int i = 0; i < K / 2; ++i)
        {
            u32x2 v = __builtin_nontemporal_load((const u32x2*) p + i);
            w[2 * i] = v.x; w[2 * i + 1] = v.y;
        }
    }
    else
    {
        #pragma unroll
        for (int i = 0; i < K; ++i) w[i] = __builtin_nontemporal_load(p + i);
    }
}

// Input rotation of rows [0, m) over chunks [kc0, kc0 + nkc) into LDS (fp16 pairs):
// had_hf_r_128_inner<true,false> (hadamard_inner.cuh:93-150): fp16 pre-scale, fp32
// butterfly, * 1/sqrt(128), round to fp16.
__device__ __forceinline__ void rotate_input(const uint16_t* __restrict__ A, const uint16_t* __restrict__ suh,
                                             uint32_t* xs, int m, int k, int kc0, int nkc, int xs_stride)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int job = wave; job < m * nkc; job += GEMV_WAVES)
    {
        const int row = job / nkc, c = job % nkc;
        const int col = (kc0 + c) * 128 + 2 * lane;
        f16x2 v = as_h2(*(const uint32_t*) (A + (size_t) row * k + col));
        uint32_t out;
        if (suh)
        {
            v = v * as_h2(*(const uint32_t*) (suh + col));
            float v0 = (float) v.x, v1 = (float) v.y;
            fwht128_wave(v0, v1, lane);
            f16x2 o = { (f16) (v0 * EXL3_HAD_RSCALE), (f16) (v1 * EXL3_HAD_RSCALE) };
            out = as_u32(o);
        }
        else out = as_u32(v);
        xs[row * xs_stride + c * 64 + lane] = out;
    }
}

// Output rotation of one fp32 row chunk held as (v0, v1) = elements 2l, 2l+1, then store.
// Half output: had_fh_r_128_inner (hadamard_inner.cuh:216-281); float output: had_ff.
__device__ __forceinline__ void store_output(float v0, float v1, void* C, int c_fp32, const uint16_t* svh,
                                             size_t idx, int col, int lane)
{
    if (svh)
    {
        fwht128_wave(v0, v1, lane);
        v0 *= EXL3_HAD_RSCALE;
        v1 *= EXL3_HAD_RSCALE;
        f16x2 s = as_h2(*(const uint32_t*) (svh + col));
        if (c_fp32)
        {
            v0 *= (float) s.x;
            v1 *= (float) s.y;
        }
        else
        {
            f16x2 h = { (f16) v0, (f16) v1 };
            h = h * s;
            *(uint32_t*) ((uint16_t*) C + idx) = as_u32(h);
            return;
        }
    }
    if (c_fp32)
    {
        float2 o = { v0, v1 };
        *(float2*) ((float*) C + idx) = o;
    }
    else
    {
        f16x2 h = { (f16) v0, (f16) v1 };
        *(uint32_t*) ((uint16_t*) C + idx) = as_u32(h);
    }
}

template <int K, int CB, int MT>
__global__ __launch_bounds__(GEMV_THREADS)
void gemv_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ trellis,
                 void* __restrict__ C, const uint16_t* __restrict__ suh,
                 const uint16_t* __restrict__ svh, int m, int k, int n, int c_fp32,
                 int kc_per_split, float* __restrict__ partials, int* __restrict__ counters)
{
    extern __shared__ uint32_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = blockIdx.x, split = blockIdx.y, nsplit = gridDim.y;
    const int kchunks = k / 128;
    const int kc0 = split * kc_per_split;
    const int nkc = min(kc_per_split, kchunks - kc0);
    const int xs_stride = kc_per_split * 64;            // u32 (fp16 pairs) per row
    uint32_t* xs = smem;                                 // [MT][kc_per_split * 64]
    float* red = (float*) (smem + MT * xs_stride);       // [GEMV_WAVES][MT][128]

    rotate_input(A, suh, xs, m, k, kc0, nkc, xs_stride);
    __syncthreads();

    const DecodeRegs r = make_decode_regs<CB>();
    const int tiles_n = n / 16;
    const int nslices = nkc * 8;
    const int kt0 = kc0 * 8;
    // wave w handles local slices w, w + 4, ... : the 4 waves stream 4 adjacent 256K-byte rows
    const int myn = nslices > wave ? (nslices - wave + GEMV_WAVES - 1) / GEMV_WAVES : 0;
    const uint32_t* bp = (const uint32_t*) trellis
                       + ((size_t) (kt0 + wave) * tiles_n + chunk * 8) * (8 * K) + (size_t) lane * K;
    const size_t wstride = (size_t) GEMV_WAVES * tiles_n * 8 * K;   // u32 between my slices

    float acc[MT][2];
    #pragma unroll
    for (int i = 0; i < MT; ++i) acc[i][0] = acc[i][1] = 0.0f;

    constexpr int PF = K <= 4 ? 4 : 2;
    uint32_t ring[PF][K];
    #pragma unroll
    for (int d = 0; d < PF; ++d)
        if (d < myn) load_words<K>(bp + d * wstride, ring[d]);

    for (int i0 = 0; i0 < myn; i0 += PF)
    {
        #pragma unroll
        for (int d = 0; d < PF; ++d)
        {
            const int i = i0 + d;
            if (i >= myn) break;
            uint32_t wv[K + 1];
            #pragma unroll
            for (int w = 0; w < K; ++w) wv[w + 1] = ring[d][w];
            if (i + PF < myn) load_words<K>(bp + (size_t) (i + PF) * wstride, ring[d]);
            wv[0] = ring_prev(wv[K], lane);
            uint32_t pairs[16];
            decode_lane32<K, CB>(wv, pairs, r);

            const int sl = wave + i * GEMV_WAVES;         // local slice index
            #pragma unroll
            for (int row = 0; row < MT; ++row)
            {
                if (MT > 1 && row >= m) break;
                const u32x4* xp = (const u32x4*) (xs + row * xs_stride + sl * 8);
                u32x4 xa = xp[0], xb = xp[1];
                uint32_t x8[8] = { xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w };
                #pragma unroll
                for (int q = 0; q < 16; ++q)
                {
                    const int xi = (q >> 2) + 4 * (q & 1);      // rows pair_row(q), +1
                    float& a = acc[row][(q >> 1) & 1];
                    a = __builtin_amdgcn_fdot2(as_h2(x8[xi]), as_h2(pairs[q]), a, false);
                }
            }
        }
    }

    // cross-wave reduction (fixed order), columns: tile (lane / 8), col j and j + 8
    const int c0 = (lane >> 3) * 16 + (lane & 7);
    #pragma unroll
    for (int row = 0; row < MT; ++row)
    {
        if (MT > 1 && row >= m) break;
        red[(wave * MT + row) * 128 + c0] = acc[row][0];
        red[(wave * MT + row) * 128 + c0 + 8] = acc[row][1];
    }
    __syncthreads();

    __shared__ int last;
    if (nsplit > 1)
    {
        for (int idx = threadIdx.x; idx < m * 128; idx += GEMV_THREADS)
        {
            const int row = idx >> 7, c = idx & 127;
            float s = red[row * 128 + c];
            #pragma unroll
            for (int w = 1; w < GEMV_WAVES; ++w) s += red[(w * MT + row) * 128 + c];
            partials[((size_t) split * m + row) * n + chunk * 128 + c] = s;
        }
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0)
        {
            int prev = __hip_atomic_fetch_add(counters + chunk, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            last = prev == nsplit - 1;
            if (last) __hip_atomic_store(counters + chunk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last) return;
        __threadfence();
    }

    // epilogue: one wave per row: sum splits in order, output rotation, store
    for (int row = wave; row < m; row += GEMV_WAVES)
    {
        float v[2];
        #pragma unroll
        for (int e = 0; e < 2; ++e)
        {
            const int c = 2 * lane + e;
            float s;
            if (nsplit > 1)
            {
                s = 0.0f;
                for (int sp = 0; sp < nsplit; ++sp)
                    s += __builtin_nontemporal_load(partials + ((size_t) sp * m + row) * n + chunk * 128 + c);
            }
            else
            {
                s = red[row * 128 + c];
                #pragma unroll
                for (int w = 1; w < GEMV_WAVES; ++w) s += red[(w * MT + row) * 128 + c];
            }
            v[e] = s;
        }
        const int col = chunk * 128 + 2 * lane;
        store_output(v[0], v[1], C, c_fp32, svh, (size_t) row * n + col, col, lane);
    }
}

template <int K, int CB, int MT>
int launch_gemv_t(const GemvArgs& g, hipStream_t s)
{
    const int kchunks = g.k / 128;
    const int kcps = (kchunks + g.splits - 1) / g.splits;
    const int nsplit = (kchunks + kcps - 1) / kcps;
    const size_t lds = (size_t) MT * kcps * 64 * 4 + (size_t) GEMV_WAVES * MT * 128 * 4;
    dim3 grid(g.n / 128, nsplit);
    hipLaunchKernelGGL((gemv_kernel<K, CB, MT>), grid, dim3(GEMV_THREADS), lds, s,
                       g.A, g.trellis, g.C, g.suh, g.svh, g.m, g.k, g.n, g.c_fp32, kcps,
                       g.partials, g.counters);
    return (int) hipGetLastError();
}

template <int K, int CB>
int launch_gemv_m(const GemvArgs& g, hipStream_t s)
{
    if (g.m == 1) return launch_gemv_t<K, CB, 1>(g, s);
    if (g.m <= 4) return launch_gemv_t<K, CB, 4>(g, s);
    return launch_gemv_t<K, CB, 8>(g, s);
}

}  // namespace

#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)

int EXL3_CAT(exl3k_gemv_k, EXL3_INST_K)(const GemvArgs& g, int cb, hipStream_t s)
{
    switch (cb)
    {
        case 0: return launch_gemv_m<EXL3_INST_K, 0>(g, s);
        case 1: return launch_gemv_m<EXL3_INST_K, 1>(g, s);
        case 2: return launch_gemv_m<EXL3_INST_K, 2>(g, s);
    }
    return -1;
}
