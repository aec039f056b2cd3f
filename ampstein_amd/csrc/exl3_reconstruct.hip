// Trellis -> fp16 weight reconstruction for gfx950.
//
//   reconstruct      W_hat (k, n) in the Hadamard basis        (quant/reconstruct.cu:14-98)
//   reconstruct_had  W = diag(suh) H W_hat H diag(svh) per 128x128 block, original basis,
//                    with the reference's fp16 rounding points  (quant/reconstruct.cu:212-364)
//
// Both are bit-exact restatements: the decode is the codebook arithmetic of exl3_common.cuh,
// and every fp16 operation of the fused form is issued in the reference's order (the column
// pass rounds after each add / sub and after the 1/sqrt(128) multiply; the row pass runs its
// first two butterfly stages in fp32, then fp16).
#include "exl3_common.cuh"
#include "exl3_kernels.h"

using namespace exl3;

namespace {

// Load this lane's K words of the 8-tile chunk; ring_prev supplies the word before them.
template <int K>
__device__ __forceinline__ void load_lane_words(const uint32_t* __restrict__ p, uint32_t* w)
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

// Decode one k-slice x 128-column chunk per wave: returns the 16 packed pairs of this lane.
template <int K, int CB>
__device__ __forceinline__ void decode_slice(const uint16_t* __restrict__ trellis, int tiles_n,
                                             int kt, int nt0, int lane, uint32_t* pairs,
                                             const DecodeRegs& r)
{
    constexpr int KB = kbits(K);
    uint32_t wv[KB + 1];
    if constexpr (khalf(K))
    {
        const uint32_t* tile = (const uint32_t*) trellis
                             + ((size_t) kt * tiles_n + nt0 + (lane >> 3)) * tile_words(K);
        load_frame_half<K>(tile, lane & 7, wv);
    }
    else
    {
        const uint32_t* base = (const uint32_t*) trellis
                             + ((size_t) kt * tiles_n + nt0) * (8 * K) + (size_t) lane * K;
        load_lane_words<K>(base, wv + 1);
        wv[0] = ring_prev(wv[K], lane);
    }
    decode_lane32<K, CB>(wv, pairs, r);
}

// ------------------------------------------------------------------------------ reconstruct
// Grid (n / 128, ceil(k / 64)), 256 threads: wave w decodes k-slice 4*blockIdx.y + w of the
// 128-column chunk, transposes through LDS and writes 16 coalesced 256-byte rows.
template <int K, int CB>
__global__ __launch_bounds__(256)
void reconstruct_kernel(uint16_t* __restrict__ W, const uint16_t* __restrict__ trellis,
                        int k, int n, int tiles_n, int nt_off)
{
    __shared__ __align__(16) uint32_t sh[4][16][64 + 4];     // per wave: 16 rows x 128 halves (+pad)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kt = blockIdx.y * 4 + wave;
    const int chunk = blockIdx.x;
    if (kt >= k / 16) return;
    const DecodeRegs r = make_decode_regs<CB>();

    uint32_t pairs[16];
    decode_slice<K, CB>(trellis, tiles_n, kt, nt_off + chunk * 8, lane, pairs, r);

    uint16_t* s16 = (uint16_t*) &sh[wave][0][0];
    const int j = lane & 7, tcol = (lane >> 3) * 16;
    #pragma unroll
    for (int q = 0; q < 16; ++q)
    {
        const int c = tcol + pair_col(j, q), row = pair_row(q);
        s16[row * 136 + c] = (uint16_t) pairs[q];
        s16[(row + 1) * 136 + c] = (uint16_t)(pairs[q] >> 16);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // 4 stores of 64 lanes x 16 bytes: lane -> row (4i + lane/16), 8 halves at (lane%16)*8
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int row = 4 * i + (lane >> 4), c8 = (lane & 15) * 8;
        u32x4 v = *(const u32x4*) (s16 + row * 136 + c8);
        *(u32x4*) (W + (size_t) (kt * 16 + row) * n + chunk * 128 + c8) = v;
    }
}

// ---------------------------------------------------------------------------- reconstruct_t
// W_hat transposed, (n, k) row-major: the layout the recon GEMM reads fastest (both operands
// k-contiguous).  Same grid as reconstruct_kernel: wave w decodes k-slice 4 blockIdx.y + w of the
// chunk; lane (tile t, j) holds the 16 rows of columns j and j + 8 of its tile, i.e. 32-byte runs
// of two transposed rows.  The workgroup's 128 columns x 64 k meet in LDS and leave as whole
// 128-byte lines (8 threads per transposed row).
//
// With svh (the rotated branch of the recon GEMM), every k row of the tile is then rotated
// across its 128 columns and scaled: W' = W_hat H128 diag(svh) / sqrt(128), fp32 butterflies from
// the fp16 weights, one fp16 rounding.  y = had(x o suh) @ W' then needs no output rotation.
template <int K, int CB>
__global__ __launch_bounds__(256)
void reconstruct_t_kernel(uint16_t* __restrict__ WT, const uint16_t* __restrict__ trellis,
                          int k, int tiles_n, int nt_off, const uint16_t* __restrict__ svh, int slabs)
{
    __shared__ __align__(16) uint32_t sh[128][32 + 4];    // [column][64 k as 32 pairs] (+pad)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kt = blockIdx.y * 4 + wave;
    const int chunk = blockIdx.x;
    const int nks = min(4, k / 16 - blockIdx.y * 4);     // k-slices of this workgroup
    if (wave < nks)
    {
        const DecodeRegs r = make_decode_regs<CB>();
        uint32_t p[16];
        decode_slice<K, CB>(trellis, tiles_n, kt, nt_off + chunk * 8, lane, p, r);
        // pair q holds rows pair_row(q), +1 of column pair_col(j, q): column j = pairs 0,4,8,12
        // (rows 0-7) and 1,5,9,13 (rows 8-15); column j + 8 = pairs 2,6,10,14 and 3,7,11,15
        const int ca = (lane >> 3) * 16 + (lane & 7);
        *(u32x4*) &sh[ca][8 * wave] = (u32x4) { p[0], p[4], p[8], p[12] };
        *(u32x4*) &sh[ca][8 * wave + 4] = (u32x4) { p[1], p[5], p[9], p[13] };
        *(u32x4*) &sh[ca + 8][8 * wave] = (u32x4) { p[2], p[6], p[10], p[14] };
        *(u32x4*) &sh[ca + 8][8 * wave + 4] = (u32x4) { p[3], p[7], p[11], p[15] };
    }
    __syncthreads();
    if (svh)
    {
        // wave w: k pairs 8 w .. 8 w + 7; lane l holds columns 2 l, 2 l + 1 (the GEMV output layout)
        const f16x2 sv = as_h2(*to_global((const uint32_t*) (svh + chunk * 128 + 2 * lane)));
        const float s0 = (float) sv.x * EXL3_HAD_RSCALE, s1 = (float) sv.y * EXL3_HAD_RSCALE;
        #pragma unroll 2
        for (int q = 0; q < 8; ++q)
        {
            const int pr = 8 * wave + q;
            const f16x2 a = as_h2(sh[2 * lane][pr]), b = as_h2(sh[2 * lane + 1][pr]);
            float a0 = (float) a.x, b0 = (float) b.x, a1 = (float) a.y, b1 = (float) b.y;
            fwht128_wave(a0, b0, lane);
            fwht128_wave(a1, b1, lane);
            sh[2 * lane][pr] = as_u32((f16x2) { (f16) (a0 * s0), (f16) (a1 * s0) });
            sh[2 * lane + 1][pr] = as_u32((f16x2) { (f16) (b0 * s1), (f16) (b1 * s1) });
        }
        __syncthreads();
    }
    // 128 rows x (nks x 32 bytes): thread t writes 16-byte piece t % 8 of rows t / 8 + 32 i
    const int piece = threadIdx.x & 7;
    if (piece < 2 * nks)
    {
        #pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const int row = (threadIdx.x >> 3) + 32 * i;
            const u32x4 v = *(const u32x4*) &sh[row][4 * piece];
            const int kk = blockIdx.y * 64 + 8 * piece;
            // k slabs ([k / 32][n][32], n = gridDim.x * 128) or row-major (n, k)
            const size_t o = slabs ? (size_t) (kk >> 5) * gridDim.x * 128 * 32 + (size_t) (chunk * 128 + row) * 32 + (kk & 31)
                                   : (size_t) (chunk * 128 + row) * k + kk;
            *to_global_w((u32x4*) (WT + o)) = v;
        }
    }
}

// -------------------------------------------------------------------------- reconstruct_had
// One 128x128 block per workgroup.  LDS holds the block as 128 rows x 64 dwords with the
// dword index of (row R, column pair cp) swizzled to cp ^ (2 * ((R >> 2) & 31)): conflict-free
// for the column pass (32 lanes, 4 rows each, one column pair) and 8-byte aligned for the row
// pass (32 lanes, 4 columns each).
__device__ __forceinline__ int rh_dw(int R, int cp) { return R * 64 + (cp ^ (((R >> 2) & 31) << 1)); }


// fp16 lane stages xor 1..16 within a 32-lane half: lower lane a + b, upper (-b) + a
// (shuffle_had_h2x32, hadamard_inner.cuh:83-93).  The partner value moves by DPP / permlane
// (exl3_common.cuh xor_partner), not through LDS.
template <int M>
__device__ __forceinline__ f16x2 had_h2_stage(f16x2 v, int lane)
{
    // one v_pk_fma_f16 with a +-1 factor: exactly v + p (lower lane) or p - v (upper), one rounding
    // the partner through the LDS crossbar: this kernel is VALU-bound (measured 8 % faster than
    // the DPP partner)
    const f16x2 p = as_h2(__builtin_bit_cast(uint32_t, xor_partner_sw<M>(__builtin_bit_cast(float, as_u32(v)))));
    const f16 sg = (lane & M) ? (f16) -1.0f : (f16) 1.0f;
    const f16x2 sg2 = { sg, sg };
    return __builtin_elementwise_fma(v, sg2, p);
}

// Stage-major over N independent values, so each DPP read has other values' work in front of it
// instead of the read-after-write wait states of one chain.
template <int N>
__device__ __forceinline__ void had_h2x32_n(f16x2 (&v)[N], int lane)
{
    #pragma unroll
    for (int i = 0; i < N; ++i) v[i] = had_h2_stage<1>(v[i], lane);
    #pragma unroll
    for (int i = 0; i < N; ++i) v[i] = had_h2_stage<2>(v[i], lane);
    #pragma unroll
    for (int i = 0; i < N; ++i) v[i] = had_h2_stage<4>(v[i], lane);
    #pragma unroll
    for (int i = 0; i < N; ++i) v[i] = had_h2_stage<8>(v[i], lane);
    #pragma unroll
    for (int i = 0; i < N; ++i) v[i] = had_h2_stage<16>(v[i], lane);
}

__device__ __forceinline__ f16x2 had_h2x32(f16x2 v, int lane)
{
    v = had_h2_stage<1>(v, lane);
    v = had_h2_stage<2>(v, lane);
    v = had_h2_stage<4>(v, lane);
    v = had_h2_stage<8>(v, lane);
    return had_h2_stage<16>(v, lane);
}

// TR: write the block transposed, WT (n, k) row-major (the layout the recon route's dense GEMM
// reads): the row pass leaves its fp16 results in LDS, then each wave stores whole 128-element
// columns.  The values are those of the (k, n) form, bit for bit.
template <int K, int CB, bool TR>
__global__ __launch_bounds__(256)
void reconstruct_had_kernel(uint16_t* __restrict__ W, const uint16_t* __restrict__ trellis,
                            const uint16_t* __restrict__ suh, const uint16_t* __restrict__ svh,
                            int n, int tiles_n, int nt_off, int k, int slabs)
{
    __shared__ __align__(16) uint32_t blk[128 * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = blockIdx.x, kb = blockIdx.y;
    const DecodeRegs r = make_decode_regs<CB>();
    uint16_t* b16 = (uint16_t*) blk;

    // 1. decode 8 k-slices x 8 tiles (wave w: slices w, w + 4)
    #pragma unroll
    for (int it = 0; it < 2; ++it)
    {
        const int js = wave + 4 * it;
        uint32_t pairs[16];
        decode_slice<K, CB>(trellis, tiles_n, kb * 8 + js, nt_off + nb * 8, lane, pairs, r);
        const int j = lane & 7, tcol = (lane >> 3) * 16;
        #pragma unroll
        for (int q = 0; q < 16; ++q)
        {
            const int c = tcol + pair_col(j, q), R = js * 16 + pair_row(q);
            b16[rh_dw(R, c >> 1) * 2 + (c & 1)] = (uint16_t) pairs[q];
            b16[rh_dw(R + 1, c >> 1) * 2 + (c & 1)] = (uint16_t)(pairs[q] >> 16);
        }
    }
    __syncthreads();

    const f16x2 rs2 = { (f16) 0.08838834764831845f, (f16) 0.08838834764831845f };
    const int t = lane & 31, half = lane >> 5;

    // 2. column pass (reconstruct.cu:290-325): per column pair, rows 4t..4t+3 in lane t;
    //    fp16 4-point stage, times rs, fp16 lane stages
    for (int it = 0; it < 8; ++it)
    {
        const int cp = (wave * 8 + it) * 2 + half;
        f16x2 v[4];
        #pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = as_h2(blk[rh_dw(4 * t + i, cp)]);
        f16x2 s0 = v[0] + v[1], d0 = v[0] - v[1];
        f16x2 s1 = v[2] + v[3], d1 = v[2] - v[3];
        v[0] = (s0 + s1) * rs2;
        v[1] = (d0 + d1) * rs2;
        v[2] = (s0 - s1) * rs2;
        v[3] = (d0 - d1) * rs2;
        had_h2x32_n<4>(v, lane);
        #pragma unroll
        for (int i = 0; i < 4; ++i) blk[rh_dw(4 * t + i, cp)] = as_u32(v[i]);
    }
    __syncthreads();

    // 3. row pass fused with the store (reconstruct.cu:331-357): row R, columns 4t..4t+3 in
    //    lane t; fp32 4-point stage, round, times rs in fp16, fp16 lane stages, * suh * svh
    const uint32_t sv01 = ((const uint32_t*) svh)[nb * 64 + 2 * t];
    const uint32_t sv23 = ((const uint32_t*) svh)[nb * 64 + 2 * t + 1];
    for (int it = 0; it < 16; ++it)
    {
        const int R = (wave * 16 + it) * 2 + half;
        const int d = rh_dw(R, 2 * t);
        f16x2 a = as_h2(blk[d]), b = as_h2(blk[d + 1]);
        float v0 = (float) a.x, v1 = (float) a.y, v2 = (float) b.x, v3 = (float) b.y;
        float s0 = v0 + v1, d0 = v0 - v1, s1 = v2 + v3, d1 = v2 - v3;
        f16x2 h01 = { (f16) (s0 + s1), (f16) (d0 + d1) };
        f16x2 h23 = { (f16) (s0 - s1), (f16) (d0 - d1) };
        h01 = h01 * rs2;
        h23 = h23 * rs2;
        f16x2 hh[2] = { h01, h23 };
        had_h2x32_n<2>(hh, lane);
        h01 = hh[0];
        h23 = hh[1];
        const f16 su = as_h(suh[kb * 128 + R]);
        const f16x2 su2 = { su, su };
        h01 = (h01 * su2) * as_h2(sv01);
        h23 = (h23 * su2) * as_h2(sv23);
        if constexpr (TR)
        {
            blk[d] = as_u32(h01);                          // in place: this lane's own words
            blk[d + 1] = as_u32(h23);
        }
        else
        {
            u32x2 o = { as_u32(h01), as_u32(h23) };
            *(u32x2*) (W + (size_t) (kb * 128 + R) * n + nb * 128 + 4 * t) = o;
        }
    }
    if constexpr (TR)
    {
        // 4. transposed store.  Unit (column quad q, row group g) = columns 4 q .. 4 q + 3 at k rows
        //    8 g .. 8 g + 7 of the block: eight ds_read_b64 (the quad's two column-pair dwords of a
        //    row sit side by side: the swizzle flips even bits only), repacked by v_perm into four
        //    16-byte runs of 8 k, one per column.  Thread t takes units t and t + 256 (g = unit % 16,
        //    so 16 consecutive lanes store one column's 128 k contiguously; with slabs, 4 x 64 bytes).
        //    (The former store, one u32 of two 16-bit LDS reads per lane and column, took ~290 us
        //    at 8192 x 28672 against ~215 us for the (k, n) form.)
        __syncthreads();
        #pragma unroll
        for (int u = 0; u < 2; ++u)
        {
            const int unit = threadIdx.x + 256 * u;
            const int q = unit >> 4, g = unit & 15;
            uint32_t lo[8], hi[8];
            #pragma unroll
            for (int i = 0; i < 8; ++i)
            {
                const u32x2 v = *(const u32x2*) &blk[rh_dw(8 * g + i, 2 * q)];
                lo[i] = v.x;                                   // columns 4 q, 4 q + 1
                hi[i] = v.y;                                   // columns 4 q + 2, 4 q + 3
            }
            const int kk = kb * 128 + 8 * g;
            #pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                const uint32_t* src = j < 2 ? lo : hi;
                const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;   // high or low halves
                const u32x4 o = { __builtin_amdgcn_perm(src[1], src[0], sel), __builtin_amdgcn_perm(src[3], src[2], sel),
                                  __builtin_amdgcn_perm(src[5], src[4], sel), __builtin_amdgcn_perm(src[7], src[6], sel) };
                const int c = nb * 128 + 4 * q + j;
                const size_t off = slabs ? (size_t) (kk >> 5) * n * 32 + (size_t) c * 32 + (kk & 31)
                                         : (size_t) c * k + kk;
                *(u32x4*) (W + off) = o;
            }
        }
    }
}

template <int K, int CB>
int launch_reconstruct_t(uint16_t* W, const uint16_t* trellis, int k, int n, int tiles_n,
                         int nt_off, hipStream_t s)
{
    dim3 grid(n / 128, (k / 16 + 3) / 4);
    hipLaunchKernelGGL((reconstruct_kernel<K, CB>), grid, dim3(256), 0, s, W, trellis, k, n, tiles_n, nt_off);
    return (int) hipGetLastError();
}

template <int K, int CB>
int launch_reconstruct_tr(uint16_t* WT, const uint16_t* trellis, int k, int n, int tiles_n,
                          int nt_off, const uint16_t* svh, int slabs, hipStream_t s)
{
    dim3 grid(n / 128, (k / 16 + 3) / 4);
    hipLaunchKernelGGL((reconstruct_t_kernel<K, CB>), grid, dim3(256), 0, s, WT, trellis, k, tiles_n, nt_off, svh, slabs);
    return (int) hipGetLastError();
}

template <int K, int CB>
int launch_reconstruct_had_t(uint16_t* W, const uint16_t* trellis, const uint16_t* suh,
                             const uint16_t* svh, int k, int n, int tiles_n, int nt_off,
                             hipStream_t s)
{
    dim3 grid(n / 128, k / 128);
    hipLaunchKernelGGL((reconstruct_had_kernel<K, CB, false>), grid, dim3(256), 0, s, W, trellis, suh, svh, n, tiles_n,
                       nt_off, k, 0);
    return (int) hipGetLastError();
}

template <int K, int CB>
int launch_reconstruct_had_tr(uint16_t* WT, const uint16_t* trellis, const uint16_t* suh,
                              const uint16_t* svh, int k, int n, int tiles_n, int nt_off,
                              int slabs, hipStream_t s)
{
    dim3 grid(n / 128, k / 128);
    hipLaunchKernelGGL((reconstruct_had_kernel<K, CB, true>), grid, dim3(256), 0, s, WT, trellis, suh, svh, n, tiles_n,
                       nt_off, k, slabs);
    return (int) hipGetLastError();
}

}  // namespace

#define EXL3_DISPATCH_K_CB(K, CB, FN, ...)                                        \
    switch (CB * 32 + K)                                                          \
    {                                                                             \
        case 2 * 32 + 17: return FN<17, 2>(__VA_ARGS__);                          \
        case 2 * 32 + 18: return FN<18, 2>(__VA_ARGS__);                          \
        case 2 * 32 + 19: return FN<19, 2>(__VA_ARGS__);                          \
        case 0 * 32 + 1: return FN<1, 0>(__VA_ARGS__);                            \
        case 0 * 32 + 2: return FN<2, 0>(__VA_ARGS__);                            \
        case 0 * 32 + 3: return FN<3, 0>(__VA_ARGS__);                            \
        case 0 * 32 + 4: return FN<4, 0>(__VA_ARGS__);                            \
        case 0 * 32 + 5: return FN<5, 0>(__VA_ARGS__);                            \
        case 0 * 32 + 6: return FN<6, 0>(__VA_ARGS__);                            \
        case 0 * 32 + 7: return FN<7, 0>(__VA_ARGS__);                            \
        case 0 * 32 + 8: return FN<8, 0>(__VA_ARGS__);                            \
        case 1 * 32 + 1: return FN<1, 1>(__VA_ARGS__);                            \
        case 1 * 32 + 2: return FN<2, 1>(__VA_ARGS__);                            \
        case 1 * 32 + 3: return FN<3, 1>(__VA_ARGS__);                            \
        case 1 * 32 + 4: return FN<4, 1>(__VA_ARGS__);                            \
        case 1 * 32 + 5: return FN<5, 1>(__VA_ARGS__);                            \
        case 1 * 32 + 6: return FN<6, 1>(__VA_ARGS__);                            \
        case 1 * 32 + 7: return FN<7, 1>(__VA_ARGS__);                            \
        case 1 * 32 + 8: return FN<8, 1>(__VA_ARGS__);                            \
        case 2 * 32 + 1: return FN<1, 2>(__VA_ARGS__);                            \
        case 2 * 32 + 2: return FN<2, 2>(__VA_ARGS__);                            \
        case 2 * 32 + 3: return FN<3, 2>(__VA_ARGS__);                            \
        case 2 * 32 + 4: return FN<4, 2>(__VA_ARGS__);                            \
        case 2 * 32 + 5: return FN<5, 2>(__VA_ARGS__);                            \
        case 2 * 32 + 6: return FN<6, 2>(__VA_ARGS__);                            \
        case 2 * 32 + 7: return FN<7, 2>(__VA_ARGS__);                            \
        case 2 * 32 + 8: return FN<8, 2>(__VA_ARGS__);                            \
    }                                                                             \
    return -1;

int exl3k_reconstruct(uint16_t* W, const uint16_t* trellis, int k, int n, int tiles_n,
                      int nt_off, int K, int cb, hipStream_t s)
{
    EXL3_DISPATCH_K_CB(K, cb, launch_reconstruct_t, W, trellis, k, n, tiles_n, nt_off, s)
}

int exl3k_reconstruct_had(uint16_t* W, const uint16_t* trellis, const uint16_t* suh,
                          const uint16_t* svh, int k, int n, int tiles_n, int nt_off,
                          int K, int cb, hipStream_t s)
{
    EXL3_DISPATCH_K_CB(K, cb, launch_reconstruct_had_t, W, trellis, suh, svh, k, n, tiles_n, nt_off, s)
}

int exl3k_reconstruct_tr(uint16_t* WT, const uint16_t* trellis, int k, int n, int tiles_n,
                         int nt_off, int K, int cb, const uint16_t* svh, int slabs, hipStream_t s)
{
    EXL3_DISPATCH_K_CB(K, cb, launch_reconstruct_tr, WT, trellis, k, n, tiles_n, nt_off, svh, slabs, s)
}

int exl3k_reconstruct_had_tr(uint16_t* WT, const uint16_t* trellis, const uint16_t* suh,
                             const uint16_t* svh, int k, int n, int tiles_n, int nt_off,
                             int K, int cb, int slabs, hipStream_t s)
{
    EXL3_DISPATCH_K_CB(K, cb, launch_reconstruct_had_tr, WT, trellis, suh, svh, k, n, tiles_n, nt_off, slabs, s)
}
