// Prefill-shaped EXL3 GEMM for gfx950 (m > 8): C = had(A_had @ W_hat) o svh with fp16 MFMA
// and fp32 accumulation.  Semantics of exl3_gemm_kernel / exl3_gemm_kernel_inner
// (quant/exl3_gemm_kernel.cuh:8-84, quant/exl3_gemm_inner.cuh:31-1009): the output Hadamard
// reads the fp32 sums (had_fh / had_ff, hadamard_inner.cuh:154-281), the input rotation A_had =
// had_hf(A o suh) is written by the caller-side pre-pass (exl3k_had128).
//
// Tiling.  A workgroup (4 waves) owns a 256-row x 128-column output tile; wave w the 32 columns
// [32w, 32w + 32) of it for all 256 rows: eight v_mfma_f32_32x32x16_f16 accumulators (128
// fp32 per lane).  Per 16-row k-slice the workgroup stages the A slice (256 x 16 fp16) and the
// slice's 8 trellis tiles in LDS (double buffer, register prefetch PF slices deep), and every
// lane decodes exactly the 8 weights of its MFMA B operand -- each weight of the tile once per
// workgroup.
//
// B operand from the trellis.  MFMA lane l holds column l % 32 and k-slots 8(l/32)..+7.  The
// k order inside a slice is free as long as A uses the same: lane (column c, half h) takes the
// tile positions 32(c%8) + 4(c/8) + 16h + 8q + j (q < 2, j < 4), which are rows
// rho_h = {0,1,8,9,2,3,10,11} (h = 0) / {4,5,12,13,6,7,14,15} (h = 1) of column c
// (make_tc_perm, cpu/moe_mul1.cpp:124-139), a 12-position run of the bit ring: the lane
// normalises its run to bit 0 with one alignbit per word, then all 8 windows sit at
// compile-time offsets.  A is staged into LDS in the same permuted k order.
//
// Weights are the reference's fp16 values exactly: 3INST / MCG lo + hi rounded by one
// v_pk_add_f16 per pair, MUL1 by v_pk_fma_f16 (codebook.cuh:57-90).
//
// Compiled once per K (EXL3_INST_K).
#include "exl3_common.cuh"
#include "exl3_kernels.h"

#ifndef EXL3_INST_K
#define EXL3_INST_K 4
#endif

using namespace exl3;

namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float acc16 __attribute__((ext_vector_type(16)));

constexpr int GT = 256;          // threads per workgroup
constexpr int BM = 256;          // rows per workgroup
constexpr int BN = 128;          // columns per workgroup
constexpr int PF = 4;            // register prefetch depth, k-slices

template <int K> struct GemmLds
{
    static constexpr int TW = 8 * K + 1;                 // words per staged tile: ring word -1, then 8K
    static constexpr int A_U32 = BM * 8;                 // one A slice: 256 rows x 16 fp16
    static constexpr int T_U32 = 8 * TW;                 // 8 tiles
    static constexpr int BUF = A_U32 + T_U32;
};

// 16-bit window at MSB-first bit offset REL of a normalised word run.
template <int REL>
__device__ __forceinline__ uint32_t win16(const uint32_t* nw)
{
    constexpr int w = REL / 32, off = REL % 32;
    if constexpr (off <= 16) return __builtin_amdgcn_ubfe(nw[w], 16 - off, 16);
    else return __builtin_amdgcn_alignbit(nw[w], nw[w + 1], 48 - off) & 0xffffu;
}

template <int CB>
__device__ __forceinline__ uint32_t cb_raw(uint32_t s)
{
    if constexpr (CB == 0) return ((s * 89226354u + 64248484u) & 0x8fff8fffu) ^ 0x3b603b60u;   // codebook.cuh:61-63
    else if constexpr (CB == 1) return ((s * 0xCBAC1FEDu) & 0x8fff8fffu) ^ 0x3b603b60u;        // codebook.cuh:69-72
    else return __builtin_amdgcn_sad_u8(s * 0x83DCD12Du, 0u, 0x6400u);                        // codebook.cuh:78-84
}

// Two decoded weights (slots i, i + 1) packed as the fp16 pair of one B-operand register.
template <int CB>
__device__ __forceinline__ uint32_t weight_pair(uint32_t r0, uint32_t r1)
{
    if constexpr (CB == 2)
    {
        const f16x2 h = as_h2(__builtin_amdgcn_perm(r1, r0, 0x05040100u));
        const f16x2 kinv = { as_h(0x1eee), as_h(0x1eee) }, bias = { as_h(0xc931), as_h(0xc931) };
        return as_u32(__builtin_elementwise_fma(h, kinv, bias));                   // fp16 fma, one rounding
    }
    else
    {
        const f16x2 lo = as_h2(__builtin_amdgcn_perm(r1, r0, 0x05040100u));
        const f16x2 hi = as_h2(__builtin_amdgcn_perm(r1, r0, 0x07060302u));
        return as_u32(lo + hi);                                                    // fp16 add, one rounding
    }
}

// This lane's B operand for one k-slice: 8 weights of column (l % 32), k-slots 8h..8h+7.
template <int K, int CB>
__device__ __forceinline__ void decode_b(const uint32_t* __restrict__ tl, int sh, uint32_t* b)
{
    constexpr int NW = (11 * K + 16 + 31) / 32;          // normalised words covering the run
    uint32_t rw[NW + 1], nw[NW + 1];
    #pragma unroll
    for (int i = 0; i <= NW; ++i) rw[i] = tl[i];
    #pragma unroll
    for (int i = 0; i < NW; ++i) nw[i] = __builtin_amdgcn_alignbit(rw[i], rw[i + 1], 32 - sh);
    nw[NW] = 0u;
    uint32_t r[8];
    r[0] = cb_raw<CB>(win16<0 * K>(nw));
    r[1] = cb_raw<CB>(win16<1 * K>(nw));
    r[2] = cb_raw<CB>(win16<2 * K>(nw));
    r[3] = cb_raw<CB>(win16<3 * K>(nw));
    r[4] = cb_raw<CB>(win16<8 * K>(nw));
    r[5] = cb_raw<CB>(win16<9 * K>(nw));
    r[6] = cb_raw<CB>(win16<10 * K>(nw));
    r[7] = cb_raw<CB>(win16<11 * K>(nw));
    #pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = weight_pair<CB>(r[2 * i], r[2 * i + 1]);
}

// Output rotation of one fp32 row chunk (elements 2l, 2l+1) and store: had_fh / had_ff.
__device__ __forceinline__ void gemm_store(float v0, float v1, void* C, int c_fp32, bool has_svh, uint32_t svp,
                                           size_t idx, int lane)
{
    if (has_svh)
    {
        fwht128_wave(v0, v1, lane);
        v0 *= EXL3_HAD_RSCALE;
        v1 *= EXL3_HAD_RSCALE;
        const f16x2 s = as_h2(svp);
        if (!c_fp32)
        {
            f16x2 h = { (f16) v0, (f16) v1 };
            h = h * s;
            *(uint32_t*) ((uint16_t*) C + idx) = as_u32(h);
            return;
        }
        v0 *= (float) s.x;
        v1 *= (float) s.y;
    }
    if (c_fp32)
    {
        f32x2 o = { v0, v1 };
        *(f32x2*) ((float*) C + idx) = o;
    }
    else
    {
        f16x2 h = { (f16) v0, (f16) v1 };
        *(uint32_t*) ((uint16_t*) C + idx) = as_u32(h);
    }
}

template <int K, int CB>
__global__ __launch_bounds__(GT, 1)
void gemm_kernel(const uint16_t* __restrict__ Ain, const uint16_t* __restrict__ trellis, void* __restrict__ C,
                 const uint16_t* __restrict__ svh, int M, int k, int n, int c_fp32)
{
    using LD = GemmLds<K>;
    __shared__ __align__(16) uint32_t lds[2 * LD::BUF + 4];   // +4: the last tile's run may read one word past it
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = threadIdx.x;
    const int KS = k / 16;
    const int nbn = n / BN, nmb = (M + BM - 1) / BM;

    // workgroup -> (column chunk, row block): the row blocks of one column chunk run together on
    // one XCD (workgroup b on XCD b % 8) when the chunk count allows, sharing its trellis in L2
    int nb, mb;
    if (nbn % 8 == 0)
    {
        const int x = blockIdx.x % 8, r = blockIdx.x / 8;
        nb = x + 8 * (r / nmb);
        mb = r % nmb;
    }
    else
    {
        nb = blockIdx.x / nmb;
        mb = blockIdx.x % nmb;
    }

    // ---- staging assignment: thread t holds A row t of the block, and (t < 16K) trellis words 4t..4t+3
    const int arow = min(mb * BM + t, M - 1);
    const uint32_t* ag = (const uint32_t*) (Ain + (size_t) arow * k);                 // + 8 u32 per slice
    const int tn = n / 16;
    const bool tload = t < 16 * K;
    const uint32_t* tg = (const uint32_t*) trellis + (size_t) nb * 8 * (8 * K) + (tload ? 4 * t : 0);
    const size_t tstride = (size_t) tn * 8 * K;                                         // u32 per k-slice row

    // ---- decode assignment: column c of tile tt, half h
    const int h = lane >> 5;
    const int col32 = lane & 31;
    const int tt = 2 * wave + (col32 >> 4);
    const int c = col32 & 15;
    const int base_pos = 32 * (c & 7) + 4 * (c >> 3) + 16 * h;
    const int B0 = (base_pos + 1) * K - 16;             // first window's first bit (may be < 0: ring)
    const int f = B0 - 1 >= 0 ? (B0 - 1) / 32 : -1;     // first staged word (-1: the ring word)
    const int sh = B0 - 32 * f;                         // 1..32
    const int toff = LD::A_U32 + tt * LD::TW + 1 + f;   // LDS word of that first word

    uint32_t apf[PF][8];
    u32x4 tpf[PF];
    auto load_slice = [&](int s, uint32_t* a, u32x4& tw) {
        const int sc = min(s, KS - 1);
        const u32x4 lo = __builtin_nontemporal_load((const u32x4*) (ag + 8 * sc));
        const u32x4 hi = __builtin_nontemporal_load((const u32x4*) (ag + 8 * sc) + 1);
        // permuted k order: pairs 0,4,1,5 | 2,6,3,7 (columns rho_0 | rho_1)
        a[0] = lo.x; a[1] = hi.x; a[2] = lo.y; a[3] = hi.y;
        a[4] = lo.z; a[5] = hi.z; a[6] = lo.w; a[7] = hi.w;
        tw = __builtin_nontemporal_load((const u32x4*) (tg + sc * tstride));
    };
    // LDS slots of this thread's 4 trellis words (and the ring copy of a tile's last word)
    int tli[4], tring = -1;
    #pragma unroll
    for (int e = 0; e < 4; ++e)
    {
        const int j = 4 * t + e;
        const int tile = j / (8 * K), wi = j - tile * (8 * K);
        tli[e] = LD::A_U32 + tile * LD::TW + 1 + wi;
        if (wi == 8 * K - 1) tring = LD::A_U32 + tile * LD::TW;
    }
    auto store_slice = [&](uint32_t* buf, const uint32_t* a, const u32x4& tw) {
        *(u32x4*) (buf + 8 * t) = (u32x4) { a[0], a[1], a[2], a[3] };
        *(u32x4*) (buf + 8 * t + 4) = (u32x4) { a[4], a[5], a[6], a[7] };
        if (tload)
        {
            buf[tli[0]] = tw.x; buf[tli[1]] = tw.y; buf[tli[2]] = tw.z; buf[tli[3]] = tw.w;
            if (tring >= 0) buf[tring] = tw.w;          // a tile's last word is always e = 3 (8K % 4 == 0)
        }
    };

    #pragma unroll
    for (int d = 0; d < PF; ++d) load_slice(d, apf[d], tpf[d]);
    store_slice(lds, apf[0], tpf[0]);
    load_slice(PF, apf[0], tpf[0]);
    __syncthreads();

    acc16 acc[8];
    #pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = (acc16) { };

    for (int s0 = 0; s0 < KS; s0 += PF)
    {
        #pragma unroll
        for (int d = 0; d < PF; ++d)
        {
            const int s = s0 + d;
            if (s >= KS) break;
            const uint32_t* buf = lds + (s & 1) * LD::BUF;
            uint32_t b[4];
            decode_b<K, CB>(buf + toff, sh, b);
            const h8v bv = __builtin_bit_cast(h8v, (u32x4) { b[0], b[1], b[2], b[3] });
            #pragma unroll
            for (int mt = 0; mt < 8; ++mt)
            {
                const u32x4 av = *(const u32x4*) (buf + 8 * (mt * 32 + col32) + 4 * h);
                acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, av), bv, acc[mt], 0, 0, 0);
            }
            if (s + 1 < KS)
            {
                const int nd = (d + 1) % PF;
                store_slice(lds + ((s + 1) & 1) * LD::BUF, apf[nd], tpf[nd]);
                load_slice(s + 1 + PF, apf[nd], tpf[nd]);
            }
            __syncthreads();
        }
    }

    // ---- epilogue: per 32-row tile, exchange through LDS so each row's 128 columns meet in one wave
    float* E = (float*) lds;                              // [32][128] fp32
    const bool has_svh = svh != nullptr;
    const uint32_t svp = has_svh ? *(const uint32_t*) (svh + nb * BN + 2 * lane) : 0u;
    #pragma unroll
    for (int mt = 0; mt < 8; ++mt)
    {
        #pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                E[(8 * j + 4 * h + i) * BN + 32 * wave + col32] = acc[mt][4 * j + i];
        }
        __syncthreads();
        #pragma unroll
        for (int rr = 0; rr < 8; ++rr)
        {
            const int r = 8 * wave + rr;
            const int row = mb * BM + mt * 32 + r;
            const f32x2 v = *(const f32x2*) (E + r * BN + 2 * lane);
            if (row < M)
                gemm_store(v.x, v.y, C, c_fp32, has_svh, svp, (size_t) row * n + nb * BN + 2 * lane, lane);
        }
        __syncthreads();
    }
}

template <int K, int CB>
int launch_gemm(const GemmArgs& g, hipStream_t s)
{
    const int blocks = (g.n / BN) * ((g.m + BM - 1) / BM);
    hipLaunchKernelGGL((gemm_kernel<K, CB>), dim3(blocks), dim3(GT), 0, s,
                       g.A_rot, g.trellis, g.C, g.svh, g.m, g.k, g.n, g.c_fp32);
    return (int) hipGetLastError();
}

}  // namespace

#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)

int EXL3_CAT(exl3k_gemm_k, EXL3_INST_K)(const GemmArgs& g, int cb, hipStream_t s)
{
    switch (cb)
    {
        case 0: return launch_gemm<EXL3_INST_K, 0>(g, s);
        case 1: return launch_gemm<EXL3_INST_K, 1>(g, s);
        case 2: return launch_gemm<EXL3_INST_K, 2>(g, s);
    }
    return -1;
}
