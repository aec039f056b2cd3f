// Dense fp16 GEMM of the recon route (exl3_gemm_recon, src/torch/amp_torch.cpp:11083-11230: the
// reference reconstructs the weight to fp16 once and runs a dense GEMM on cuBLAS):
//
//     C (m, n) = A (m, k) . WT (n, k)^T            fp16 operands, fp32 accumulation
//     optional epilogue: each 128-column chunk of the fp32 row rotated by H128 / sqrt(128), x svh
//
// The weight is stored transposed, (n, k) row-major (exl3_amd_reconstruct_t /
// exl3_amd_reconstruct_had_t write it so), so both operands are k-contiguous: a lane's MFMA operand
// (8 consecutive k of one row or column) is one 16-byte LDS read, and both tiles are staged by the
// same LDS DMA with the same swizzle.
//
// Tiling: a workgroup owns a 256 x 256 output tile.  The k loop runs in stages of 32.  Each
// stage's A and WT blocks (256 x 32 fp16 each) go from global memory straight into LDS with
// global_load_lds_dwordx4; D + 1 LDS buffers per operand, D stages in flight.  Two forms: four
// waves of 128 x 128 (default, dense_gemm4_kernel) and eight waves of 128 x 64 (dense_gemm_kernel,
// policy EXL3_AMD_RECON_MM_8WAVES).  Measured on MI355X, 2048 rows, interleaved runs (median
// TFLOPS, four-wave / eight-wave): 28672 -> 8192 1072 / 986, 8192 -> 28672 977 / 932,
// 24576 -> 8192 1043 / 968.  Also measured and not kept: D = 4 (160 KiB of LDS; 1051 / 962 /
// 1034 for the four-wave form) and register staging (global_load_dwordx4 two stages ahead, then
// ds_write_b128; 1080 / 894 / 994).  Workgroups b and b + 8 run on one XCD: the row blocks of one column block
// are consecutive on an XCD, so each 256-column slice of WT is read from HBM once per XCD and
// served to the other row blocks from its L2.
#include "exl3_common.cuh"
#include "exl3_kernels.h"

using namespace exl3;

namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float acc16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int DENSE_T = 512;              // threads per workgroup (8 waves)
constexpr int DENSE_BM = 256;             // rows per workgroup
constexpr int DENSE_BN = 256;             // columns per workgroup
constexpr int DENSE_TILE_U32 = 256 * 16;  // one operand block: 256 rows x 32 fp16
constexpr int DENSE_A0 = 0;
// D stages of DMA in flight, D + 1 LDS buffers per operand: 32 KiB per stage (D = 3: 128 KiB,
// D = 4: 160 KiB); the epilogue reuses 64 KiB
template <int D> struct DenseLds
{
    static constexpr int NB = D + 1;
    static constexpr int B0 = NB * DENSE_TILE_U32;
    static constexpr int U32 = 2 * NB * DENSE_TILE_U32;
    static_assert(U32 >= 64 * DENSE_BN, "the epilogue's 64 x 256 fp32 rows fit the staging buffers");
};

// 16-byte chunk c (0..3) of staged row r: chunk c ^ ((r >> 2) & 3) of the row's 64 bytes, so that
// the 16 lanes of each ds_read_b128 phase (rows r .. r + 15, one chunk) hit 16 distinct 16-byte
// bank groups of the 64-bank LDS.
__device__ __forceinline__ int x_off(int row, int chunk) { return row * 16 + 4 * (chunk ^ ((row >> 2) & 3)); }

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
#define DENSE_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (((n) >> 4) << 14))

// An operand's global layout (rows x k fp16, k-contiguous per row), in fp16 elements: row-major
// (row r at r k; one k stage of 32 is 64 bytes of each row) or k slabs ([k / 32][rows][32]: stage
// c is one contiguous rows x 64-byte slab, so every 1 KiB DMA reads 16 rows' 64 bytes in one
// contiguous kilobyte, 8 whole 128-byte lines, instead of 64 bytes of 16 different lines:
// measured 6 % faster per operand so laid out at 2048 x 8192 x 28672).
struct DenseOperand
{
    size_t row, stage;                                   // element strides of a row and of a k stage
    __device__ DenseOperand(int rows, int k, int slabs)
        : row(slabs ? 32 : (size_t) k), stage(slabs ? (size_t) rows * 32 : 32) { }
    // element offset of 16-byte chunk ch (0..3) of stage 0, row r
    __device__ size_t at(int r, int ch) const { return (size_t) r * row + 8 * ch; }
};

template <int D>
__global__ __launch_bounds__(DENSE_T, 1)
void dense_gemm_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ WT, void* __restrict__ C,
                       const uint16_t* __restrict__ svh, int M, int k, int n, int c_fp32, int a_slabs, int w_slabs,
                       int ldc)
{
    constexpr int MT = 4, NB = DenseLds<D>::NB, DENSE_B0 = DenseLds<D>::B0;
    __shared__ __align__(16) uint32_t lds[DenseLds<D>::U32];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int NST = k / 32;
    const int nbn = (n + DENSE_BN - 1) / DENSE_BN;       // n % 128 == 0: the last block may be half
    const int nmb = (M + DENSE_BM - 1) / DENSE_BM;
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

    // wave w's DMAs j = 0, 1 fill the 1 KiB blocks q = w + 8 j (rows 16 q .. 16 q + 15) of each
    // operand; lane L fills slot L, i.e. row 16 q + L / 4 and the global chunk that x_off puts in
    // slot L % 4.  Rows past M and columns past n read a valid row (results dropped).
    const DenseOperand ao(M, k, a_slabs), bo(n, k, w_slabs);
    const uint16_t* a_src[2];
    const uint16_t* b_src[2];
    #pragma unroll
    for (int j = 0; j < 2; ++j)
    {
        const int q = wave + 8 * j, row = 16 * q + (lane >> 2), ch = (lane & 3) ^ ((row >> 2) & 3);
        a_src[j] = A + ao.at(min(mb * DENSE_BM + row, M - 1), ch);
        b_src[j] = WT + bo.at(min(nb * DENSE_BN + row, n - 1), ch);
    }
    auto issue = [&](int st) {
        const int c = min(st, NST - 1);                  // past the end: rewrites a buffer nobody reads
        const int buf = (st % NB) * DENSE_TILE_U32;
        #pragma unroll
        for (int j = 0; j < 2; ++j)
        {
            __builtin_amdgcn_global_load_lds((const void*) (a_src[j] + c * ao.stage),
                                             (lds_ptr_t) (lds + DENSE_A0 + buf + 256 * (wave + 8 * j)), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const void*) (b_src[j] + c * bo.stage),
                                             (lds_ptr_t) (lds + DENSE_B0 + buf + 256 * (wave + 8 * j)), 16, 0, 0);
        }
    };

    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, lh = lane >> 5;

    #pragma unroll
    for (int g = 0; g < D; ++g) issue(g);
    DENSE_VM_LGKM0(4 * (D - 1));                          // this wave's stage-0 DMAs have landed
    __builtin_amdgcn_s_barrier();

    acc16 acc[MT][2];
    #pragma unroll
    for (int i = 0; i < MT; ++i) { acc[i][0] = (acc16) { }; acc[i][1] = (acc16) { }; }

    for (int s = 0; s < NST; ++s)
    {
        issue(s + D);                                    // its buffers were last read in stage s - 1
        const uint32_t* As = lds + DENSE_A0 + (s % NB) * DENSE_TILE_U32;
        const uint32_t* Bs = lds + DENSE_B0 + (s % NB) * DENSE_TILE_U32;
        h8v av[2][MT], bv[2][2];
        #pragma unroll
        for (int sl = 0; sl < 2; ++sl)
        {
            #pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                bv[sl][nt] = __builtin_bit_cast(h8v, *(const u32x4*) (Bs + x_off(64 * wn + 32 * nt + l32, 2 * sl + lh)));
            #pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                av[sl][mt] = __builtin_bit_cast(h8v, *(const u32x4*) (As + x_off(128 * wm + 32 * mt + l32, 2 * sl + lh)));
        }
        // all 12 operand reads in flight before the first MFMA (they return in order, so the
        // MFMAs of slice 0 wait only for theirs)
        __builtin_amdgcn_sched_barrier(0);
        #pragma unroll
        for (int sl = 0; sl < 2; ++sl)
        {
            #pragma unroll
            for (int mt = 0; mt < MT; ++mt)
            {
                #pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[sl][mt], bv[sl][nt], acc[mt][nt], 0, 0, 0);
            }
        }
        // the next stage's DMAs (issued D - 1 stages ago) have landed for this wave, and its LDS
        // reads of this stage are complete: then the barrier
        DENSE_VM_LGKM0(4 * (D - 1));
        __builtin_amdgcn_s_barrier();
    }
    DENSE_VM_LGKM0(0);                                    // no DMA may still write LDS under the epilogue
    __builtin_amdgcn_s_barrier();

    // epilogue: MT rounds of 64 rows; a row's 256 columns meet in LDS, then each wave stores
    // (rotating, with svh) whole 128-column chunks
    float* E = (float*) lds;                              // [64][256] fp32
    const bool has_svh = svh != nullptr;
    #pragma unroll
    for (int mt = 0; mt < MT; ++mt)
    {
        #pragma unroll
        for (int nt = 0; nt < 2; ++nt)
        {
            #pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                    E[(32 * wm + 8 * j + 4 * lh + i) * DENSE_BN + 64 * wn + 32 * nt + l32] = acc[mt][nt][4 * j + i];
            }
        }
        __syncthreads();
        #pragma unroll 2
        for (int q = 0; q < 16; ++q)
        {
            const int rc = wave * 16 + q;
            const int er = rc >> 1, ch = rc & 1;
            const int row = mb * DENSE_BM + 128 * (er >> 5) + 32 * mt + (er & 31);
            const int col = nb * DENSE_BN + 128 * ch + 2 * lane;
            if (nb * DENSE_BN + 128 * ch >= n) continue;          // half block: chunk past n (uniform per wave)
            const f32x2 v = *(const f32x2*) (E + er * DENSE_BN + 128 * ch + 2 * lane);
            const uint32_t svp = has_svh ? *(const uint32_t*) (svh + col) : 0u;
            if (row < M) gemm_store(v.x, v.y, C, c_fp32, has_svh, svp, (size_t) row * ldc + col, lane);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------
// Four-wave form (default): one wave per SIMD, each wave a 128 x 128 quarter of the 256 x 256 tile
// (4 x 4 accumulators of v_mfma_f32_32x32x16_f16, held in AGPRs).  Per 16-k slice a wave reads 8
// operand blocks for 16 MFMAs (the eight-wave form: 6 for 8), so the LDS serves a third less per
// flop.  With one wave per SIMD the wave hides its own LDS latency: the operand reads of slice
// s + 1 are issued between the MFMAs of slice s (two register sets), and the stage barrier sits
// between the two slices of a stage, so the first slice of stage s + 1 is read while the second
// slice of stage s computes.
constexpr int DENSE4_T = 256;

// Tile body of the four-wave form: WN = columns per wave (128: the 256 x 256 tile; 64: a 256 x 128
// half tile, used for the last partial round of tiles), output tile (mb, nb) of 256 x 2 WN.
//
// k range: stages st0 .. st0 + nst - 1 (of 32 k).  part non-null (split k): the tile's fp32 sums
// go to part (256 x 256, row-major) for the fixup kernel instead of the epilogue's rotation and
// store.
template <int D, int WN, bool BUF>
__device__ __forceinline__ void dense4_tile(uint32_t* lds, const uint16_t* __restrict__ A, const uint16_t* __restrict__ WT,
                                            void* __restrict__ C, const uint16_t* __restrict__ svh, int M, int k, int n,
                                            int c_fp32, int mb, int nb, int a_slabs, int w_slabs, int ldc,
                                            int st0, int nst, float* __restrict__ part)
{
    constexpr int NB = DenseLds<D>::NB, DENSE_B0 = DenseLds<D>::B0;
    constexpr int BN = 2 * WN;
    constexpr int NTN = WN / 32;                         // 32-column MFMA blocks per wave
    constexpr int NT = 4 * NTN;                          // MFMAs per 16-k slice
    constexpr int NR = 4 + NTN;                          // operand reads per slice
    constexpr int NDMA = 4 + NTN;                        // DMAs per stage per wave (A: 4, WT: NTN)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int NST = nst;

    // wave w's DMAs fill the 1 KiB blocks q = w + 4 j (rows 16 q .. 16 q + 15) of each operand:
    // j < 4 for A (256 rows), j < NTN for WT (BN rows)
    const DenseOperand ao(M, k, a_slabs), bo(n, k, w_slabs);
    const uint16_t* a_src[4];
    const uint16_t* b_src[NTN];
    #pragma unroll
    for (int j = 0; j < 4; ++j)
    {
        const int q = wave + 4 * j, row = 16 * q + (lane >> 2), ch = (lane & 3) ^ ((row >> 2) & 3);
        a_src[j] = A + ao.at(min(mb * DENSE_BM + row, M - 1), ch);
        if (j < NTN) b_src[j] = WT + bo.at(min(nb * BN + row, n - 1), ch);
    }
    // BUF: the DMAs go through buffer resources over A and WT (operands below 4 GiB, checked on
    // the host): a 32-bit lane offset fixed per DMA slot and the stage's byte offset in an SGPR,
    // so that no VALU address arithmetic sits between the MFMAs (measured 1-2 % faster than
    // global_load_lds with 64-bit lane addresses)
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*) A, (short) 0, (int) (uint32_t) ((size_t) M * k * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*) WT, (short) 0, (int) (uint32_t) ((size_t) n * k * 2), 0x00020000);
    uint32_t a_off[4], b_off[NTN];
    if constexpr (BUF)
    {
        #pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            a_off[j] = (uint32_t) (2 * (a_src[j] - A));
            if (j < NTN) b_off[j] = (uint32_t) (2 * (b_src[j] - WT));
        }
    }
    // DMA q of a stage: A and WT blocks alternate while both last, then the rest of A
    auto issue_one = [&](int st, int q) {
        const int c = st0 + min(st, NST - 1);            // past the end: rewrites a buffer nobody reads
        const int buf = (st % NB) * DENSE_TILE_U32;
        const bool isb = q < 2 * NTN && (q & 1);
        const int j = q < 2 * NTN ? q >> 1 : q - NTN;
        if constexpr (BUF)
        {
            if (isb)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t) (lds + DENSE_B0 + buf + 256 * (wave + 4 * j)), 16,
                                                         b_off[j], (uint32_t) (2 * c * bo.stage), 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t) (lds + DENSE_A0 + buf + 256 * (wave + 4 * j)), 16,
                                                         a_off[j], (uint32_t) (2 * c * ao.stage), 0, 0);
            return;
        }
        if (isb)
            __builtin_amdgcn_global_load_lds((const void*) (b_src[j] + c * bo.stage),
                                             (lds_ptr_t) (lds + DENSE_B0 + buf + 256 * (wave + 4 * j)), 16, 0, 0);
        else
            __builtin_amdgcn_global_load_lds((const void*) (a_src[j] + c * ao.stage),
                                             (lds_ptr_t) (lds + DENSE_A0 + buf + 256 * (wave + 4 * j)), 16, 0, 0);
    };

    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, lh = lane >> 5;
    #pragma unroll
    for (int g = 0; g < D; ++g)
        #pragma unroll
        for (int q = 0; q < NDMA; ++q) issue_one(g, q);
    DENSE_VM_LGKM0(NDMA * (D - 1));
    __builtin_amdgcn_s_barrier();

    acc16 acc[4][NTN];
    #pragma unroll
    for (int i = 0; i < 4; ++i)
        #pragma unroll
        for (int j = 0; j < NTN; ++j) acc[i][j] = (acc16) { };

    // The loop body is written out in issue order, fenced by sched_barrier: the NR operand reads of
    // the next slice are spread over the NT MFMAs of a slice (read r after MFMA r NT / NR), and
    // half of stage s + D's NDMA LDS DMAs sit in each slice, one every NT / (NDMA / 2) MFMAs, so
    // that no burst of memory instructions holds up the matrix pipe (a wave whose VMEM issue
    // stalls cannot issue MFMAs meanwhile; without the DMAs the loop runs ~1.5x faster, and DMAs
    // of a quarter the size are no cheaper: the cost is per instruction).  Reads are issued in the
    // order the MFMAs consume them (a[0], b[0..NTN-1], a[1..3]), so each MFMA waits only for its
    // own operands.
    h8v a0[4], b0[NTN], a1[4], b1[NTN];
    auto read_one = [&](int st, int sl, int q, h8v* av, h8v* bv) {
        const uint32_t* As = lds + DENSE_A0 + (st % NB) * DENSE_TILE_U32;
        const uint32_t* Bs = lds + DENSE_B0 + (st % NB) * DENSE_TILE_U32;
        if (q == 0) av[0] = __builtin_bit_cast(h8v, *(const u32x4*) (As + x_off(128 * wm + l32, 2 * sl + lh)));
        else if (q <= NTN) bv[q - 1] = __builtin_bit_cast(h8v, *(const u32x4*) (Bs + x_off(WN * wn + 32 * (q - 1) + l32, 2 * sl + lh)));
        else av[q - NTN] = __builtin_bit_cast(h8v, *(const u32x4*) (As + x_off(128 * wm + 32 * (q - NTN) + l32, 2 * sl + lh)));
    };
    #pragma unroll
    for (int q = 0; q < NR; ++q) read_one(0, 0, q, a0, b0);
    for (int s = 0; s < NST; ++s)
    {
        // first slice: after MFMA t, events [t E / NT, (t + 1) E / NT) of the interleaved list
        // read 0, DMA 0, read 1, DMA 1, ... (E = NR + NDMA)
        #pragma unroll
        for (int t = 0; t < NT; ++t)
        {
            acc[t / NTN][t % NTN] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0[t / NTN], b0[t % NTN], acc[t / NTN][t % NTN], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            #pragma unroll
            for (int r = 0; r < NR; ++r)
                if (r * NT / NR == t) read_one(s, 1, r, a1, b1);
            #pragma unroll
            for (int i = 0; i < NDMA / 2; ++i)
                if ((i + 1) * NT / (NDMA / 2) - 1 == t) issue_one(s + D, i);
            __builtin_amdgcn_sched_barrier(0);
        }
        // stage s + 1 landed for this wave (stages s + 2 .. s + D - 1 and the first half of
        // s + D may be in flight), its own reads of stage s are complete: barrier, after which
        // every wave's reads of stage s are complete too (its buffer is refilled from the next
        // stage's first DMA on)
        DENSE_VM_LGKM0(NDMA * (D - 2) + NDMA / 2);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // slice 0 of stage s + 1 read under the MFMAs of slice 1 (past the end: an unread buffer)
        #pragma unroll
        for (int t = 0; t < NT; ++t)
        {
            acc[t / NTN][t % NTN] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[t / NTN], b1[t % NTN], acc[t / NTN][t % NTN], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            #pragma unroll
            for (int r = 0; r < NR; ++r)
                if (r * NT / NR == t) read_one(s + 1, 0, r, a0, b0);
            #pragma unroll
            for (int i = 0; i < NDMA / 2; ++i)
                if ((i + 1) * NT / (NDMA / 2) - 1 == t) issue_one(s + D, NDMA / 2 + i);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    DENSE_VM_LGKM0(0);
    __builtin_amdgcn_s_barrier();

    // epilogue: 4 rounds; round r holds rows 128 wm + 32 r + (0..31) of each wave in E[64][BN]
    constexpr int NCH = BN / 128;                        // 128-column chunks per row
    float* E = (float*) lds;
    const bool has_svh = svh != nullptr;
    #pragma unroll
    for (int r = 0; r < 4; ++r)
    {
        #pragma unroll
        for (int j = 0; j < NTN; ++j)
        {
            #pragma unroll
            for (int jj = 0; jj < 4; ++jj)
            {
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                    E[(32 * wm + 8 * jj + 4 * lh + i) * BN + WN * wn + 32 * j + l32] = acc[r][j][4 * jj + i];
            }
        }
        __syncthreads();
        #pragma unroll 2
        for (int q = 0; q < 16 * NCH; ++q)
        {
            const int rc = wave * 16 * NCH + q;
            const int er = rc / NCH, ch = rc % NCH;
            const int row = mb * DENSE_BM + 128 * (er >> 5) + 32 * r + (er & 31);
            const int col = nb * BN + 128 * ch + 2 * lane;
            if (nb * BN + 128 * ch >= n) continue;       // half block: chunk past n (uniform per wave)
            const f32x2 v = *(const f32x2*) (E + er * BN + 128 * ch + 2 * lane);
            if (part)
            {
                // rows past M are neither stored nor read by the fixup
                if (row < M) *(f32x2*) (part + (size_t) (row - mb * DENSE_BM) * DENSE_BN + 128 * ch + 2 * lane) = v;
                continue;
            }
            const uint32_t svp = has_svh ? *(const uint32_t*) (svh + col) : 0u;
            if (row < M) gemm_store(v.x, v.y, C, c_fp32, has_svh, svp, (size_t) row * ldc + col, lane);
        }
        __syncthreads();
    }
}

// Four-wave form (default): one wave per SIMD, each wave a 128 x 128 quarter of the 256 x 256 tile
// (4 x 4 accumulators of v_mfma_f32_32x32x16_f16, held in AGPRs).  Per 16-k slice a wave reads 8
// operand blocks for 16 MFMAs (the eight-wave form: 6 for 8), so the LDS serves a third less per
// flop.  With one wave per SIMD the wave hides its own LDS latency: the operand reads of slice
// s + 1 are issued between the MFMAs of slice s (two register sets), and the stage barrier sits
// between the two slices of a stage, so the first slice of stage s + 1 is read while the second
// slice of stage s computes.
//
// Grid: full tiles first (column blocks 0 .. nfull - 1 of 256), then, when the tiles would leave
// a last round less than half full, the remaining column blocks as 256 x 128 half tiles (2 per
// block).  The dispatcher hands the half tiles to the CUs as they finish their last full tile, so
// the partial round takes about half a tile's time instead of a whole one (8192 -> 28672 at 2048
// rows: 896 tiles = 3.5 rounds on 256 CUs).
template <int D, bool BUF>
__global__ __launch_bounds__(DENSE4_T, 1)
void dense_gemm4_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ WT, void* __restrict__ C,
                        const uint16_t* __restrict__ svh, int M, int k, int n, int c_fp32, int nfull,
                        int a_slabs, int w_slabs, int ldc, int splits, float* __restrict__ part)
{
    __shared__ __align__(16) uint32_t lds[DenseLds<D>::U32];
    const int nmb = (M + DENSE_BM - 1) / DENSE_BM;
    // tile -> (nb, mb): with a multiple of 8 column blocks, the 8 consecutive workgroups that
    // share an XCD take one column block's row blocks in turn
    auto map = [&](int b, int nbn, int& nb, int& mb) {
        if (nbn % 8 == 0)
        {
            const int x = b % 8, r = b / 8;
            nb = x + 8 * (r / nmb);
            mb = r % nmb;
        }
        else
        {
            nb = b / nmb;
            mb = b % nmb;
        }
    };
    const int b = blockIdx.x;
    const int NST = k / 32;
    int nb, mb;
    if (splits > 1)
    {
        // split k: workgroups S t .. S t + S - 1 take the S k ranges of tile t
        const int t = b / splits, h = b % splits;
        nb = t / nmb;
        mb = t % nmb;
        const int s0 = h * NST / splits, s1 = (h + 1) * NST / splits;
        dense4_tile<D, 128, BUF>(lds, A, WT, C, svh, M, k, n, c_fp32, mb, nb, a_slabs, w_slabs, ldc, s0, s1 - s0,
                                 part + (size_t) b * DENSE_BM * DENSE_BN);
    }
    else if (b < nfull * nmb)
    {
        map(b, nfull, nb, mb);
        dense4_tile<D, 128, BUF>(lds, A, WT, C, svh, M, k, n, c_fp32, mb, nb, a_slabs, w_slabs, ldc, 0, NST, nullptr);
    }
    else
    {
        const int nbn = (n + DENSE_BN - 1) / DENSE_BN;
        map(b - nfull * nmb, 2 * (nbn - nfull), nb, mb);
        dense4_tile<D, 64, BUF>(lds, A, WT, C, svh, M, k, n, c_fp32, mb, nb + 2 * nfull, a_slabs, w_slabs, ldc, 0, NST,
                                nullptr);
    }
}

// Split-k fixup (this GEMM and the fused trellis GEMM, exl3_gemm.hip, whose tiles are also 256 x
// 256 with tile t = (column block t / nmb, row block t % nmb)): tile t's S fp32 partial sums,
// part[(t S + h) 256 x 256], added in k order (h = 0 .. S - 1), then the epilogue's rotation and
// store.  One wave per (row, 128-column chunk) of a tile.
__global__ __launch_bounds__(256)
void dense_split_fixup(const float* __restrict__ part, void* __restrict__ C, const uint16_t* __restrict__ svh, int M,
                       int n, int ldc, int c_fp32, int nmb, int tiles, int splits)
{
    const int lane = threadIdx.x & 63;
    const long job = (long) blockIdx.x * 4 + (threadIdx.x >> 6);  // (tile, row, chunk)
    if (job >= (long) tiles * DENSE_BM * 2) return;
    const int t = (int) (job / (DENSE_BM * 2)), rc = (int) (job % (DENSE_BM * 2));
    const int r = rc >> 1, ch = rc & 1;
    const int nb = t / nmb, mb = t % nmb;
    const int row = mb * DENSE_BM + r, c0 = nb * DENSE_BN + 128 * ch;
    if (row >= M || c0 >= n) return;
    const float* p = part + (size_t) t * splits * DENSE_BM * DENSE_BN + (size_t) r * DENSE_BN + 128 * ch + 2 * lane;
    float v0 = 0.0f, v1 = 0.0f;
    for (int h = 0; h < splits; ++h)
    {
        const f32x2 a = __builtin_nontemporal_load((const f32x2*) (p + (size_t) h * DENSE_BM * DENSE_BN));
        v0 += a.x;
        v1 += a.y;
    }
    const bool has_svh = svh != nullptr;
    const uint32_t svp = has_svh ? *(const uint32_t*) (svh + c0 + 2 * lane) : 0u;
    gemm_store(v0, v1, C, c_fp32, has_svh, svp, (size_t) row * ldc + c0 + 2 * lane, lane);
}

}  // namespace

int exl3k_dense_gemm(const uint16_t* A, const uint16_t* WT, void* C, int c_fp32, const uint16_t* svh,
                     int m, int k, int n, int a_slabs, int w_slabs, int ldc, int variant, int cus,
                     float* part, size_t part_bytes, hipStream_t s)
{
    const int nbn = (n + DENSE_BN - 1) / DENSE_BN, nmb = (m + DENSE_BM - 1) / DENSE_BM;
    const int blocks = nbn * nmb;
    if (variant == 1)
    {
        hipLaunchKernelGGL((dense_gemm_kernel<3>), dim3(blocks), dim3(DENSE_T), 0, s, A, WT, C, svh, m, k, n, c_fp32,
                           a_slabs, w_slabs, ldc);
        return (int) hipGetLastError();
    }
    // split k when the tiles fill at most half the CUs: S = as many k ranges as keep every CU
    // busy, at least 4 stages of 32 k each, and the S fp32 partial tiles within `part`
    int splits = 1;
    if (variant != 5 && part && cus > 0 && 2 * blocks <= cus)
    {
        const long tile_bytes = (long) DENSE_BM * DENSE_BN * sizeof(float);
        splits = min(cus / blocks, (k / 32) / 4);
        splits = (int) min((long) splits, (long) (part_bytes / (tile_bytes * blocks)));
        if (splits < 2) splits = 1;
    }
    // half tiles for a last round at most half full: whole column blocks (n a multiple of 256),
    // at least one full round before it
    const int rem = cus > 0 ? blocks % cus : 0;
    int nfull = nbn;
    if (splits == 1 && variant != 2 && n % DENSE_BN == 0 && blocks > cus && rem > 0 && 2 * rem <= cus && rem % nmb == 0)
        nfull = nbn - rem / nmb;
    const int grid = splits > 1 ? blocks * splits : nfull * nmb + 2 * (nbn - nfull) * nmb;
    float* sp = splits > 1 ? part : nullptr;
    // buffer-resource DMAs for operands below 4 GiB (32-bit offsets and record counts)
    // (variant 3 forces the 64-bit-address form, for tests)
    const bool buf = variant != 3 && (size_t) m * k * 2 < (1ull << 32) && (size_t) n * k * 2 < (1ull << 32);
    if (buf)
        hipLaunchKernelGGL((dense_gemm4_kernel<3, true>), dim3(grid), dim3(DENSE4_T), 0, s, A, WT, C, svh, m, k, n, c_fp32, nfull,
                           a_slabs, w_slabs, ldc, splits, sp);
    else
        hipLaunchKernelGGL((dense_gemm4_kernel<3, false>), dim3(grid), dim3(DENSE4_T), 0, s, A, WT, C, svh, m, k, n, c_fp32, nfull,
                           a_slabs, w_slabs, ldc, splits, sp);
    if (splits > 1) return exl3k_split_fixup(part, C, svh, m, n, ldc, c_fp32, nmb, blocks, splits, s);
    return (int) hipGetLastError();
}

int exl3k_split_fixup(const float* part, void* C, const uint16_t* svh, int m, int n, int ldc, int c_fp32, int nmb,
                      int tiles, int splits, hipStream_t s)
{
    const long jobs = (long) tiles * DENSE_BM * 2;
    hipLaunchKernelGGL(dense_split_fixup, dim3((unsigned) ((jobs + 3) / 4)), dim3(256), 0, s, part, C, svh, m, n, ldc,
                       c_fp32, nmb, tiles, splits);
    return (int) hipGetLastError();
}
