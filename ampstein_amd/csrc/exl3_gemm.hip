// Prefill-shaped EXL3 GEMM for gfx950 (m > 8): C = had(A_had @ W_hat) o svh with fp16 MFMA
// and fp32 accumulation.  Semantics of exl3_gemm_kernel / exl3_gemm_kernel_inner
// (quant/exl3_gemm_kernel.cuh:8-84, quant/exl3_gemm_inner.cuh:31-1009): the output Hadamard
// reads the fp32 sums (had_fh / had_ff, hadamard_inner.cuh:154-281); the input rotation A_had =
// had_hf(A o suh) is written by the caller-side pre-pass (exl3k_had128).
//
// Tiling.  A workgroup (8 waves, 2 per SIMD) owns a 256 x 256 output tile; wave (wm, wn) the
// 128 rows [128 wm, +128) x 64 columns [64 wn, +64): 4 x 2 v_mfma_f32_32x32x16_f16
// accumulators.  The k loop runs in stages of 32 (two 16-row trellis slices).  Per stage the
// workgroup stages the A block (256 x 32 fp16, coalesced 16-byte loads, register prefetch PF
// stages ahead) and the stage's 2 x 16 trellis tiles in LDS, and decodes every weight of the
// 32 x 256 B block ONCE into LDS (fp16, MFMA-operand order).  Decode of stage s + 1 runs in
// the same iteration as the MFMAs of stage s; one barrier per stage.
//
// Decode.  Thread (column c of the block, half h) produces the 8 weights of rows 8h..8h+7 of
// column c of one trellis tile, i.e. tile positions 32(c%8) + 4(c/8) + 2h + {0,1,8,9,16,17,
// 24,25} (make_tc_perm, cpu/moe_mul1.cpp:124-139): a 26-position run of the tile's bit ring.
// The run is normalised to bit 0 with one alignbit per word, then the 8 windows sit at
// compile-time offsets.  Weights are the reference's fp16 values exactly: 3INST / MCG lo + hi
// rounded by one v_pk_add_f16 per pair, MUL1 by one v_pk_fma_f16 (codebook.cuh:57-90).
//
// LDS layouts are XOR-swizzled for the bank rules measured on MI355X: a ds_read_b128 serves 16
// lanes at a time over 64 banks, a ds_write_b128 8 lanes at a time over 32 banks.  The trellis
// words are staged with one 16-byte store per staging thread.
//
// Compiled once per K (EXL3_INST_K).
#include <cstdlib>
#include <cstring>

#include "exl3_common.cuh"
#include "exl3_gemv_core.cuh"
#include "exl3_kernels.h"

#ifndef EXL3_INST_K
#define EXL3_INST_K 4
#endif

using namespace exl3;

namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float acc16 __attribute__((ext_vector_type(16)));

constexpr int GT = 512;          // threads per workgroup (8 waves)
constexpr int BM = 256;          // rows per workgroup
constexpr int BN = 256;          // columns per workgroup
constexpr int PF = 3;            // register prefetch depth, stages (32 k each)

// Rate code K (exl3_common.cuh kbits / khalf): 1..8, or 16 + b for b + 1/2 (mul1).  The window of
// tile position t ends at ring bit tile_end(t): (t + 1) K for integer rates; for b + 1/2 the
// positions alternate b and b + 1 bits (exl3_dq.cuh:254-285, cpu/moe_mul1.cpp:78-83).
template <int K>
__host__ __device__ constexpr int tile_end(int t)
{
    return khalf(K) ? (t >> 1) * (2 * kbits(K) + 1) + ((t & 1) ? 2 * kbits(K) + 1 : kbits(K)) : (t + 1) * K;
}
// Offset of position t0 + d's window from position t0's (t0 even: the decode runs start there).
template <int K>
__host__ __device__ constexpr int run_rel(int d) { return tile_end<K>(d) - tile_end<K>(0); }
// Words of a normalised run: the 26 positions t0 .. t0 + 25 plus the 16-bit window of t0.
template <int K>
__host__ __device__ constexpr int run_words() { return (run_rel<K>(25) + 16 + 31) / 32; }

template <int K, int RB> struct GemmLds
{
    // words per staged tile: the tile's words, padded to a multiple of 4 so that each staging
    // thread writes its 4 words with one ds_write_b128 (a tile always holds a multiple of 4 words).
    // The padding at 8 and 2.5 bits spreads the decode's word reads over more LDS banks (the
    // fewest bank conflicts among multiple-of-4 strides, measured on MI355X).
    static constexpr int TW = tile_words(K) + ((K == 8 || K == 18) ? 4 : 0);
    static constexpr int A_U32 = RB * 16;                // A block: RB rows x 32 fp16
    static constexpr int B_U32 = 2 * BN * 8;             // B block: 2 slices x 256 columns x 16 fp16
    static constexpr int T_U32 = 2 * 16 * TW;            // 2 slices x 16 tiles
    static constexpr int A0 = 0;
    static constexpr int B0 = 2 * A_U32;
    static constexpr int T0 = B0 + 2 * B_U32;
    static constexpr int DUMMY = T0 + 2 * T_U32 + 4;     // (+4: a run may read one word past the last tile)
    // (at least the epilogue's 64 x 256 fp32)
    static constexpr int TOTAL = DUMMY > 64 * BN ? DUMMY : 64 * BN;
};

// 16-bit window at MSB-first bit offset REL of a normalised word run.
template <int REL>
__device__ __forceinline__ uint32_t win16(const uint32_t* nw)
{
    constexpr int w = REL / 32, off = REL % 32;
    if constexpr (off <= 16) return __builtin_amdgcn_ubfe(nw[w], 16 - off, 16);
    else return __builtin_amdgcn_alignbit(nw[w], nw[w + 1], 48 - off) & 0xffffu;
}

// 3INST multiply-add as one v_mad_u64_u32 (its low word): ~full rate on gfx950, where mul + add
// would take two ops.
__device__ __forceinline__ uint32_t mad_3inst(uint32_t s)
{
    uint64_t r;
    asm("v_mad_u64_u32 %0, vcc, %1, %2, %3" : "=&v"(r) : "v"(s), "s"(89226354u), "v"((uint64_t) 64248484u) : "vcc");
    return (uint32_t) r;
}

template <int CB>
__device__ __forceinline__ uint32_t cb_raw(uint32_t s)
{
    if constexpr (CB == 0) return (mad_3inst(s) & 0x8fff8fffu) ^ 0x3b603b60u;                   // codebook.cuh:61-63
    else if constexpr (CB == 1) return ((s * 0xCBAC1FEDu) & 0x8fff8fffu) ^ 0x3b603b60u;        // codebook.cuh:69-72
    else return __builtin_amdgcn_sad_u8(s * 0x83DCD12Du, 0u, 0x6400u);                        // codebook.cuh:78-84
}

// Two decoded weights (rows i, i + 1) packed as one fp16 pair.
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

// Weights of rows 8h..8h+7 of one column from its normalised 26-position run: words tl[0..NW],
// with tl[0] read from t0 instead (the tile's last word when the run starts in the ring word -1).
template <int K, int CB>
__device__ __forceinline__ u32x4 decode_run(const uint32_t* __restrict__ tl, const uint32_t* __restrict__ t0, int sh)
{
    constexpr int NW = run_words<K>();
    uint32_t rw[NW + 1], nw[NW + 1];
    rw[0] = *t0;
    #pragma unroll
    for (int i = 1; i <= NW; ++i) rw[i] = tl[i];
    #pragma unroll
    for (int i = 0; i < NW; ++i) nw[i] = __builtin_amdgcn_alignbit(rw[i], rw[i + 1], 32 - sh);
    nw[NW] = 0u;
    uint32_t r[8];
    r[0] = cb_raw<CB>(win16<run_rel<K>(0)>(nw));
    r[1] = cb_raw<CB>(win16<run_rel<K>(1)>(nw));
    r[2] = cb_raw<CB>(win16<run_rel<K>(8)>(nw));
    r[3] = cb_raw<CB>(win16<run_rel<K>(9)>(nw));
    r[4] = cb_raw<CB>(win16<run_rel<K>(16)>(nw));
    r[5] = cb_raw<CB>(win16<run_rel<K>(17)>(nw));
    r[6] = cb_raw<CB>(win16<run_rel<K>(24)>(nw));
    r[7] = cb_raw<CB>(win16<run_rel<K>(25)>(nw));
    return (u32x4) { weight_pair<CB>(r[0], r[1]), weight_pair<CB>(r[2], r[3]),
                     weight_pair<CB>(r[4], r[5]), weight_pair<CB>(r[6], r[7]) };
}

// Swizzled LDS offsets (u32 units).  A: row stride 16 u32 (4 chunks of 16 B), chunk ^= (row >> 2) & 3
// (gfx950 LDS: 64 banks; the 16 lanes of a ds_read_b128 phase touch 16 distinct 16-byte groups).
// B: per slice, column stride 8 u32 (2 chunks), chunk ^= ((col >> 2) ^ (col >> 3)) & 1.  The
// decode's ds_write_b128 is served 8 lanes (8 consecutive columns) at a time over 32 banks, so
// columns c and c + 4 must take different chunks; the MFMA reads (16 lanes over 64 banks) need
// columns c and c + 8 to differ, which the (col >> 3) term keeps.
__device__ __forceinline__ int a_off(int row, int chunk) { return row * 16 + 4 * (chunk ^ ((row >> 2) & 3)); }
__device__ __forceinline__ int b_off(int slice, int col, int h) { return slice * (BN * 8) + col * 8 + 4 * (h ^ (((col >> 2) ^ (col >> 3)) & 1)); }

template <int K, int CB, bool GROUP, int RB>
__global__ __launch_bounds__(GT, 1)
void gemm_kernel(const uint16_t* __restrict__ Ain, const uint16_t* __restrict__ trellis, void* __restrict__ C,
                 const uint16_t* __restrict__ svh, int M, int k, int n, int c_fp32, GemmGroupArgs grp)
{
    using LD = GemmLds<K, RB>;
    constexpr int MT = RB / 64;                          // 32-row MFMA tiles per wave (2 waves along m)
    constexpr int AJ = RB >= 256 ? 2 : 1;                // A chunks staged per thread
    __shared__ __align__(16) uint32_t lds[LD::TOTAL];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = threadIdx.x;
    const int NST = k / 32;                              // stages
    const int nbn = (n + BN - 1) / BN;                   // n % 128 == 0: a last block may be half

    // workgroup -> (column block, row block): the row blocks of one column block run together on
    // one XCD (workgroups b and b + 8 on one XCD) when the block count allows, sharing its trellis in L2
    int nb, mb;
    if constexpr (GROUP)
    {
        // grouped launch: one row tile of one expert per workgroup (uniform early exit past the
        // list: no barrier has been reached)
        nb = blockIdx.x % nbn;
        const int t2 = blockIdx.x / nbn;
        const int mat = t2 % grp.mats, li = t2 / grp.mats;
        if (li >= *(mat ? grp.count[1] : grp.count[0])) return;
        const int tid = (mat ? grp.list[1] : grp.list[0])[li];
        const int e = grp.rt[3 * tid], row0 = grp.rt[3 * tid + 1];
        M = grp.rt[3 * tid + 2];
        Ain = (mat ? grp.A[1] : grp.A[0]) + (size_t) row0 * k;
        C = (mat ? grp.C[1] : grp.C[0]) + (size_t) row0 * n;
        trellis = (const uint16_t*) (mat ? grp.tab[1] : grp.tab[0])[e];
        svh = nullptr;
        c_fp32 = 0;
        mb = 0;
    }
    const int nmb = (M + RB - 1) / RB;
    if constexpr (GROUP) { }           // (nb, mb) from the row tile above
    else if (nbn % 8 == 0)
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

    // ---- A staging: chunks u = t, t + 512 (row u / 4, 16-byte chunk u % 4 of the row's 64 bytes)
    // (RB = 64: threads t and t + 256 stage the same chunk, an identical duplicate store)
    int a_lds[2];
    const u32x4* a_src[2];
    #pragma unroll
    for (int j = 0; j < 2; ++j)
    {
        const int u = (t + GT * (j % AJ)) % (RB * 4), row = u >> 2, ch = u & 3;
        a_lds[j] = LD::A0 + a_off(row, ch);
        a_src[j] = (const u32x4*) (Ain + (size_t) min(mb * RB + row, M - 1) * k + 8 * ch);
    }
    // ---- trellis staging: words 4t..4t+3 of the stage's 2 slices x 16 tiles (t < 64K)
    constexpr int TWD = tile_words(K);                   // u32 per tile
    const bool tload = t < 8 * TWD;
    int t_lds;
    const uint32_t* t_src;
    {
        const int wi = 4 * (tload ? t : 0);
        const int s2 = wi / (16 * TWD), wj = wi - s2 * (16 * TWD);
        const int tile = wj / TWD, wk = wj - tile * TWD;
        t_lds = LD::T0 + (s2 * 16 + tile) * LD::TW + wk;    // 16-byte aligned: TW, wk and T0 are multiples of 4
        const int gtile = min(nb * 16 + tile, n / 16 - 1);   // columns past n: a valid tile, results dropped
        t_src = (const uint32_t*) trellis + ((size_t) s2 * (n / 16) + gtile) * TWD + wk;
    }
    const size_t t_stage = (size_t) 2 * (n / 16) * TWD;        // u32 per stage (two tile rows)

    // ---- decode assignment: column dc of the block, half dh; both slices of a stage
    const int dc = t & 255, dh = t >> 8;
    const int dtile = dc >> 4, dcc = dc & 15;
    const int dbase = 32 * (dcc & 7) + 4 * (dcc >> 3) + 2 * dh;
    const int dB0 = tile_end<K>(dbase) - 16;             // first window's first bit (< 0: ring)
    const int df = dB0 - 1 >= 0 ? (dB0 - 1) / 32 : -1;
    const int dsh = dB0 - 32 * df;                       // 1..32
    const int d_src = LD::T0 + dtile * LD::TW + df;      // + slice * 16 * TW; word df + i, i >= 1
    const int d_ring = LD::T0 + dtile * LD::TW + (df < 0 ? TWD - 1 : df);   // word df (-1: the tile's last)
    const int d_dst0 = LD::B0 + b_off(0, dc, dh), d_dst1 = LD::B0 + b_off(1, dc, dh);

    // ---- MFMA operand assignment
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, lh = lane >> 5;

    u32x4 apf[PF][2], tpf[PF];
    auto load_stage = [&](int s, u32x4* a, u32x4& tw) {
        const int sc = min(s, NST - 1);
        // the activation tile is re-read by every column block: cached loads (it stays in L2 /
        // the MALL between blocks); the trellis words are read once per row block: nontemporal
        a[0] = *(a_src[0] + 4 * sc);
        if constexpr (AJ == 2) a[1] = *(a_src[1] + 4 * sc);
        tw = __builtin_nontemporal_load((const u32x4*) (t_src + sc * t_stage));
    };
    auto store_stage = [&](int buf, const u32x4* a, const u32x4& tw) {
        *(u32x4*) (lds + buf * LD::A_U32 + a_lds[0]) = a[0];
        if constexpr (AJ == 2) *(u32x4*) (lds + buf * LD::A_U32 + a_lds[1]) = a[1];
    };
    auto store_trellis = [&](int buf, const u32x4& tw) {
        if (tload) *(u32x4*) (lds + buf * LD::T_U32 + t_lds) = tw;
    };
    auto decode_slice = [&](int buf, int sl) {
        const uint32_t* T = lds + buf * LD::T_U32;
        uint32_t* B = lds + buf * LD::B_U32;
        *(u32x4*) (B + (sl ? d_dst1 : d_dst0)) = decode_run<K, CB>(T + d_src + sl * 16 * LD::TW, T + d_ring + sl * 16 * LD::TW, dsh);
    };
    auto decode_stage = [&](int buf) { decode_slice(buf, 0); decode_slice(buf, 1); };

    // prologue: A(0), trellis(0), trellis(1) staged; B(0) decoded
    #pragma unroll
    for (int d = 0; d < PF; ++d) load_stage(d, apf[d], tpf[d]);
    store_stage(0, apf[0], tpf[0]);
    store_trellis(0, tpf[0]);
    store_trellis(1, tpf[1]);
    __syncthreads();
    decode_stage(0);
    // slot 0 now free: A(PF) / trellis(PF); A(1) still waits in slot 1, trellis(2) in slot 2
    load_stage(PF, apf[0], tpf[0]);
    __syncthreads();

    acc16 acc[MT][2];
    #pragma unroll
    for (int i = 0; i < MT; ++i) { acc[i][0] = (acc16) { }; acc[i][1] = (acc16) { }; }

    for (int s0 = 0; s0 < NST; s0 += PF)
    {
        #pragma unroll
        for (int d = 0; d < PF; ++d)
        {
            const int s = s0 + d;
            if (s >= NST) break;
            const int cur = s & 1, nxt = cur ^ 1;
            // per slice: load this stage's MFMA operands from LDS, then decode the same slice of
            // B(s + 1) from trellis(s + 1) (staged last iteration; past the last stage it decodes
            // stale words into a buffer nobody reads, keeping the body one basic block) while the
            // slice's 8 MFMAs run on the operands already in registers
            const uint32_t* A = lds + LD::A0 + cur * LD::A_U32;
            const uint32_t* B = lds + LD::B0 + cur * LD::B_U32;
            #pragma unroll
            for (int sl = 0; sl < 2; ++sl)
            {
                h8v bv[2], av[MT];
                #pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    bv[nt] = __builtin_bit_cast(h8v, *(const u32x4*) (B + b_off(sl, 64 * wn + 32 * nt + l32, lh)));
                #pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    av[mt] = __builtin_bit_cast(h8v, *(const u32x4*) (A + a_off((RB / 2) * wm + 32 * mt + l32, 2 * sl + lh)));
                // the decode of this slice of B(s + 1), cut into 8 pieces that ride in the shadow
                // of the 8 MFMAs (each 32 cycles on the matrix pipe); sched_barrier keeps the cuts
                constexpr int NW = run_words<K>();
                const uint32_t* tl = lds + nxt * LD::T_U32 + d_src + sl * 16 * LD::TW;
                uint32_t rw[NW + 1], nw[NW + 1], r[8], wp[4];
                rw[0] = lds[nxt * LD::T_U32 + d_ring + sl * 16 * LD::TW];
                #pragma unroll
                for (int i = 1; i <= NW; ++i) rw[i] = tl[i];
#define EXL3_MFMA_STEP(mt, nt) \
                __builtin_amdgcn_sched_barrier(0); \
                if constexpr ((mt) < MT) \
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bv[nt], acc[mt][nt], 0, 0, 0); \
                __builtin_amdgcn_sched_barrier(0);
                EXL3_MFMA_STEP(0, 0)
                #pragma unroll
                for (int i = 0; i < NW; ++i) nw[i] = __builtin_amdgcn_alignbit(rw[i], rw[i + 1], 32 - dsh);
                nw[NW] = 0u;
                EXL3_MFMA_STEP(0, 1)
                r[0] = cb_raw<CB>(win16<run_rel<K>(0)>(nw));
                r[1] = cb_raw<CB>(win16<run_rel<K>(1)>(nw));
                EXL3_MFMA_STEP(1, 0)
                r[2] = cb_raw<CB>(win16<run_rel<K>(8)>(nw));
                r[3] = cb_raw<CB>(win16<run_rel<K>(9)>(nw));
                EXL3_MFMA_STEP(1, 1)
                wp[0] = weight_pair<CB>(r[0], r[1]);
                wp[1] = weight_pair<CB>(r[2], r[3]);
                EXL3_MFMA_STEP(2, 0)
                r[4] = cb_raw<CB>(win16<run_rel<K>(16)>(nw));
                r[5] = cb_raw<CB>(win16<run_rel<K>(17)>(nw));
                EXL3_MFMA_STEP(2, 1)
                r[6] = cb_raw<CB>(win16<run_rel<K>(24)>(nw));
                r[7] = cb_raw<CB>(win16<run_rel<K>(25)>(nw));
                EXL3_MFMA_STEP(3, 0)
                wp[2] = weight_pair<CB>(r[4], r[5]);
                wp[3] = weight_pair<CB>(r[6], r[7]);
                EXL3_MFMA_STEP(3, 1)
#undef EXL3_MFMA_STEP
                *(u32x4*) (lds + nxt * LD::B_U32 + (sl ? d_dst1 : d_dst0)) = (u32x4) { wp[0], wp[1], wp[2], wp[3] };
            }
            // stage A(s + 1) and trellis(s + 2) (clamped loads: past the end they rewrite unread
            // buffers); prefetch further
            const int n1 = (d + 1) % PF, n2 = (d + 2) % PF;
            store_stage(nxt, apf[n1], tpf[n1]);
            store_trellis(cur, tpf[n2]);
            load_stage(s + 1 + PF, apf[n1], tpf[n1]);

            __syncthreads();
        }
    }

    // ---- epilogue: MT rounds of 64 rows; the 256 columns of each row meet in LDS, each wave then
    // rotates whole 128-column chunks
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
                    E[(32 * wm + 8 * j + 4 * lh + i) * BN + 64 * wn + 32 * nt + l32] = acc[mt][nt][4 * j + i];
            }
        }
        __syncthreads();
        // 64 rows x 2 chunks = 128 row-chunks, 16 per wave
        #pragma unroll 2
        for (int q = 0; q < 16; ++q)
        {
            const int rc = wave * 16 + q;
            const int er = rc >> 1, ch = rc & 1;
            const int row = mb * RB + (RB / 2) * (er >> 5) + 32 * mt + (er & 31);
            const f32x2 v = *(const f32x2*) (E + er * BN + 128 * ch + 2 * lane);
            const int col = nb * BN + 128 * ch + 2 * lane;
            if (nb * BN + 128 * ch >= n) continue;        // half block: chunk past n (uniform per wave)
            const uint32_t svp = has_svh ? *(const uint32_t*) (svh + col) : 0u;
            if (row < M) gemm_store(v.x, v.y, C, c_fp32, has_svh, svp, (size_t) row * n + col, lane);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------
// LDS-DMA form of gemm_kernel for dense launches (256-row tiles, same tiling, decode schedule and
// epilogue).  The A tile and the stage's trellis words go from global memory straight into LDS
// with global_load_lds_dwordx4: no register staging and no ds_write for them.  Each has 4 LDS
// buffers; the DMA for stage s + 3 (A) and s + 4 (trellis) is issued at the start of stage s, and
// each wave waits for its own DMAs of the next stage (vmcnt, counted per wave) before the stage
// barrier.  A lane's 16 bytes land at the wave's LDS block + 16 * lane, so the A swizzle is
// applied by choosing which global chunk each lane loads.
constexpr int DMA_D = 3;                                 // stages of DMA in flight
constexpr int DMA_NB = DMA_D + 1;                         // LDS buffers for A and for trellis

template <int K> struct DmaLds
{
    static constexpr int TWD = tile_words(K);
    static constexpr int A_U32 = 256 * 16;                // A block: 256 rows x 32 fp16
    static constexpr int B_U32 = 2 * BN * 8;              // decoded B block: 2 slices x 256 columns x 16 fp16
    static constexpr int T_U32 = 2 * 16 * TWD;            // 2 slices x 16 tiles, unpadded
    static constexpr int A0 = 0;
    static constexpr int B0 = DMA_NB * A_U32;
    static constexpr int T0 = B0 + 2 * B_U32;
    static constexpr int END = T0 + DMA_NB * T_U32 + 4;    // (+4: a run may read one word past the last tile)
    static constexpr int TOTAL = END > 64 * BN ? END : 64 * BN;
};

// s_waitcnt with vmcnt(n) and lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
#define EXL3_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (((n) >> 4) << 14))

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int K, int CB>
__global__ __launch_bounds__(GT, 1)
void gemm_dma_kernel(const uint16_t* __restrict__ Ain, const uint16_t* __restrict__ trellis, void* __restrict__ C,
                     const uint16_t* __restrict__ svh, int M, int k, int n, int c_fp32, int splits,
                     float* __restrict__ part)
{
    using LD = DmaLds<K>;
    constexpr int RB = 256, MT = 4, TWD = tile_words(K), D = DMA_D, NB = DMA_NB;
    __shared__ __align__(16) uint32_t lds[LD::TOTAL];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = threadIdx.x;
    const int nbn = (n + BN - 1) / BN;
    const int nmb = (M + RB - 1) / RB;
    int nb, mb;
    // k stages st0 .. st0 + NST - 1 of this workgroup (all of k, or range h of the split)
    int st0 = 0, NST = k / 32;
    float* tpart = nullptr;
    if (splits > 1)
    {
        const int tt = blockIdx.x / splits, h = blockIdx.x % splits;
        nb = tt / nmb;
        mb = tt % nmb;
        st0 = h * (k / 32) / splits;
        NST = (h + 1) * (k / 32) / splits - st0;
        tpart = part + (size_t) blockIdx.x * RB * BN;
    }
    else if (nbn % 8 == 0)
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

    // A: wave w's DMAs j = 0, 1 fill the 1 KB blocks q = w + 8 j (rows 16 q .. 16 q + 15); lane L
    // fills slot L, i.e. row 16 q + L / 4 and the chunk that a_off puts in slot L % 4
    const u32x4* a_src[2];
    #pragma unroll
    for (int j = 0; j < 2; ++j)
    {
        const int q = wave + 8 * j, row = 16 * q + (lane >> 2), ch = (lane & 3) ^ ((row >> 2) & 3);
        a_src[j] = (const u32x4*) (Ain + (size_t) min(mb * RB + row, M - 1) * k + 8 * ch);
    }
    // trellis: thread t < 8 TWD copies words 4t .. 4t + 3 of the stage's 2 slices x 16 tiles
    const bool tload = t < 8 * TWD;
    const bool t_wave = 64 * wave < 8 * TWD;              // the wave issues a trellis DMA
    const uint32_t* t_src;
    {
        const int wi = 4 * (tload ? t : 0);
        const int s2 = wi / (16 * TWD), wj = wi - s2 * (16 * TWD);
        const int tile = wj / TWD, wk = wj - tile * TWD;
        const int gtile = min(nb * 16 + tile, n / 16 - 1);   // columns past n: a valid tile, results dropped
        t_src = (const uint32_t*) trellis + ((size_t) s2 * (n / 16) + gtile) * TWD + wk;
    }
    const size_t t_stage = (size_t) 2 * (n / 16) * TWD;

    auto issue_a = [&](int sa) {
        const int c = st0 + min(sa, NST - 1);
        #pragma unroll
        for (int j = 0; j < 2; ++j)
            __builtin_amdgcn_global_load_lds((const void*) (a_src[j] + 4 * c),
                                             (lds_ptr_t) (lds + LD::A0 + (sa % NB) * LD::A_U32 + 256 * (wave + 8 * j)), 16, 0, 0);
    };
    auto issue_t = [&](int st) {
        const int c = st0 + min(st, NST - 1);
        if (tload)
            __builtin_amdgcn_global_load_lds((const void*) (t_src + c * t_stage),
                                             (lds_ptr_t) (lds + LD::T0 + (st % NB) * LD::T_U32 + 256 * wave), 16, 0, 0);
    };

    // ---- decode assignment (as gemm_kernel, unpadded tiles)
    const int dc = t & 255, dh = t >> 8;
    const int dtile = dc >> 4, dcc = dc & 15;
    const int dbase = 32 * (dcc & 7) + 4 * (dcc >> 3) + 2 * dh;
    const int dB0 = tile_end<K>(dbase) - 16;
    const int df = dB0 - 1 >= 0 ? (dB0 - 1) / 32 : -1;
    const int dsh = dB0 - 32 * df;
    const int d_src = LD::T0 + dtile * TWD + df;
    const int d_ring = LD::T0 + dtile * TWD + (df < 0 ? TWD - 1 : df);
    const int d_dst0 = LD::B0 + b_off(0, dc, dh), d_dst1 = LD::B0 + b_off(1, dc, dh);
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, lh = lane >> 5;

    // prologue: T(0), then groups g = 0 .. D - 1 of (A(g), T(g + 1)); B(0) decoded from T(0)
    issue_t(0);
    #pragma unroll
    for (int g = 0; g < D; ++g) { issue_a(g); issue_t(g + 1); }
    if (t_wave) EXL3_VM_LGKM0(3 * D); else EXL3_VM_LGKM0(2 * D);
    __builtin_amdgcn_s_barrier();
    #pragma unroll
    for (int sl = 0; sl < 2; ++sl)
    {
        const uint32_t* T = lds + sl * 16 * TWD;
        *(u32x4*) (lds + (sl ? d_dst1 : d_dst0)) = decode_run<K, CB>(T + d_src, T + d_ring, dsh);
    }
    if (t_wave) EXL3_VM_LGKM0(3 * (D - 1)); else EXL3_VM_LGKM0(2 * (D - 1));
    __builtin_amdgcn_s_barrier();

    acc16 acc[MT][2];
    #pragma unroll
    for (int i = 0; i < MT; ++i) { acc[i][0] = (acc16) { }; acc[i][1] = (acc16) { }; }

    for (int s = 0; s < NST; ++s)
    {
        // stage s + D's A and s + D + 1's trellis: their buffers were last read in stage s - 1
        issue_a(s + D);
        issue_t(s + D + 1);
        const uint32_t* A = lds + LD::A0 + (s % NB) * LD::A_U32;
        const uint32_t* B = lds + LD::B0 + (s & 1) * LD::B_U32;
        const uint32_t* Tn = lds + ((s + 1) % NB) * LD::T_U32;
        uint32_t* Bn = lds + ((s + 1) & 1) * LD::B_U32;
        #pragma unroll
        for (int sl = 0; sl < 2; ++sl)
        {
            h8v bv[2], av[MT];
            #pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                bv[nt] = __builtin_bit_cast(h8v, *(const u32x4*) (B + b_off(sl, 64 * wn + 32 * nt + l32, lh)));
            #pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                av[mt] = __builtin_bit_cast(h8v, *(const u32x4*) (A + a_off((RB / 2) * wm + 32 * mt + l32, 2 * sl + lh)));
            constexpr int NW = run_words<K>();
            const uint32_t* tl = Tn + d_src + sl * 16 * TWD;
            uint32_t rw[NW + 1], nw[NW + 1], r[8], wp[4];
            rw[0] = Tn[d_ring + sl * 16 * TWD];
            #pragma unroll
            for (int i = 1; i <= NW; ++i) rw[i] = tl[i];
#define EXL3_MFMA_STEP(mt, nt) \
            __builtin_amdgcn_sched_barrier(0); \
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bv[nt], acc[mt][nt], 0, 0, 0); \
            __builtin_amdgcn_sched_barrier(0);
            EXL3_MFMA_STEP(0, 0)
            #pragma unroll
            for (int i = 0; i < NW; ++i) nw[i] = __builtin_amdgcn_alignbit(rw[i], rw[i + 1], 32 - dsh);
            nw[NW] = 0u;
            EXL3_MFMA_STEP(0, 1)
            r[0] = cb_raw<CB>(win16<run_rel<K>(0)>(nw));
            r[1] = cb_raw<CB>(win16<run_rel<K>(1)>(nw));
            EXL3_MFMA_STEP(1, 0)
            r[2] = cb_raw<CB>(win16<run_rel<K>(8)>(nw));
            r[3] = cb_raw<CB>(win16<run_rel<K>(9)>(nw));
            EXL3_MFMA_STEP(1, 1)
            wp[0] = weight_pair<CB>(r[0], r[1]);
            wp[1] = weight_pair<CB>(r[2], r[3]);
            EXL3_MFMA_STEP(2, 0)
            r[4] = cb_raw<CB>(win16<run_rel<K>(16)>(nw));
            r[5] = cb_raw<CB>(win16<run_rel<K>(17)>(nw));
            EXL3_MFMA_STEP(2, 1)
            r[6] = cb_raw<CB>(win16<run_rel<K>(24)>(nw));
            r[7] = cb_raw<CB>(win16<run_rel<K>(25)>(nw));
            EXL3_MFMA_STEP(3, 0)
            wp[2] = weight_pair<CB>(r[4], r[5]);
            wp[3] = weight_pair<CB>(r[6], r[7]);
            EXL3_MFMA_STEP(3, 1)
#undef EXL3_MFMA_STEP
            *(u32x4*) (Bn + (sl ? d_dst1 : d_dst0)) = (u32x4) { wp[0], wp[1], wp[2], wp[3] };
        }
        // the next stage's A and trellis (issued D stages ago) have landed, this stage's B stores
        // are done: then the barrier
        if (t_wave) EXL3_VM_LGKM0(3 * (D - 1)); else EXL3_VM_LGKM0(2 * (D - 1));
        __builtin_amdgcn_s_barrier();
    }
    // no DMA may still write LDS when the epilogue reuses it
    EXL3_VM_LGKM0(0);
    __builtin_amdgcn_s_barrier();

    // ---- epilogue (as gemm_kernel)
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
                    E[(32 * wm + 8 * j + 4 * lh + i) * BN + 64 * wn + 32 * nt + l32] = acc[mt][nt][4 * j + i];
            }
        }
        __syncthreads();
        #pragma unroll 2
        for (int q = 0; q < 16; ++q)
        {
            const int rc = wave * 16 + q;
            const int er = rc >> 1, ch = rc & 1;
            const int row = mb * RB + (RB / 2) * (er >> 5) + 32 * mt + (er & 31);
            const f32x2 v = *(const f32x2*) (E + er * BN + 128 * ch + 2 * lane);
            const int col = nb * BN + 128 * ch + 2 * lane;
            if (nb * BN + 128 * ch >= n) continue;
            if (tpart)
            {
                // rows past M are neither stored nor read by the fixup
                if (row < M) *(f32x2*) (tpart + (size_t) (row - mb * RB) * BN + 128 * ch + 2 * lane) = v;
                continue;
            }
            const uint32_t svp = has_svh ? *(const uint32_t*) (svh + col) : 0u;
            if (row < M) gemm_store(v.x, v.y, C, c_fp32, has_svh, svp, (size_t) row * n + col, lane);
        }
        __syncthreads();
    }
}

template <int K, int CB>
int launch_gemm(const GemmArgs& g, hipStream_t s)
{
    const int nmb = (g.m + BM - 1) / BM;
    const int blocks = ((g.n + BN - 1) / BN) * nmb;
    GemmGroupArgs none;
    memset(&none, 0, sizeof(none));
    if (!g.reg_staging && g.splits > 1)
    {
        hipLaunchKernelGGL((gemm_dma_kernel<K, CB>), dim3(blocks * g.splits), dim3(GT), 0, s,
                           g.A_rot, g.trellis, g.C, g.svh, g.m, g.k, g.n, g.c_fp32, g.splits, g.part);
        if (int rc = (int) hipGetLastError()) return rc;
        return exl3k_split_fixup(g.part, g.C, g.svh, g.m, g.n, g.n, g.c_fp32, nmb, blocks, g.splits, s);
    }
    if (!g.reg_staging)
        hipLaunchKernelGGL((gemm_dma_kernel<K, CB>), dim3(blocks), dim3(GT), 0, s,
                           g.A_rot, g.trellis, g.C, g.svh, g.m, g.k, g.n, g.c_fp32, 1, (float*) nullptr);
    else
        hipLaunchKernelGGL((gemm_kernel<K, CB, false, BM>), dim3(blocks), dim3(GT), 0, s,
                           g.A_rot, g.trellis, g.C, g.svh, g.m, g.k, g.n, g.c_fp32, none);
    return (int) hipGetLastError();
}

template <int K, int CB>
int launch_gemm_group(const GemmGroupArgs& g, hipStream_t s)
{
    const long blocks = (long) g.nrt * g.mats * ((g.n + BN - 1) / BN);
    if (blocks <= 0) return 0;
    const dim3 grid((unsigned) blocks), block(GT);
    const uint16_t* nul = nullptr;
    if (g.tile_rows == 64)
        hipLaunchKernelGGL((gemm_kernel<K, CB, true, 64>), grid, block, 0, s, nul, nul, (void*) nullptr, nul, 0, g.k, g.n, 0, g);
    else if (g.tile_rows == 128)
        hipLaunchKernelGGL((gemm_kernel<K, CB, true, 128>), grid, block, 0, s, nul, nul, (void*) nullptr, nul, 0, g.k, g.n, 0, g);
    else
        hipLaunchKernelGGL((gemm_kernel<K, CB, true, 256>), grid, block, 0, s, nul, nul, (void*) nullptr, nul, 0, g.k, g.n, 0, g);
    return (int) hipGetLastError();
}


// ---------------------------------------------------------------------------------------------
// Register-decode grouped GEMM of the token-sorted MoE (moeg_kernel).
//
// The token-sorted MoE's row tiles hold few rows (T * topk / experts: 16 at T = 512, 64 at
// T = 2048), so the weight decode, not the matrix pipe, bounds its GEMMs.  Here every weight is
// decoded once per row tile straight into MFMA operand registers (no LDS round trip and no
// barrier for the weights), and each decoded fragment feeds one v_mfma_f32_16x16x32_f16 per
// 16-row group of the tile.
//
// Work item = (row tile, matrix, 128-column chunk); a workgroup of 4 waves owns the chunk, wave w
// the column tiles 2w, 2w+1.  Per unit of 4 k-tiles (64 k) lane l decodes tile (k-tile l/16,
// column tile 2w + (l%16)/8) at position j = l%8 -- columns j and j+8, all 16 rows -- into 16
// packed fp16 pairs (pair q: rows 2(q>>2) + 8(q&1) + {0,1}, column half (q>>1)&1).  Operand A
// (16 columns x 32 k) for column half c and row half h is lane l's rows 8h..8h+7 of its column,
// pairs {h+2c, 4+h+2c, 8+h+2c, 12+h+2c}, in natural k order; operand B (32 k x 16 rows) is, for
// lane l, row l%16 of the group at k = 64u + 16(l/16) + 8h .. +7: 16 contiguous bytes in LDS.
//
// MUL1 weights enter as h = 1024 + byte sum, the decode's exact fp16 value, and the codebook's
// affine map is applied to the sums: y = kinv sum(h x) + bias sum(x) (codebook.cuh:78-84), with
// sum(x) from the 128-chunk sums the staging kernels write beside the rows (psum, added in a
// fixed order).  MCG weights are the reference's fp16 lo + hi (one rounding).
//
// The rows are staged one unit at a time into LDS, double-buffered through registers, one
// barrier per unit.  Items run persistently and XCD-aware: the workgroups of XCD x (blockIdx % 8)
// take the (row tile, matrix) entries e with e % 8 == x, so all chunks of an entry share one L2.
// Tuning, measured on MI355X (256 experts 4096 -> 2048 -> 4096, T = 512 / 2048): a trellis ring of
// 2 units, X loaded 2 units ahead, one unit per barrier, B operands read before the decode, and
// 4 waves per SIMD for 32- and 64-row tiles (3 for 96, 2 for 128); barrier count, prefetch depth and occupancy moved
// the time by under 3 %: the decode VALU and the MFMAs, which issue mostly serially on a SIMD,
// bound the kernel.
constexpr int MG_PF = 2, MG_XD = 2, MG_XU = 1;
constexpr int MG_THREADS = 256;
constexpr int MG_OW = 68;        // u32 per epilogue row: 128 fp16 + 16 bytes

template <int R> struct MgLds
{
    static constexpr int RT = 16 * R;                   // rows per tile
    static constexpr int XBUF = RT * 32 * MG_XU;        // staged rows of one phase
    static constexpr int OUT = RT * MG_OW;
    static constexpr int MAIN = 2 * XBUF > OUT ? 2 * XBUF : OUT;
    static constexpr int TOTAL = MAIN;
};


template <int K, int CB, int R>
__global__ __launch_bounds__(MG_THREADS)
__attribute__((amdgpu_waves_per_eu(R <= 4 ? 4 : (R <= 6 ? 3 : 2), R <= 4 ? 4 : (R <= 6 ? 3 : 2))))
void moeg_kernel(const GemmGroupArgs g)
{
    using LD = MgLds<R>;
    static_assert(R >= 2, "a tile stages at least 32 rows (two 16-byte loads per 8 threads)");
    constexpr int TWD = tile_words(K), KB = kbits(K), XC = R / 2;
    constexpr int PF = MG_PF, XD = MG_XD;                 // trellis ring depth, X prefetch distance (phases)
    static_assert(PF % (XD * MG_XU) == 0, "the X ring slot must be a compile-time function of the unroll index");
    __shared__ __align__(16) uint32_t lds[LD::TOTAL];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = threadIdx.x;
    const int k = g.k, n = g.n;
    const int nch = n / 128, units = k / 64, tiles_n = n / 16;   // units is even (k % 128 == 0)
    const uint32_t a3 = sconst(89226354u), b3 = vconst(64248484u);
    const int cnt0 = *to_global(g.count[0]);
    const int cnt1 = g.mats > 1 ? *to_global(g.count[1]) : 0;
    const int ents = (cnt0 > cnt1 ? cnt0 : cnt1) * g.mats;
    const int xcd = blockIdx.x & 7, lb = blockIdx.x >> 3, nlb = gridDim.x >> 3;
    const int per_xcd = ents > xcd ? (ents - xcd + 7) / 8 : 0;
    uint16_t* ot = (uint16_t*) lds;                       // epilogue [RT][2 MG_OW] fp16

    for (int it = lb; it < per_xcd * nch; it += nlb)
    {
        const int ent = xcd + 8 * (it / nch), chunk = it % nch;
        const int mat = ent % g.mats, li = ent / g.mats;
        if (li >= (mat ? cnt1 : cnt0)) continue;
        const int tid = *to_global((mat ? g.list[1] : g.list[0]) + li);
        const int e = *to_global(g.rt + 3 * tid), row0 = *to_global(g.rt + 3 * tid + 1);
        const int M = *to_global(g.rt + 3 * tid + 2);
        const uint16_t* A = (mat ? g.A[1] : g.A[0]) + (size_t) row0 * k;
        uint16_t* C = (mat ? g.C[1] : g.C[0]) + (size_t) row0 * n + chunk * 128;
        const uint32_t* trellis = (const uint32_t*) *to_global((mat ? g.tab[1] : g.tab[0]) + e);
        const int rg = (M + 15) >> 4;                     // live 16-row groups (1..R)

        const int jt = lane & 7;
        const uint32_t* tile0 = trellis + ((size_t) (lane >> 4) * tiles_n + chunk * 8 + 2 * wave + ((lane >> 3) & 1)) * TWD;
        const size_t ustride = (size_t) 4 * tiles_n * TWD;
        const int prev_off = jt == 0 ? 8 * KB - 1 : -1;
        uint32_t ring[PF][KB + 1];
        #pragma unroll
        for (int d = 0; d < PF; ++d) load_tile_lane<K>(tile0 + (size_t) min(d, units - 1) * ustride, jt, prev_off, ring[d]);

        // X: one phase of XU units (64 XU k per row) at a time into LDS, double-buffered; phase
        // p + XD is loaded while phase p computes, phase p + 1 stored after it (one barrier per
        // phase)
        constexpr int XU = MG_XU, XWD = 32 * XU;          // row stride (u32)
        static_assert(XU == 1, "the X swizzle below covers one unit (8 chunks of 16 bytes) per row");
        // 16-byte chunk c of staged row r sits at chunk c ^ s(r % 16), s(q) = (q ^ (q >> 3)) & 7: no
        // LDS bank conflicts for the B-operand reads (16 rows x 4 chunks per instruction) nor for
        // the row stores (measured on MI355X; a 16-byte row padding left 4 conflict cycles per
        // read).  Depending on r % 16 only, the offsets of the other 16-row groups are constants.
        auto xoff = [](int r, int c) { const int q = r & 15; return r * XWD + 4 * (c ^ ((q ^ (q >> 3)) & 7)); };
        const int xb0 = xoff(lane & 15, 2 * (lane >> 4));     // h = 0; h = 1 is the next chunk: ^ 4
        constexpr int PCH = 8 * XU;                       // 16-byte chunks per row and phase
        constexpr int XCP = R * XU / 2;                   // chunk loads per thread and phase
        const int phases = units / XU;
        u32x4 xr[XD][XCP];
        auto xload = [&](u32x4* x, int ph) {
            #pragma unroll
            for (int i = 0; i < XCP; ++i)
            {
                const int c = t + MG_THREADS * i, row = c / PCH;
                x[i] = *to_global((const u32x4*) (A + (size_t) min(row, M - 1) * k + min(ph, phases - 1) * 64 * XU + (c % PCH) * 8));
            }
        };
        auto xstore = [&](const u32x4* x, int buf) {
            #pragma unroll
            for (int i = 0; i < XCP; ++i)
            {
                const int c = t + MG_THREADS * i;
                *(u32x4*) (lds + buf * (LD::RT * XWD) + xoff(c / PCH, c % PCH)) = x[i];
            }
        };
        #pragma unroll
        for (int d = 0; d < XD; ++d) xload(xr[d], d);
        xstore(xr[0], 0);
        xload(xr[0], XD);                                 // slot p % XD holds phase p
        f32x4 acc[2][R];
        #pragma unroll
        for (int r = 0; r < R; ++r) { acc[0][r] = (f32x4) { }; acc[1][r] = (f32x4) { }; }
        __syncthreads();

        for (int u0 = 0; u0 < units; u0 += PF)
        {
            #pragma unroll
            for (int d = 0; d < PF; ++d)
            {
                const int u = u0 + d;                     // (PF divides units: no tail)
                const int ph = u / XU;
                // this unit's B operands first: their LDS latency hides behind the decode
                const uint32_t* xb = lds + (ph & 1) * (LD::RT * XWD);
                h8v bx[2][R];
                #pragma unroll
                for (int h = 0; h < 2; ++h)
                {
                    #pragma unroll
                    for (int r = 0; r < R; ++r)
                        bx[h][r] = __builtin_bit_cast(h8v, *(const u32x4*) (xb + 16 * r * XWD + (xb0 ^ (4 * h))));
                }
                uint32_t wv[KB + 1], pk[16];
                #pragma unroll
                for (int w = 0; w <= KB; ++w) wv[w] = ring[d][w];
                if constexpr (CB == 2) mul1_pairs<K>(wv, pk);
                else
                {
                    uint32_t raw[32];
                    raw32<K, CB>(wv, raw, a3, b3);
                    #pragma unroll
                    for (int q = 0; q < 16; ++q) pk[q] = weight_pair<CB>(raw[2 * q], raw[2 * q + 1]);
                }
                load_tile_lane<K>(tile0 + (size_t) min(u + PF, units - 1) * ustride, jt, prev_off, ring[d]);
                #pragma unroll
                for (int h = 0; h < 2; ++h)
                {
                    const u32x4 a0 = { pk[h], pk[4 + h], pk[8 + h], pk[12 + h] };
                    const u32x4 a1 = { pk[2 + h], pk[6 + h], pk[10 + h], pk[14 + h] };
                    #pragma unroll
                    for (int r = 0; r < R; ++r)
                    {
                        if (r >= rg) break;
                        const h8v b = bx[h][r];
                        acc[0][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, a0), b, acc[0][r], 0, 0, 0);
                        acc[1][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, a1), b, acc[1][r], 0, 0, 0);
                    }
                }
                if ((d + 1) % XU == 0)
                {
                    const int slot = ((d + 1) / XU) % XD;     // phase ph + 1's slot
                    xstore(xr[slot], (ph + 1) & 1);           // (past the last phase: an unread buffer)
                    xload(xr[slot], ph + 1 + XD);             // (clamped past the end)
                    __syncthreads();
                }
            }
        }

        // epilogue: D[i][nn] of acc[c][r] (lane l: i = 4 (l/16) + e, nn = l%16) is column
        // 32 w + 16 (i/8) + i%8 + 8 c, row 16 r + nn; rows meet in LDS for coalesced stores
        const int kc = k / 128;
        const float* ps = (mat ? g.psum[1] : g.psum[0]) + (size_t) row0 * kc;
        // MUL1 row sums sum(x) from the 128-chunk sums: lane quarter q4 = lane / 16 adds chunks
        // q4, q4 + 4, ... of its row, all groups' loads issued together, then the quarters
        // combine in a fixed order (q4 0 + 1, 2 + 3, then the pairs)
        float sxr[R];
        if (CB == 2)
        {
            constexpr int PQ = 8;                             // loads in flight per lane and group
            #pragma unroll
            for (int r = 0; r < R; ++r) sxr[r] = 0.0f;
            const int q4 = lane >> 4;
            for (int c0 = 0; c0 < kc; c0 += 4 * PQ)
            {
                float v[R][PQ];
                #pragma unroll
                for (int r = 0; r < R; ++r)
                {
                    const float* pr = ps + (size_t) min(16 * r + (lane & 15), M - 1) * kc;
                    #pragma unroll
                    for (int i = 0; i < PQ; ++i)
                    {
                        const int c = c0 + 4 * i + q4;
                        v[r][i] = *to_global(pr + min(c, kc - 1));
                    }
                }
                #pragma unroll
                for (int r = 0; r < R; ++r)
                {
                    #pragma unroll
                    for (int i = 0; i < PQ; ++i)
                        if (c0 + 4 * i + q4 < kc) sxr[r] += v[r][i];
                }
            }
            #pragma unroll
            for (int r = 0; r < R; ++r)
            {
                float t = sxr[r] + __shfl_xor(sxr[r], 16, 64);
                t += __shfl_xor(t, 32, 64);
                sxr[r] = t * (float) as_h(0xc931);
            }
        }
        #pragma unroll
        for (int r = 0; r < R; ++r)
        {
            if (r >= rg) break;
            const int row = 16 * r + (lane & 15);
            const float sx = CB == 2 ? sxr[r] : 0.0f;
            #pragma unroll
            for (int c = 0; c < 2; ++c)
            {
                #pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const int i = 4 * (lane >> 4) + q;
                    const int col = 32 * wave + 16 * (i >> 3) + (i & 7) + 8 * c;
                    float v = acc[c][r][q];
                    if (CB == 2) v = v * (float) as_h(0x1eee) + sx;
                    ot[row * (2 * MG_OW) + col] = h_bits((f16) v);
                }
            }
        }
        __syncthreads();
        for (int q = t; q < M * 16; q += MG_THREADS)
        {
            const int row = q >> 4, part = q & 15;
            *to_global_w((u32x4*) (C + (size_t) row * n + part * 8)) = *(const u32x4*) (ot + row * (2 * MG_OW) + part * 8);
        }
        __syncthreads();
    }
}

template <int K, int CB>
int launch_moeg(const GemmGroupArgs& g, hipStream_t s)
{
    const long items = (long) g.nrt * g.mats * (g.n / 128);
    long grid = g.grid_wgs > 0 && g.grid_wgs < items ? g.grid_wgs : items;
    grid = (grid + 7) / 8 * 8;
    if (items <= 0) return 0;
    const dim3 gr((unsigned) grid), block(MG_THREADS);
    if (g.tile_rows <= 32) hipLaunchKernelGGL((moeg_kernel<K, CB, 2>), gr, block, 0, s, g);
    else if (g.tile_rows <= 64) hipLaunchKernelGGL((moeg_kernel<K, CB, 4>), gr, block, 0, s, g);
    else if (g.tile_rows <= 96) hipLaunchKernelGGL((moeg_kernel<K, CB, 6>), gr, block, 0, s, g);
    else hipLaunchKernelGGL((moeg_kernel<K, CB, 8>), gr, block, 0, s, g);
    return (int) hipGetLastError();
}
}  // namespace

#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)

int EXL3_CAT(exl3k_gemm_k, EXL3_INST_K)(const GemmArgs& g, int cb, hipStream_t s)
{
#if EXL3_INST_K >= 16
    return cb == 2 ? launch_gemm<EXL3_INST_K, 2>(g, s) : -1;       // half rates: mul1 only
#endif
    switch (cb)
    {
        case 0: return launch_gemm<EXL3_INST_K, 0>(g, s);
        case 1: return launch_gemm<EXL3_INST_K, 1>(g, s);
        case 2: return launch_gemm<EXL3_INST_K, 2>(g, s);
    }
    return -1;
}

int EXL3_CAT(exl3k_moeg_k, EXL3_INST_K)(const GemmGroupArgs& g, int cb, hipStream_t s)
{
#if EXL3_INST_K >= 16
    return cb == 2 ? launch_moeg<EXL3_INST_K, 2>(g, s) : -1;
#endif
    switch (cb)
    {
        case 1: return launch_moeg<EXL3_INST_K, 1>(g, s);
        case 2: return launch_moeg<EXL3_INST_K, 2>(g, s);
    }
    return -1;
}

int EXL3_CAT(exl3k_gemm_group_k, EXL3_INST_K)(const GemmGroupArgs& g, int cb, hipStream_t s)
{
    // the token-sorted MoE takes the mcg and mul1 codebooks only (exl3_moe.cu:242)
#if EXL3_INST_K >= 16
    return cb == 2 ? launch_gemm_group<EXL3_INST_K, 2>(g, s) : -1;
#endif
    switch (cb)
    {
        case 1: return launch_gemm_group<EXL3_INST_K, 1>(g, s);
        case 2: return launch_gemm_group<EXL3_INST_K, 2>(g, s);
    }
    return -1;
}
