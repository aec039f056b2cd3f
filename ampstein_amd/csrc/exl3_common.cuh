// Shared device code for the EXL3 kernels (gfx950 / CDNA4, wave64).
//
// Data layout (identical to the reference's, quant/reconstruct.cu:31-34, moe_mul1.cpp:1508):
//   trellis  uint16 (k/16, n/16, 16K [+8 for K+0.5]) row-major; tile (kt, nt) covers W rows
//            kt*16..+15 (input dim) and columns nt*16..+15 (output dim).
//   A tile's 256 positions form one MSB-first bit ring over its uint32 words
//   (word i = u16[2i] | u16[2i+1] << 16).  Position t's 16-bit state is the window ending
//   (t+1)*K bits into the ring (quant/exl3_dq.cuh:15-31).
//
// Lane mapping used by every kernel here: the 8 tiles of one 128-column chunk of one k-slice
// are 8*8K uint32 words = 64 lanes x K words.  Lane l holds words [j*K, j*K+K) of tile l/8
// (j = l%8) and decodes the 32 positions whose windows END inside those words: t = 32j..32j+31.
// With the reference's tile permutation (cpu/moe_mul1.cpp:124-139) those positions are exactly
// columns j and j+8 of the tile, all 16 rows.  The only word a lane needs from outside is the
// last word of lane (j-1)%8 of the same tile (the window start of t = 32j).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exl3_kernels.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));

#define EXL3_HAD_RSCALE 0.088388347648f     // 1/sqrt(128) as the reference writes it

// Global-address-space view of a pointer.  Pointers read from memory (pointer tables) or
// carried in by-value structs are generic to the compiler, whose loads then become flat loads
// that also count in lgkmcnt (every scalar-load wait then waits for them too).
#define EXL3_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const EXL3_GLOBAL T* to_global(const T* p) { return (const EXL3_GLOBAL T*) p; }
template <typename T>
__device__ __forceinline__ EXL3_GLOBAL T* to_global_w(T* p) { return (EXL3_GLOBAL T*) p; }

namespace exl3 {

__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ f16 as_h(uint16_t v) { return __builtin_bit_cast(f16, v); }
__device__ __forceinline__ uint16_t h_bits(f16 v) { return __builtin_bit_cast(uint16_t, v); }

// Opaque register constants: keeps the compiler from rematerialising them inside loops.
__device__ __forceinline__ uint32_t sconst(uint32_t v) { asm volatile("" : "+s"(v)); return v; }
__device__ __forceinline__ uint32_t vconst(uint32_t v) { asm volatile("" : "+v"(v)); return v; }

// Codebook multipliers split into 16-bit halves: x = s * (A1 << 16 | A0) + B  (mod 2^32).
// 3INST: codebook.cuh:61-62; MCG: :69; MUL1: :78.
template <int CB> struct cb_consts;
template <> struct cb_consts<0> { static constexpr uint32_t A0 = 0x7C72u, A1 = 0x0551u, B = 64248484u; };
template <> struct cb_consts<1> { static constexpr uint32_t A0 = 0x1FEDu, A1 = 0xCBACu, B = 0u; };
template <> struct cb_consts<2> { static constexpr uint32_t A0 = 0xD12Du, A1 = 0x83DCu, B = 0u; };

// Registers holding the decode constants, created once per kernel.
struct DecodeRegs
{
    uint32_t a0, a1;      // SGPR: multiplier halves
    uint32_t b;           // VGPR: additive constant
    uint32_t mask;        // SGPR: 0x8fff8fff
    uint32_t xorv;        // VGPR: 0x3b603b60
    uint32_t acc;         // VGPR: 0x6400     (mul1 byte-sum bias -> fp16 1024.0)
    uint32_t kinv2;       // SGPR: fp16x2 0x1eee (mul1 scale)
    uint32_t bias2;       // VGPR: fp16x2 0xc931 (mul1 bias)
    uint32_t sel;         // SGPR: v_perm selector packing two low halves
};

template <int CB>
__device__ __forceinline__ DecodeRegs make_decode_regs()
{
    DecodeRegs r;
    r.a0 = sconst(cb_consts<CB>::A0);
    r.a1 = sconst(cb_consts<CB>::A1);
    r.b = vconst(cb_consts<CB>::B);
    r.mask = sconst(0x8fff8fffu);
    r.xorv = vconst(0x3b603b60u);
    r.acc = vconst(0x6400u);
    r.kinv2 = sconst(0x1eee1eeeu);
    r.bias2 = vconst(0xc931c931u);
    r.sel = sconst(0x05040100u);
    return r;
}

// ---------------------------------------------------------------------------------------------
// Codebook decode of four windows into two packed fp16 pairs (w0, w1), (w2, w3).  Window w's
// 16-bit state is half H<w> of register s<w>.
//   x = state * A + B (mod 2^32): v_mad_u32_u16 gives state * A0 + B; v_mad_u16 then adds
//   state * A1 into the high half (mod 2^16).
//   3INST / MCG: (x & 0x8fff8fff) ^ 0x3b603b60 (lop3 0x6a of codebook.cuh:47 = v_bitop3 0x6a),
//   then the fp16 sum of its halves, rounded once (written as fma(lo, 1.0, hi)).
//   MUL1: byte sum + 0x6400 read as fp16 (1024 + sum), then one fp16 fma with 0x1eee, 0xc931.
//   The byte sum is v_sad_u8(x, 0, 0x6400) (sum of |byte - 0|, the vabsdiff4 form noted at
//   codebook.cuh:31-34): a plain VALU op, unlike v_dot4 whose result needs 3 wait states.
// One asm block per group: the four chains are interleaved so that no instruction reads a
// register written by the instruction just before it (gfx950 needs one wait state after a
// write to the high half only), and the compiler adds a single wait after the block.
// ---------------------------------------------------------------------------------------------
#define EXL3_S(x) #x
#define EXL3_XS(x) EXL3_S(x)

#define EXL3_MUL_BLOCK(H0, H1, H2, H3, BREG)                                                   \
    "v_mad_u32_u16 %[t0], %[s0], %[a0], " BREG " op_sel:[" EXL3_XS(H0) ",0,0,0]\n\t"           \
    "v_mad_u32_u16 %[t1], %[s1], %[a0], " BREG " op_sel:[" EXL3_XS(H1) ",0,0,0]\n\t"           \
    "v_mad_u32_u16 %[t2], %[s2], %[a0], " BREG " op_sel:[" EXL3_XS(H2) ",0,0,0]\n\t"           \
    "v_mad_u32_u16 %[t3], %[s3], %[a0], " BREG " op_sel:[" EXL3_XS(H3) ",0,0,0]\n\t"           \
    "v_mad_u16 %[t0], %[s0], %[a1], %[t0] op_sel:[" EXL3_XS(H0) ",0,1,1]\n\t"                  \
    "v_mad_u16 %[t1], %[s1], %[a1], %[t1] op_sel:[" EXL3_XS(H1) ",0,1,1]\n\t"                  \
    "v_mad_u16 %[t2], %[s2], %[a1], %[t2] op_sel:[" EXL3_XS(H2) ",0,1,1]\n\t"                  \
    "v_mad_u16 %[t3], %[s3], %[a1], %[t3] op_sel:[" EXL3_XS(H3) ",0,1,1]\n\t"

#define EXL3_QUAD_SPEC(H0, H1, H2, H3)                                                         \
template <> struct Quad<0, H0, H1, H2, H3> {                                                   \
    static __device__ __forceinline__ void run(uint32_t s0, uint32_t s1, uint32_t s2,         \
        uint32_t s3, uint32_t& o0, uint32_t& o1, const DecodeRegs& r)                          \
    {                                                                                          \
        uint32_t t0, t1, t2, t3;                                                               \
        asm(EXL3_MUL_BLOCK(H0, H1, H2, H3, "%[b]")                                             \
            "v_bitop3_b32 %[t0], %[t0], %[m], %[x] bitop3:0x6a\n\t"                            \
            "v_bitop3_b32 %[t1], %[t1], %[m], %[x] bitop3:0x6a\n\t"                            \
            "v_bitop3_b32 %[t2], %[t2], %[m], %[x] bitop3:0x6a\n\t"                            \
            "v_bitop3_b32 %[t3], %[t3], %[m], %[x] bitop3:0x6a\n\t"                            \
            "v_fma_f16 %[o0], %[t0], 1.0, %[t0] op_sel:[0,0,1,0]\n\t"                          \
            "v_fma_f16 %[o1], %[t2], 1.0, %[t2] op_sel:[0,0,1,0]\n\t"                          \
            "v_fma_f16 %[o0], %[t1], 1.0, %[t1] op_sel:[0,0,1,1]\n\t"                          \
            "v_fma_f16 %[o1], %[t3], 1.0, %[t3] op_sel:[0,0,1,1]"                              \
            : [t0] "=&v"(t0), [t1] "=&v"(t1), [t2] "=&v"(t2), [t3] "=&v"(t3),                  \
              [o0] "=&v"(o0), [o1] "=&v"(o1)                                                   \
            : [s0] "v"(s0), [s1] "v"(s1), [s2] "v"(s2), [s3] "v"(s3), [a0] "s"(r.a0),          \
              [a1] "s"(r.a1), [b] "v"(r.b), [m] "s"(r.mask), [x] "v"(r.xorv));                 \
    }                                                                                          \
};                                                                                             \
template <> struct Quad<2, H0, H1, H2, H3> {                                                   \
    static __device__ __forceinline__ void run(uint32_t s0, uint32_t s1, uint32_t s2,         \
        uint32_t s3, uint32_t& o0, uint32_t& o1, const DecodeRegs& r)                          \
    {                                                                                          \
        uint32_t t0, t1, t2, t3;                                                               \
        asm(EXL3_MUL_BLOCK(H0, H1, H2, H3, "0")                                                \
            "v_sad_u8 %[t0], %[t0], 0, %[acc]\n\t"                                  \
            "v_sad_u8 %[t1], %[t1], 0, %[acc]\n\t"                                  \
            "v_sad_u8 %[t2], %[t2], 0, %[acc]\n\t"                                  \
            "v_sad_u8 %[t3], %[t3], 0, %[acc]\n\t"                                  \
            "v_perm_b32 %[o0], %[t1], %[t0], %[sel]\n\t"                                       \
            "v_perm_b32 %[o1], %[t3], %[t2], %[sel]\n\t"                                       \
            "v_pk_fma_f16 %[o0], %[o0], %[kinv], %[bias]\n\t"                                  \
            "v_pk_fma_f16 %[o1], %[o1], %[kinv], %[bias]"                                      \
            : [t0] "=&v"(t0), [t1] "=&v"(t1), [t2] "=&v"(t2), [t3] "=&v"(t3),                  \
              [o0] "=&v"(o0), [o1] "=&v"(o1)                                                   \
            : [s0] "v"(s0), [s1] "v"(s1), [s2] "v"(s2), [s3] "v"(s3), [a0] "s"(r.a0),          \
              [a1] "s"(r.a1), [acc] "v"(r.acc), [sel] "s"(r.sel),          \
              [kinv] "s"(r.kinv2), [bias] "v"(r.bias2));                                       \
    }                                                                                          \
};

// CB 0 (3INST) and 1 (MCG) share the code; the constants differ.
template <int CB, int H0, int H1, int H2, int H3> struct Quad
{
    static __device__ __forceinline__ void run(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t s3,
                                               uint32_t& o0, uint32_t& o1, const DecodeRegs& r)
    {
        Quad<0, H0, H1, H2, H3>::run(s0, s1, s2, s3, o0, o1, r);
    }
};

EXL3_QUAD_SPEC(0, 0, 0, 0) EXL3_QUAD_SPEC(0, 0, 0, 1) EXL3_QUAD_SPEC(0, 0, 1, 0) EXL3_QUAD_SPEC(0, 0, 1, 1)
EXL3_QUAD_SPEC(0, 1, 0, 0) EXL3_QUAD_SPEC(0, 1, 0, 1) EXL3_QUAD_SPEC(0, 1, 1, 0) EXL3_QUAD_SPEC(0, 1, 1, 1)
EXL3_QUAD_SPEC(1, 0, 0, 0) EXL3_QUAD_SPEC(1, 0, 0, 1) EXL3_QUAD_SPEC(1, 0, 1, 0) EXL3_QUAD_SPEC(1, 0, 1, 1)
EXL3_QUAD_SPEC(1, 1, 0, 0) EXL3_QUAD_SPEC(1, 1, 0, 1) EXL3_QUAD_SPEC(1, 1, 1, 0) EXL3_QUAD_SPEC(1, 1, 1, 1)

// ---------------------------------------------------------------------------------------------
// Window extraction for integer K.  wv[0] is the previous lane's last word, wv[1..K] this
// lane's K words.  Window i (0..31) ends at local bit (i+1)*K + 32 of that 32(K+1)-bit string,
// so its 16 bits lie inside words hi-1, hi (hi = (end-1)/32).  The state is the low or high
// half of alignbit(wv[hi-1], wv[hi], s & 15) with s the right shift of the window's end;
// windows whose shifts differ by 16 share one alignbit, and s & 15 == 0 costs nothing.
// ---------------------------------------------------------------------------------------------
// Rate codes: K = 1..8 is the integer bitrate; K = 16 + b (b = 1..3) is b + 1/2 (mul1 only,
// bits_k.cuh:8-27).  A 16x16 tile holds tile_words(K) u32.
__host__ __device__ constexpr int kbits(int K) { return K & 15; }
__host__ __device__ constexpr bool khalf(int K) { return K >= 16; }
__host__ __device__ constexpr int tile_words(int K) { return 8 * kbits(K) + (khalf(K) ? 4 : 0); }

template <int K, bool H = khalf(K)> struct Win
{
    static constexpr int e(int i) { return (i + 1) * K + 32; }
    static constexpr int hi(int i) { return (e(i) - 1) / 32; }
    static constexpr int s(int i) { return (hi(i) + 1) * 32 - e(i); }
    static constexpr int sb(int i) { return s(i) & 15; }
    static constexpr int h(int i) { return s(i) >> 4; }
};

// Half-integer rates (K = 16 + b): a tile holds 8b + 4 words, and lane j of the tile (j = lane
// % 8) decodes positions 32j..32j+31, whose windows end at tile bits S_j + r(i),
// S_j = j (32b + 16), r(i) = (i/2)(2b + 1) + (i odd ? 2b + 1 : b) (exl3_dq.cuh:254-285).  The
// lane's frame wv[0..b] holds bits [S_j - 16, S_j + 32b + 16) (load_frame_half), so window i
// ends at frame bit r(i) + 16; windows inside wv[0] (e <= 32) need no left word.
template <int K> struct Win<K, true>
{
    static constexpr int B = K & 15;
    static constexpr int e(int i) { return (i >> 1) * (2 * B + 1) + ((i & 1) ? 2 * B + 1 : B) + 16; }
    static constexpr int hi(int i) { return (e(i) - 1) / 32; }
    static constexpr int s(int i) { return (hi(i) + 1) * 32 - e(i); }
    static constexpr int sb(int i) { return s(i) & 15; }
    static constexpr int h(int i) { return s(i) >> 4; }
};

template <int K, int I>
__device__ __forceinline__ uint32_t win_reg(const uint32_t* wv)
{
    constexpr int hi = Win<K>::hi(I), sb = Win<K>::sb(I);
    if constexpr (sb == 0) return wv[hi];
    else return __builtin_amdgcn_alignbit(wv[hi > 0 ? hi - 1 : 0], wv[hi], sb);
}

// Frame of a half-rate lane (see Win<K, true>): the b + 2 words from word jb + j/2 - 1 of the
// tile (lane 0: the ring wraps to the tile's last word), shifted left by 16 bits for even j so
// that the frame starts at word 0, bit 0 (MSB-first).
template <int K>
__device__ __forceinline__ void load_frame_half(const uint32_t* __restrict__ tile, int j, uint32_t* wv)
{
    constexpr int B = kbits(K);
    const int b = j * B + (j >> 1) - 1;
    uint32_t raw[B + 2];
    raw[0] = __builtin_nontemporal_load(to_global(tile) + (b < 0 ? tile_words(K) - 1 : b));
    #pragma unroll
    for (int i = 1; i < B + 2; ++i) raw[i] = __builtin_nontemporal_load(to_global(tile) + b + i);
    const uint32_t sh = (j & 1) ? 0u : 16u;
    #pragma unroll
    for (int i = 0; i <= B; ++i) wv[i] = __builtin_amdgcn_alignbit(raw[i], raw[i + 1], sh);
}

// Decode the lane's 32 windows into 16 packed pairs: out[q] = (window 2q, window 2q+1).
// Pair q holds column (j + 8 * ((q >> 1) & 1)), rows 2(q >> 2) + 8 (q & 1) and +1.
template <int K, int CB, int G>
__device__ __forceinline__ void decode_g(const uint32_t* wv, uint32_t* out, const DecodeRegs& r)
{
    constexpr int i = 4 * G;
    Quad<CB, Win<K>::h(i), Win<K>::h(i + 1), Win<K>::h(i + 2), Win<K>::h(i + 3)>::run(
        win_reg<K, i>(wv), win_reg<K, i + 1>(wv), win_reg<K, i + 2>(wv), win_reg<K, i + 3>(wv),
        out[2 * G], out[2 * G + 1], r);
}

template <int K, int CB>
__device__ __forceinline__ void decode_lane32(const uint32_t* wv, uint32_t* out, const DecodeRegs& r)
{
    decode_g<K, CB, 0>(wv, out, r); decode_g<K, CB, 1>(wv, out, r);
    decode_g<K, CB, 2>(wv, out, r); decode_g<K, CB, 3>(wv, out, r);
    decode_g<K, CB, 4>(wv, out, r); decode_g<K, CB, 5>(wv, out, r);
    decode_g<K, CB, 6>(wv, out, r); decode_g<K, CB, 7>(wv, out, r);
}

// Column (0..15 within the tile) and first row of pair q decoded by tile lane j.
__device__ __forceinline__ constexpr int pair_col(int j, int q) { return j + 8 * ((q >> 1) & 1); }
__device__ __forceinline__ constexpr int pair_row(int q) { return 2 * (q >> 2) + 8 * (q & 1); }

// Previous word of the tile ring: lane (j-1)%8 of the same 8-lane tile group.
__device__ __forceinline__ uint32_t ring_prev(uint32_t last_word, int lane)
{
    int src = (lane & ~7) | ((lane - 1) & 7);
    return __builtin_amdgcn_ds_bpermute(src << 2, last_word);
}

// ---------------------------------------------------------------------------------------------
// Hadamard-128 helpers (natural / Sylvester order; butterfly order of hadamard_inner.cuh:17-41).
// A 128-vector over a wave: lane l holds elements 2l, 2l+1.  In-lane stage (width 1), then
// xor-1..32 lane stages (widths 2..64): lower index a+b, upper a-b, fp32.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float xor_shfl(float v, int mask, int lane)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, v)));
}

// silu(x) = x / (1 + exp(-x)) in fp32 (amp_silu_mul_kernel, src/torch/amp_kernels.cu:235-251).
// SiLU in fp32 from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each),
// a few ops instead of the IEEE expf and division sequences; the fp16 result it feeds stays
// within one ulp of the exact value (the reference's own SiLU is an fp16 h2exp / h2rcp form)
__device__ __forceinline__ float silu_f32(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Value of lane (lane ^ M) without LDS: DPP quad permutes (M = 1, 2), two bank-masked row
// shifts (M = 4), a row rotate (M = 8), gfx950 permlane swaps (M = 16, 32).
template <int M>
__device__ __forceinline__ float xor_partner(float v, int lane)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    uint32_t p;
    // (full row and bank masks with a permutation inside each row: every lane is written, so
    // v_mov_b32_dpp needs no old value, and none is materialised)
    if constexpr (M == 1) p = __builtin_amdgcn_mov_dpp(u, 0xB1, 0xf, 0xf, false);               // quad_perm [1,0,3,2]
    else if constexpr (M == 2) p = __builtin_amdgcn_mov_dpp(u, 0x4E, 0xf, 0xf, false);          // quad_perm [2,3,0,1]
    else if constexpr (M == 4)
    {
        p = __builtin_amdgcn_update_dpp(0u, u, 0x104, 0xf, 0x5, false);   // row_shl:4 into banks 0, 2
        p = __builtin_amdgcn_update_dpp(p, u, 0x114, 0xf, 0xa, false);    // row_shr:4 into banks 1, 3
    }
    else if constexpr (M == 8) p = __builtin_amdgcn_mov_dpp(u, 0x128, 0xf, 0xf, false);         // row_ror:8
    else if constexpr (M == 16)
    {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        p = (lane & 16) ? r[0] : r[1];
    }
    else
    {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        p = (lane & 32) ? r[0] : r[1];
    }
    return __builtin_bit_cast(float, p);
}

// The same partner through the LDS crossbar (ds_swizzle_b32, bit mode: lane ^ M within each
// 32-lane half; no LDS memory is touched), for M <= 16.  One instruction on the LDS pipe instead
// of one or two VALU ops: for kernels whose VALU, not latency, is the limit.
template <int M>
__device__ __forceinline__ float xor_partner_sw(float v)
{
    static_assert(M >= 1 && M <= 16, "ds_swizzle xor reaches within 32 lanes");
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1f | (M << 10)));
}

// One butterfly stage: lower lane a + b, upper lane a - b (a = lower element), one rounding each
// (fma with a +-1 factor is exactly the sum or the difference).
template <int M>
__device__ __forceinline__ void fwht_stage(float& v0, float& v1, int lane)
{
    const float p0 = xor_partner<M>(v0, lane), p1 = xor_partner<M>(v1, lane);
    const float sg = (lane & M) ? -1.0f : 1.0f;
    v0 = __builtin_fmaf(sg, v0, p0);
    v1 = __builtin_fmaf(sg, v1, p1);
}

__device__ __forceinline__ void fwht128_wave(float& v0, float& v1, int lane)
{
    float s = v0 + v1, d = v0 - v1;
    v0 = s; v1 = d;
    fwht_stage<1>(v0, v1, lane);
    fwht_stage<2>(v0, v1, lane);
    fwht_stage<4>(v0, v1, lane);
    fwht_stage<8>(v0, v1, lane);
    fwht_stage<16>(v0, v1, lane);
    fwht_stage<32>(v0, v1, lane);
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

// The decode step's residual norm split over 128-column chunks (rms_norm_res,
// amp_kernels.cu:279-365, computed by its neighbours): the producer of a row adds its residual
// chunk by chunk and keeps each chunk's sum of squares; the consumer of the row forms the scale
// from those sums and normalises its input on load.  Lane l of a wave owns columns 2 l, 2 l + 1 of
// a chunk.  Each function is the only statement of its step, so every kernel that uses it
// produces the same bits.

// Sum over the wave in every lane: xor butterfly 1, 2, .., 32 on DPP / permlane (no LDS; every
// lane active).  One fixed order, so every caller forms the same bits.
__device__ __forceinline__ float xor_sum64(float v, int lane)
{
    v += xor_partner<1>(v, lane);
    v += xor_partner<2>(v, lane);
    v += xor_partner<4>(v, lane);
    v += xor_partner<8>(v, lane);
    v += xor_partner<16>(v, lane);
    v += xor_partner<32>(v, lane);
    return v;
}

// y = fp16(h + c) for the lane's pair, h's pair hv already loaded from h + idx (y is stored
// back there); returns the chunk's fp32 sum of y^2 in every lane (explicit fma per pair, then
// xor_sum64).
__device__ __forceinline__ float res_pair_sq(uint32_t hv, uint32_t cpair, uint16_t* h, size_t idx, int lane)
{
    const f16x2 a = as_h2(hv), b = as_h2(cpair);
    const f16x2 y = { (f16) ((float) a.x + (float) b.x), (f16) ((float) a.y + (float) b.y) };
    *to_global_w((uint32_t*) (h + idx)) = as_u32(y);
    return xor_sum64(__builtin_fmaf((float) y.x, (float) y.x, (float) y.y * (float) y.y), lane);
}

// The row's scale 1 / sqrt(mean(y^2) + eps) from its nchunks chunk sums (nchunks <= 64 *
// SQ_SCALE_MAX_PER_LANE, exl3_kernels.h), in two steps so that a kernel can issue the loads early
// and reduce later: lane l loads chunks l, l + 64, ...; sq_scale adds them in that order, then
// xor_sum64.  Uniform across the wave.
__device__ __forceinline__ void sq_load(const float* sq, int nchunks, int lane, float (&v)[SQ_SCALE_MAX_PER_LANE])
{
    #pragma unroll
    for (int i = 0; i < SQ_SCALE_MAX_PER_LANE; ++i)
        v[i] = lane + 64 * i < nchunks ? *to_global(sq + lane + 64 * i) : 0.0f;
}

__device__ __forceinline__ float sq_scale(const float (&v)[SQ_SCALE_MAX_PER_LANE], int dim, float eps, int lane)
{
    float t = v[0];
    #pragma unroll
    for (int i = 1; i < SQ_SCALE_MAX_PER_LANE; ++i) t += v[i];
    t = xor_sum64(t, lane);
    return 1.0f / sqrtf(t / (float) dim + eps);
}

// The normalised pair fp16(fp16(y * scale) * w).
__device__ __forceinline__ uint32_t norm_pair(uint32_t yv, uint32_t wv, float scale)
{
    const f16x2 y = as_h2(yv);
    return as_u32((f16x2) { (f16) ((float) y.x * scale), (f16) ((float) y.y * scale) } * as_h2(wv));
}

}  // namespace exl3
