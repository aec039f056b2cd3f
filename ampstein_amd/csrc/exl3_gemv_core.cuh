// GEMV building blocks shared by the decode GEMV (exl3_gemv.hip) and the MoE expert GEMV
// (exl3_moe.hip): trellis word loads, window extraction at compile-time offsets, codebook words
// for the v_dot2 against (x, x) pairs.  See exl3_gemv.hip for the lane mapping.
#pragma once

#include "exl3_common.cuh"

namespace exl3 {

// Weight-stream loads: nontemporal (the packed weights are read once per launch)
#define EXL3_WLOAD(ptr) __builtin_nontemporal_load(ptr)

// Load this lane's K words of a slice into w[1..K] and the word before them (the last word of
// the previous lane of the same tile, cyclically: the window start of the lane's first
// position) into w[0], all from global memory: no cross-lane traffic in the loop.
template <int K>
__device__ __forceinline__ void load_slot(const uint32_t* __restrict__ p, int prev_off, uint32_t* w);

template <int K>
__device__ __forceinline__ void load_words(const uint32_t* __restrict__ p, uint32_t* w)
{
    if constexpr (K % 4 == 0)
    {
        #pragma unroll
        for (int i = 0; i < K / 4; ++i)
        {
            u32x4 v = EXL3_WLOAD(to_global((const u32x4*) p) + i);
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    }
    else if constexpr (K % 2 == 0)
    {
        #pragma unroll
        for (int i = 0; i < K / 2; ++i)
        {
            u32x2 v = EXL3_WLOAD(to_global((const u32x2*) p) + i);
            w[2 * i] = v.x; w[2 * i + 1] = v.y;
        }
    }
    else
    {
        #pragma unroll
        for (int i = 0; i < K; ++i) w[i] = EXL3_WLOAD(to_global(p) + i);
    }
}

template <int K>
__device__ __forceinline__ void load_slot(const uint32_t* __restrict__ p, int prev_off, uint32_t* w)
{
    load_words<K>(p, w + 1);
    w[0] = EXL3_WLOAD(to_global(p) + prev_off);
}

// Slot load for any rate code.  Integer K: load_slot, p = the lane's first word (chunk base +
// lane_word_off).  Half rates: p = the 8-tile chunk's first word, the lane's frame of K + 1
// words (exl3_common.cuh load_frame_half); prev_off is unused.
template <int K>
__device__ __forceinline__ constexpr int lane_word_off(int lane) { return khalf(K) ? 0 : lane * K; }

template <int K>
__device__ __forceinline__ void load_slot_k(const uint32_t* __restrict__ p, int prev_off, int lane, uint32_t* w)
{
    if constexpr (khalf(K)) load_frame_half<K>(p + (lane >> 3) * tile_words(K), lane & 7, w);
    else load_slot<K>(p, prev_off, w);
}

// Load lane j's frame of one tile (tile = the tile's first word): integer K, words jK..jK+K-1
// and the ring predecessor (prev_off, relative to word jK); half rates, load_frame_half.
template <int K>
__device__ __forceinline__ void load_tile_lane(const uint32_t* __restrict__ tile, int j, int prev_off, uint32_t* w)
{
    if constexpr (khalf(K)) load_frame_half<K>(tile, j, w);
    else load_slot<K>(tile + j * K, prev_off, w);
}

// Clean 16-bit state of window I (exl3_common.cuh: Win): one bfe, from word hi when the window
// sits inside it, else from the half-word-shifted word alignbit(wv[hi-1], wv[hi], 16) (one per
// word, shared by the windows that straddle that word boundary).
template <int K, int I>
__device__ __forceinline__ uint32_t state16(const uint32_t* wv)
{
    constexpr int hi = Win<K>::hi(I), s = Win<K>::s(I);
    if constexpr (s + 16 <= 32) return __builtin_amdgcn_ubfe(wv[hi], s, 16);
    else return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(wv[hi - 1], wv[hi], 16), s - 16, 16);
}

// Codebook word consumed by v_dot2 against (x, x): 3INST/MCG masked halves, MUL1 (h, 0).
// (3INST goes through mad8_3inst below.)
template <int CB>
__device__ __forceinline__ uint32_t raw_weight(uint32_t s)
{
    if constexpr (CB == 0)
        return ((s * 89226354u + 64248484u) & 0x8fff8fffu) ^ 0x3b603b60u;   // codebook.cuh:61-63
    else if constexpr (CB == 1)
        return ((s * 0xCBAC1FEDu) & 0x8fff8fffu) ^ 0x3b603b60u;             // codebook.cuh:69-72
    else
        return __builtin_amdgcn_sad_u8(s * 0x83DCD12Du, 0u, 0x6400u);       // codebook.cuh:78-84
}

// 3INST for eight clean states: s * 89226354 + 64248484 as one v_mad_u64_u32 each (its low
// word; ~full rate on gfx950, where mul + add would be two ops), then the mask / xor.
__device__ __forceinline__ void mad8_3inst(uint32_t* st, uint32_t a, uint32_t b)
{
    uint64_t r0, r1, r2, r3, r4, r5, r6, r7;
    asm("v_mad_u64_u32 %0, vcc, %8, %16, %17\n\t"
        "v_mad_u64_u32 %1, vcc, %9, %16, %17\n\t"
        "v_mad_u64_u32 %2, vcc, %10, %16, %17\n\t"
        "v_mad_u64_u32 %3, vcc, %11, %16, %17\n\t"
        "v_mad_u64_u32 %4, vcc, %12, %16, %17\n\t"
        "v_mad_u64_u32 %5, vcc, %13, %16, %17\n\t"
        "v_mad_u64_u32 %6, vcc, %14, %16, %17\n\t"
        "v_mad_u64_u32 %7, vcc, %15, %16, %17"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4), "=&v"(r5), "=&v"(r6), "=&v"(r7)
        : "v"(st[0]), "v"(st[1]), "v"(st[2]), "v"(st[3]), "v"(st[4]), "v"(st[5]), "v"(st[6]), "v"(st[7]),
          "s"(a), "v"((uint64_t) b)
        : "vcc");
    st[0] = (uint32_t) r0; st[1] = (uint32_t) r1; st[2] = (uint32_t) r2; st[3] = (uint32_t) r3;
    st[4] = (uint32_t) r4; st[5] = (uint32_t) r5; st[6] = (uint32_t) r6; st[7] = (uint32_t) r7;
    #pragma unroll
    for (int i = 0; i < 8; ++i) st[i] = (st[i] & 0x8fff8fffu) ^ 0x3b603b60u;
}

template <int K, int CB, int I0>
__device__ __forceinline__ void raw8(const uint32_t* wv, uint32_t* raw, const uint32_t a3, const uint32_t b3)
{
    uint32_t st[8] = { state16<K, I0>(wv), state16<K, I0 + 1>(wv), state16<K, I0 + 2>(wv), state16<K, I0 + 3>(wv),
                       state16<K, I0 + 4>(wv), state16<K, I0 + 5>(wv), state16<K, I0 + 6>(wv), state16<K, I0 + 7>(wv) };
    if constexpr (CB == 0)
    {
        mad8_3inst(st, a3, b3);
        #pragma unroll
        for (int i = 0; i < 8; ++i) raw[I0 + i] = st[i];
    }
    else
    {
        #pragma unroll
        for (int i = 0; i < 8; ++i) raw[I0 + i] = raw_weight<CB>(st[i]);
    }
}

// MUL1 weights of windows 2q, 2q + 1 packed into one word: low half 0x6400 + byte sum of
// window 2q's product, high half that of window 2q + 1 (v_sad_u8 then v_sad_hi_u8, which adds
// its byte sum shifted left by 16): the fp16 pair (1024 + s_2q, 1024 + s_2q+1).
template <int K, int Q>
__device__ __forceinline__ uint32_t mul1_pair(const uint32_t* wv)
{
    const uint32_t p0 = state16<K, 2 * Q>(wv) * 0x83DCD12Du, p1 = state16<K, 2 * Q + 1>(wv) * 0x83DCD12Du;
    return __builtin_amdgcn_sad_hi_u8(p1, 0u, __builtin_amdgcn_sad_u8(p0, 0u, 0x64006400u));
}

template <int K>
__device__ __forceinline__ void mul1_pairs(const uint32_t* wv, uint32_t* pk)
{
    pk[0] = mul1_pair<K, 0>(wv);   pk[1] = mul1_pair<K, 1>(wv);   pk[2] = mul1_pair<K, 2>(wv);
    pk[3] = mul1_pair<K, 3>(wv);   pk[4] = mul1_pair<K, 4>(wv);   pk[5] = mul1_pair<K, 5>(wv);
    pk[6] = mul1_pair<K, 6>(wv);   pk[7] = mul1_pair<K, 7>(wv);   pk[8] = mul1_pair<K, 8>(wv);
    pk[9] = mul1_pair<K, 9>(wv);   pk[10] = mul1_pair<K, 10>(wv); pk[11] = mul1_pair<K, 11>(wv);
    pk[12] = mul1_pair<K, 12>(wv); pk[13] = mul1_pair<K, 13>(wv); pk[14] = mul1_pair<K, 14>(wv);
    pk[15] = mul1_pair<K, 15>(wv);
}

template <int K, int CB>
__device__ __forceinline__ void raw32(const uint32_t* wv, uint32_t* raw, const uint32_t a3, const uint32_t b3)
{
    raw8<K, CB, 0>(wv, raw, a3, b3);
    raw8<K, CB, 8>(wv, raw, a3, b3);
    raw8<K, CB, 16>(wv, raw, a3, b3);
    raw8<K, CB, 24>(wv, raw, a3, b3);
}

template <int K, int CB, int I>
__device__ __forceinline__ uint32_t raw_at(const uint32_t* wv) { return raw_weight<CB>(state16<K, I>(wv)); }


}  // namespace exl3
